// qsampler: decode-step token sampler for MI355X (gfx950).
//
// Replaces BatchSampler.forward (src/compute/sampler.py:25-41) behind the
// ModelRunner._sample_gpu call site (src/compute/model_runner.py:77-93) and the
// greedy argmax sites (src/compute/model_runner.py:85,353).  The arithmetic
// contract is stated in include/qsampler.h; ids are exact integers.
//
// One kernel does the sampling: grid (G chunks, B rows), 256 threads (4 waves
// of 64).  Each workgroup streams one chunk of a row into registers once
// (16-byte loads), applies the history penalties from an LDS table and then
// takes the path of its row:
//   greedy row   local argmax, one 64-bit atomic max per workgroup; the last
//                workgroup to arrive publishes the id.
//   top-k row    (0 < k <= QS_TOPK_FAST_MAX) each workgroup emits the tokens
//                above a threshold taken from its per-thread maxima; the last
//                workgroup merges them in LDS and resolves top-k, top-p and the
//                draw exactly.
//   mass row     (top-k off) the workgroups of the row cooperate through row
//                barriers: row maximum; fixed-point mass histograms over
//                y = q*log2(e) (two levels) that bracket the top-p cut; an
//                exact resolution of the bracketed tokens; the draw from
//                per-chunk kept masses.  The chunk data stay in registers.
//   fallback     a single workgroup resolves the row exactly from global
//                memory (rows with large k, candidate overflow, a missed
//                bracket).  Slow, and rare on real logits.
// Cross-workgroup data are written with device-coherent stores or atomics and
// read with device-coherent loads; ordering comes from s_waitcnt before a
// relaxed counter update.  No release/acquire fences: on this part they write
// back or invalidate the whole L2 of an XCD per workgroup.
// The finishing workgroup of every row returns the row's counters to zero, so
// the workspace needs no memset between calls.  k_probs writes the optional
// post-filter probabilities (verification output).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "qsampler.h"

typedef unsigned __int128 u128;
typedef unsigned long long u64;
typedef uint32_t u32;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kWindow = 40;
constexpr double kYClamp = 1073741824.0;  // 2^30
constexpr double kLog2e = 1.4426950408889634074;
constexpr int kTopkFast = QS_TOPK_FAST_MAX;
constexpr int kBlockCand = 256;     // candidate slots per (row, workgroup) in the workspace
constexpr int kMergeCap = 4096;     // candidates the finishing workgroup merges in LDS
constexpr int kBins = 256;          // mass histogram bins per level
constexpr int kBracketCap = 2048;   // bracketed tokens resolved exactly in LDS
constexpr int kMaxChunks = 256;     // chunks per row (G)
constexpr int kMaxHistory = QS_MAX_HISTORY;
constexpr u32 kSpinLimit = 1u << 21;

enum : u32 { kStFallback = 1u, kStTimeout = 2u, kStOverflow = 4u };

// Per-row control block.  The first 64 bytes are counters that every call
// leaves at zero; the rest holds the last call's result for k_probs.
struct __attribute__((aligned(256))) RowCtl {
  u64 pack;        // greedy: max of (gkey << 32 | ~id)
  u32 arrive;      // workgroups done
  u32 bar;         // row barrier counter
  u32 cand_n;      // top-k candidates appended
  u32 tau;         // max per-workgroup candidate threshold
  u32 kmax;        // mass rows: max key(q)
  u32 nkmin;       // mass rows: ~min key(q)
  u32 status;      // kSt* flags
  u32 brk_n;       // bracketed tokens appended
  u32 brk_kmax;    // max key among bracketed tokens
  u32 brk_nkmin;   // ~min key among bracketed tokens
  u32 probs_arrive;
  u32 probs_kept;
  u32 nout;        // top-k rows: max key among tokens no workgroup emitted
  u32 pad0;
  long long chosen;
  u64 w_lo, w_hi;  // kept mass W
  int n_max;       // row scale N
  u32 kappa_p, id_p;  // kept iff key > kappa_p || (key == kappa_p && id <= id_p)
  u32 greedy;
  u32 path;        // how the row was resolved: 0 greedy, 1 top-k, 2 mass, 3 single workgroup
  u32 pad1[37];
};
static_assert(sizeof(RowCtl) == 256, "row control block is 256 bytes");
constexpr int kCtlZeroWords = 16;

// Per-(row, workgroup) published values of a mass row.
struct __attribute__((aligned(64))) Slot {
  u64 s_lo, s_hi;  // exact mass of the chunk (plain draw) or the mass above the bracket
  u32 nb;          // bracketed tokens in the chunk
  u32 pad[11];
};
static_assert(sizeof(Slot) == 64, "slot is 64 bytes");

struct Args {
  const void* logits;
  long long row_stride;
  int B, V, H, G, CH, seg_cap, Hpad;
  u32 flags;
  const float* temperature;
  const float* top_p;
  const int* top_k;
  const float* rep;
  const float* pres;
  const float* freq;
  const int* hist;
  const float* uniforms;
  long long* out_ids;
  float* out_probs;
  int* out_kept;
  RowCtl* ctl;
  u64* cand;   // [B, G, kBlockCand]
  u64* mhist;  // [B, 2, kBins]
  u64* brk;    // [B, kBracketCap]
  Slot* slots; // [B, G]
  u64* trace;  // per-workgroup phase timestamps (trace builds only)
};

#ifdef QS_TRACE
#define QS_TR(i)                                                                          \
  do {                                                                                    \
    if (a.trace && threadIdx.x == 0)                                                      \
      a.trace[((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 16 + (i)] = wall_clock64(); \
  } while (0)
#else
#define QS_TR(i) \
  do {           \
  } while (0)
#endif

// ---------------------------------------------------------------- memory model

// Wait until this thread's outstanding memory operations have completed.
__device__ __forceinline__ void wait_mem() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
template <typename T>
__device__ __forceinline__ T ldc(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void stc(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T addc(T* p, T v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T maxc(T* p, T v) {
  return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void orc(u32* p, u32 v) {
  __hip_atomic_fetch_or(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- contract

// Sampling key: orderable bits, NaN lowest, -0 == +0.
__device__ __forceinline__ u32 skey(float z) {
  if (z != z) return 0u;
  if (z == 0.0f) z = 0.0f;
  const u32 u = __float_as_uint(z);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// Greedy key: NaN highest.
__device__ __forceinline__ u32 gkey(float z) {
  if (z != z) return 0xffffffffu;
  return skey(z);
}
__device__ __forceinline__ float f_of_key(u32 k) {
  const u32 u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}
__device__ __forceinline__ double y_of(float q) {
  if (q != q) return -kYClamp;
  double y = (double)q * kLog2e;
  y = (y >= -kYClamp) ? y : -kYClamp;
  y = (y > kYClamp) ? kYClamp : y;
  return y;
}
__device__ __forceinline__ float exp2_poly(float f) {
  float p = 0x1.c54640p-13f;
  p = __builtin_fmaf(p, f, 0x1.46d326p-10f);
  p = __builtin_fmaf(p, f, 0x1.3d0c40p-7f);
  p = __builtin_fmaf(p, f, 0x1.c688f0p-5f);
  p = __builtin_fmaf(p, f, 0x1.ebfd5ap-3f);
  p = __builtin_fmaf(p, f, 0x1.62e42cp-1f);
  p = __builtin_fmaf(p, f, 1.0f);
  return p;
}
__device__ __forceinline__ u32 mant24(float p) {
  if (!(p >= 1.0f)) p = 1.0f;
  if (p >= 2.0f) p = __uint_as_float(0x3fffffffu);
  return 0x800000u | (__float_as_uint(p) & 0x7fffffu);
}
__device__ __forceinline__ int octave_of(float q) { return (int)floor(y_of(q)); }
// u64 weight of exp(q) relative to the row scale N (0 below the window).
__device__ __forceinline__ u64 weight_y(double y, int N) {
  const double fl = floor(y);
  const int n = (int)fl;
  if (n < N - kWindow) return 0ull;
  return (u64)mant24(exp2_poly((float)(y - fl))) << (n - N + kWindow);
}
__device__ __forceinline__ u64 weight_of(float q, int N) { return weight_y(y_of(q), N); }
// floor(x * f) for f in [0, 1] given as fp32, x < 2^104.
__device__ __forceinline__ u128 mul_frac(u128 x, float f) {
  if (!(f > 0.0f)) return 0;
  const u32 b = __float_as_uint(f);
  const u32 e = (b >> 23) & 0xffu;
  u32 m = b & 0x7fffffu;
  int shift;
  if (e == 0) {
    shift = 149;
  } else {
    m |= 0x800000u;
    shift = 150 - (int)e;
  }
  if (shift >= 128) return 0;
  return (x * (u128)m) >> shift;
}
// floor(d / w) for a quotient below 2^53.
__device__ __forceinline__ u64 div_small(u128 d, u64 w) {
  u64 q = (u64)((double)(u64)(d >> 64) * 0x1p64 / (double)w + (double)(u64)d / (double)w);
  while (q > 0 && (u128)q * w > d) --q;
  while ((u128)(q + 1) * w <= d) ++q;
  return q;
}
// Same limb order as the oracle, so the fp64 value is bit-identical.
__device__ __forceinline__ double u128_to_double(u128 x) {
  const u64 lo = (u64)x, hi = (u64)(x >> 64);
  double d = (double)(u32)(hi >> 32) * 0x1p96;
  d = d + (double)(u32)hi * 0x1p64;
  d = d + (double)(u32)(lo >> 32) * 0x1p32;
  d = d + (double)(u32)lo;
  return d;
}
__device__ __forceinline__ float apply_penalty(float z, u32 c, float rep, float pres, float freq) {
  z = (z > 0.0f) ? (z / rep) : (z * rep);
  const float fc = freq * (float)c;
  z = z - fc;
  z = z - pres;
  return z;
}
__device__ __forceinline__ float bf16_to_f32(u32 h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ u128 mk128(u64 lo, u64 hi) { return ((u128)hi << 64) | lo; }
__device__ __forceinline__ int pow2_ceil(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

template <int DT>
__device__ __forceinline__ float load_logit(const Args& a, int row, int i) {
  if (DT == QS_DTYPE_F32) return ((const float*)a.logits)[(size_t)row * a.row_stride + i];
  return bf16_to_f32(((const uint16_t*)a.logits)[(size_t)row * a.row_stride + i]);
}

enum RowKind : int { kGreedy = 0, kTopK = 1, kMass = 2, kSingle = 3 };

struct RowParams {
  float T, tp, rep, pres, freq, u;
  int k;
  bool greedy, topk_on, topp_on, pen_on;
  int kind;
};

__device__ __forceinline__ RowParams row_params(const Args& a, int row) {
  RowParams p;
  p.T = a.temperature ? a.temperature[row] : 0.0f;
  p.greedy = (a.flags & QS_FLAG_ALL_GREEDY) || (p.T <= 1e-5f);
  p.k = a.top_k ? a.top_k[row] : 0;
  p.topk_on = !p.greedy && p.k > 0 && p.k < a.V;
  p.tp = ((a.flags & QS_FLAG_USE_TOP_P) && a.top_p) ? a.top_p[row] : 1.0f;
  p.topp_on = !p.greedy && (p.tp < 1.0f);
  p.rep = a.rep ? a.rep[row] : 1.0f;
  p.pres = a.pres ? a.pres[row] : 0.0f;
  p.freq = a.freq ? a.freq[row] : 0.0f;
  p.pen_on = a.hist != nullptr && a.H > 0 && (p.rep != 1.0f || p.pres != 0.0f || p.freq != 0.0f);
  p.u = a.uniforms ? a.uniforms[row] : 0.0f;
  if (!(p.u >= 0.0f)) p.u = 0.0f;
  if (p.u >= 1.0f) p.u = __uint_as_float(0x3f7fffffu);
  p.kind = p.greedy ? kGreedy : (p.topk_on ? (p.k <= kTopkFast ? kTopK : kSingle) : kMass);
  return p;
}

// ---------------------------------------------------------------- block utils

struct Scratch {   // static LDS
  u64 w[3 * kWaves + 4];  // find_bin, lds_select results
  u32 u[8];
  u32 v[kWaves][8];       // per-wave partials of the block collectives
  int i[8];               // find_bin
  u32 r[8];               // results and counters of the callers
};

// ---- wave64 collectives on DPP (row_shr, quad_perm, mirrors, row_bcast):
// the lane exchange is folded into the ALU op, no LDS round trip.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ u32 dpp_mov(u32 v) {
  return (u32)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xF, false);
}
__device__ __forceinline__ u32 lane_id() { return threadIdx.x & 63; }
// Inclusive scan (add) over the wave's lanes.
__device__ __forceinline__ u32 wave_incl_scan(u32 v) {
  v += dpp_mov<0x111, 0xF>(v);  // row_shr:1
  v += dpp_mov<0x112, 0xF>(v);  // row_shr:2
  v += dpp_mov<0x114, 0xF>(v);  // row_shr:4
  v += dpp_mov<0x118, 0xF>(v);  // row_shr:8
  v += dpp_mov<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_mov<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}
// Maximum over the wave, returned to every lane.
__device__ __forceinline__ u32 wave_max(u32 v) {
  v = max(v, dpp_mov<0xB1, 0xF>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_mov<0x4E, 0xF>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_mov<0x141, 0xF>(v));  // row_half_mirror
  v = max(v, dpp_mov<0x140, 0xF>(v));  // row_mirror
  v = max(v, dpp_mov<0x142, 0xA>(v));  // row_bcast:15
  v = max(v, dpp_mov<0x143, 0xC>(v));  // row_bcast:31
  return (u32)__builtin_amdgcn_readlane((int)v, 63);
}
template <int CTRL, int ROWMASK>
__device__ __forceinline__ void max64_step(u32& hi, u32& lo) {
  const u32 th = dpp_mov<CTRL, ROWMASK>(hi), tl = dpp_mov<CTRL, ROWMASK>(lo);
  const bool t = th > hi || (th == hi && tl > lo);
  hi = t ? th : hi;
  lo = t ? tl : lo;
}
__device__ __forceinline__ u64 wave_max64(u64 v) {
  u32 hi = (u32)(v >> 32), lo = (u32)v;
  max64_step<0xB1, 0xF>(hi, lo);
  max64_step<0x4E, 0xF>(hi, lo);
  max64_step<0x141, 0xF>(hi, lo);
  max64_step<0x140, 0xF>(hi, lo);
  max64_step<0x142, 0xA>(hi, lo);
  max64_step<0x143, 0xC>(hi, lo);
  return ((u64)(u32)__builtin_amdgcn_readlane((int)hi, 63) << 32) | (u32)__builtin_amdgcn_readlane((int)lo, 63);
}

// ---- block collectives: wave result, one LDS exchange, two barriers
__device__ __forceinline__ u64 block_max_u64(u64 v, Scratch& s) {
  v = wave_max64(v);
  const int wv = threadIdx.x >> 6;
  if (lane_id() == 0) {
    s.v[wv][0] = (u32)(v >> 32);
    s.v[wv][1] = (u32)v;
  }
  __syncthreads();
  u64 r = 0;
  for (int i = 0; i < kWaves; ++i) {
    const u64 x = ((u64)s.v[i][0] << 32) | s.v[i][1];
    r = x > r ? x : r;
  }
  __syncthreads();
  return r;
}
__device__ __forceinline__ u32 block_max_u32(u32 v, Scratch& s) {
  v = wave_max(v);
  const int wv = threadIdx.x >> 6;
  if (lane_id() == 0) s.v[wv][0] = v;
  __syncthreads();
  u32 r = 0;
  for (int i = 0; i < kWaves; ++i) r = s.v[i][0] > r ? s.v[i][0] : r;
  __syncthreads();
  return r;
}

// Appends for the lanes with `pred` set: one LDS atomic per wave, each such
// lane gets a distinct slot (counter value before its own increment).
__device__ __forceinline__ u32 wave_append(bool pred, u32* counter) {
  const u64 mask = __ballot(pred);
  if (mask == 0ull) return 0u;
  const int leader = __ffsll((long long)mask) - 1;
  const u32 rank = __builtin_amdgcn_mbcnt_hi((u32)(mask >> 32), __builtin_amdgcn_mbcnt_lo((u32)mask, 0u));
  u32 base = 0u;
  if ((int)lane_id() == leader) base = atomicAdd(counter, (u32)__popcll(mask));
  base = (u32)__builtin_amdgcn_readlane((int)base, leader);
  return base + rank;
}

// Exclusive scan of u32 in thread order; total in *total.
__device__ __forceinline__ u32 block_scan_u32(u32 v, Scratch& s, u32* total) {
  const int wv = threadIdx.x >> 6;
  const u32 inc = wave_incl_scan(v);
  if (lane_id() == 63) s.v[wv][0] = inc;
  __syncthreads();
  u32 base = 0, tot = 0;
  for (int i = 0; i < kWaves; ++i) {
    const u32 x = s.v[i][0];
    base += (i < wv) ? x : 0u;
    tot += x;
  }
  __syncthreads();
  *total = tot;
  return base + inc - v;
}

struct Acc {  // (count, 128-bit mass)
  u64 lo, hi;
  u32 c;
};
__device__ __forceinline__ Acc acc_add(Acc a, Acc b) {
  Acc r;
  r.lo = a.lo + b.lo;
  r.hi = a.hi + b.hi + (r.lo < a.lo ? 1ull : 0ull);
  r.c = a.c + b.c;
  return r;
}
__device__ __forceinline__ u128 acc_mass(const Acc& a) { return mk128(a.lo, a.hi); }
__device__ __forceinline__ Acc acc_of(u128 m, u32 c) {
  Acc r;
  r.lo = (u64)m;
  r.hi = (u64)(m >> 64);
  r.c = c;
  return r;
}

// Exclusive scan of (count, mass) in thread order; total in *total.  Masses
// below 2^88 are scanned as four 22-bit limbs (a limb sum over 256 threads
// stays below 2^30), then recombined exactly.
__device__ __forceinline__ Acc block_scan_acc(Acc v, Scratch& s, Acc* total) {
  constexpr u32 kL = (1u << 22) - 1u;
  const int wv = threadIdx.x >> 6;
  const u128 m = acc_mass(v);
  u32 x[5];
  x[0] = v.c;
  x[1] = (u32)m & kL;
  x[2] = (u32)(m >> 22) & kL;
  x[3] = (u32)(m >> 44) & kL;
  x[4] = (u32)(m >> 66) & kL;
  u32 inc[5];
#pragma unroll
  for (int j = 0; j < 5; ++j) inc[j] = wave_incl_scan(x[j]);
  if (lane_id() == 63) {
#pragma unroll
    for (int j = 0; j < 5; ++j) s.v[wv][j] = inc[j];
  }
  __syncthreads();
  u32 base[5] = {0, 0, 0, 0, 0}, tot[5] = {0, 0, 0, 0, 0};
  for (int i = 0; i < kWaves; ++i) {
#pragma unroll
    for (int j = 0; j < 5; ++j) {
      const u32 t = s.v[i][j];
      base[j] += (i < wv) ? t : 0u;
      tot[j] += t;
    }
  }
  __syncthreads();
  const u128 tm = (u128)tot[1] + ((u128)tot[2] << 22) + ((u128)tot[3] << 44) + ((u128)tot[4] << 66);
  *total = acc_of(tm, tot[0]);
  const u128 em = (u128)(base[1] + inc[1] - x[1]) + ((u128)(base[2] + inc[2] - x[2]) << 22) +
                  ((u128)(base[3] + inc[3] - x[3]) << 44) + ((u128)(base[4] + inc[4] - x[4]) << 66);
  return acc_of(em, base[0] + inc[0] - x[0]);
}
__device__ __forceinline__ Acc block_sum_acc(Acc v, Scratch& s) {
  Acc t;
  (void)block_scan_acc(v, s, &t);
  return t;
}

// Sum over threads of a u128 (returned to all threads).
__device__ __forceinline__ u128 block_sum128(u128 v, Scratch& s) { return acc_mass(block_sum_acc(acc_of(v, 0u), s)); }

// Bitonic sort of n (power of two) ints in LDS, ascending.
__device__ __forceinline__ void bitonic_i32(int* s, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += kThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const int x = s[i], y = s[ixj];
          if (((i & k) == 0) ? (x > y) : (x < y)) {
            s[i] = y;
            s[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- LDS radix select

struct SelLds {  // one 8-bit digit level of a radix select
  u32 cnt[256];
  u64 mlo[256];  // sums of the low 32 bits of the weights
  u64 mhi[256];  // sums of the high 32 bits
};

struct SelOut {
  u32 val;      // the selected 32-bit order value
  Acc before;   // members strictly before it in the scan order (count, mass)
  Acc at;       // members equal to it
  bool ok;      // false if the target is not below the members' total
};

// Over members i in [0, n) (in(i)), ordered by the 32-bit value val(i)
// descending (DESC) or ascending, find the value at which the running count
// (or, BY_MASS, the running sum of weight(i)) first exceeds `target`.
// 8-bit digits from the highest bit where members differ; all threads call it.
template <bool BY_MASS, bool DESC, typename ValF, typename InF, typename WF>
__device__ __forceinline__ SelOut lds_select(int n, ValF val, InF in, WF weight, u128 target, SelLds& L,
                                             Scratch& sc) {
  static_assert(kThreads == 256, "one digit bin per thread");
  const int tid = threadIdx.x;
  // highest bit where the members' values differ
  u32 first = 0u, any = 0u, diff = 0u;
  {
    u32 mx = 0u, mn = 0xffffffffu;
    for (int i = tid; i < n; i += kThreads) {
      if (in(i)) {
        const u32 v = val(i);
        mx = v > mx ? v : mx;
        mn = v < mn ? v : mn;
        any = 1u;
      }
    }
    mx = block_max_u32(mx, sc);
    mn = ~block_max_u32(~mn, sc);
    any = block_max_u32(any, sc);
    first = mn;
    diff = mx ^ mn;
  }
  SelOut out;
  out.before = Acc{0, 0, 0};
  out.at = Acc{0, 0, 0};
  out.val = first;
  out.ok = any != 0u;
  if (!any) return out;
  int top = 31;
  while (top > 0 && !((diff >> top) & 1u)) --top;
  // the bits above `top` are common to all members: they start the prefix
  u32 prefix = (top == 31) ? 0u : (first & ~((2u << top) - 1u));
  u32 mask = (top == 31) ? 0u : ~((2u << top) - 1u);
  int hi = top;
  for (;;) {
    const int lo = hi >= 7 ? hi - 7 : 0;
    const int width = hi - lo + 1;
    const u32 dmask = (1u << width) - 1u;
    L.cnt[tid] = 0u;
    if (BY_MASS) {
      L.mlo[tid] = 0ull;
      L.mhi[tid] = 0ull;
    }
    __syncthreads();
    for (int i = tid; i < n; i += kThreads) {
      if (!in(i)) continue;
      const u32 v = val(i);
      if ((v & mask) != prefix) continue;
      const u32 d = (v >> lo) & dmask;
      atomicAdd(&L.cnt[d], 1u);
      if (BY_MASS) {
        const u64 w = weight(i);
        if (w) {
          atomicAdd(&L.mlo[d], w & 0xffffffffull);
          atomicAdd(&L.mhi[d], w >> 32);
        }
      }
    }
    __syncthreads();
    // scan the bins in order: thread t takes bin (DESC ? 255 - t : t)
    const int b = DESC ? 255 - tid : tid;
    const bool live = b <= (int)dmask;
    Acc mine = {0, 0, 0};
    if (live) {
      mine.c = L.cnt[b];
      if (BY_MASS) mine = acc_of(mk128(L.mlo[b], 0) + ((u128)L.mhi[b] << 32), L.cnt[b]);
    }
    Acc tot;
    const Acc ex = block_scan_acc(mine, sc, &tot);
    const u128 lo_m = BY_MASS ? acc_mass(ex) : (u128)ex.c;
    const u128 sz = BY_MASS ? acc_mass(mine) : (u128)mine.c;
    if (tid == 0) sc.r[0] = 0xffffffffu;
    __syncthreads();
    if (live && sz > 0 && target >= lo_m && target < lo_m + sz) {
      sc.r[0] = (u32)b;
      sc.w[3 * kWaves] = ex.lo;
      sc.w[3 * kWaves + 1] = ex.hi;
      sc.w[3 * kWaves + 2] = ex.c;
      sc.w[3 * kWaves + 3] = ((u64)mine.c << 32);
    }
    __syncthreads();
    const u32 d = sc.r[0];
    const Acc bex = {sc.w[3 * kWaves], sc.w[3 * kWaves + 1], (u32)sc.w[3 * kWaves + 2]};
    __syncthreads();
    if (d == 0xffffffffu) {
      out.ok = false;
      return out;
    }
    out.before = acc_add(out.before, bex);
    target -= BY_MASS ? acc_mass(bex) : (u128)bex.c;
    prefix |= d << lo;
    mask |= dmask << lo;
    if (lo == 0) {
      // the bin of the last level holds exactly the members equal to prefix
      out.at.c = L.cnt[d];
      if (BY_MASS) out.at = acc_of(mk128(L.mlo[d], 0) + ((u128)L.mhi[d] << 32), L.cnt[d]);
      __syncthreads();
      break;
    }
    hi = lo - 1;
  }
  out.val = prefix;
  return out;
}

// ---------------------------------------------------------------- row sync

// Every workgroup of the row calls this the same number of times.
__device__ __forceinline__ void row_barrier(RowCtl* c, u32 G, u32 epoch) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) {
    addc(&c->bar, 1u);
    const u32 target = G * epoch;
    u32 spins = 0;
    while (ldc(&c->bar) < target) {
      if (++spins > kSpinLimit || (ldc(&c->status) & kStTimeout)) {
        orc(&c->status, kStTimeout);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

// Arrival of a workgroup that has finished with the row; true for the last one.
__device__ __forceinline__ bool arrive_last(RowCtl* c, u32 G, Scratch& s) {
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) s.r[7] = (addc(&c->arrive, 1u) == G - 1u) ? 1u : 0u;
  __syncthreads();
  const bool last = s.r[7] != 0u;
  __syncthreads();
  return last;
}

// Called by the last workgroup of the row: counters and histograms to zero.
__device__ __forceinline__ void reset_row(const Args& a, int row) {
  u32* w = (u32*)(a.ctl + row);
  if (threadIdx.x < kCtlZeroWords) stc(&w[threadIdx.x], 0u);
  u64* h = a.mhist + (size_t)row * 2 * kBins;
  for (int i = threadIdx.x; i < 2 * kBins; i += kThreads) stc(&h[i], 0ull);
}

__device__ __forceinline__ void publish_result(const Args& a, int row, long long id, int N, u128 W, u32 kp, u32 idp,
                                               bool greedy, u32 path) {
  RowCtl* c = a.ctl + row;
  c->path = path;
  a.out_ids[row] = id;
  c->chosen = id;
  c->n_max = N;
  c->w_lo = (u64)W;
  c->w_hi = (u64)(W >> 64);
  c->kappa_p = kp;
  c->id_p = idp;
  c->greedy = greedy ? 1u : 0u;
}

// ---------------------------------------------------------------- penalties

// LDS table of the history counts of one chunk [start, end): a bitmap of the
// tokens present, per-word prefix counts, and the count per present token.
struct PenTable {
  u32* bits;
  u32* wpre;
  u32* cnts;
};

__device__ __forceinline__ void pen_build(const Args& a, int row, int start, int end, PenTable t, Scratch& s) {
  constexpr int kPer = kMaxHistory / kThreads;  // history ids per thread (registers)
  const int nw = a.CH >> 5;
  for (int i = threadIdx.x; i < nw; i += kThreads) t.bits[i] = 0u;
  for (int i = threadIdx.x; i < a.seg_cap; i += kThreads) t.cnts[i] = 0u;
  // the row's history ids that fall in this chunk, chunk-relative (-1 otherwise);
  // all loads are issued before any is used
  const int* h = a.hist + (size_t)row * a.H;
  int loc[kPer];
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int i = q * kThreads + threadIdx.x;
    loc[q] = i < a.H ? h[i] : -1;
  }
#pragma unroll
  for (int q = 0; q < kPer; ++q) loc[q] = (loc[q] >= start && loc[q] < end) ? loc[q] - start : -1;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kPer; ++q)
    if (loc[q] >= 0) atomicOr(&t.bits[loc[q] >> 5], 1u << (loc[q] & 31));
  __syncthreads();
  const int per = (nw + kThreads - 1) / kThreads;
  u32 cnt = 0;
  for (int q = 0; q < per; ++q) {
    const int w = threadIdx.x * per + q;
    if (w < nw) cnt += __popc(t.bits[w]);
  }
  u32 tot;
  u32 run = block_scan_u32(cnt, s, &tot);
  for (int q = 0; q < per; ++q) {
    const int w = threadIdx.x * per + q;
    if (w < nw) {
      t.wpre[w] = run;
      run += __popc(t.bits[w]);
    }
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kPer; ++q) {
    const int l = loc[q];
    if (l >= 0) {
      const u32 bw = t.bits[l >> 5];
      atomicAdd(&t.cnts[t.wpre[l >> 5] + __popc(bw & ((1u << (l & 31)) - 1u))], 1u);
    }
  }
  __syncthreads();
}

__device__ __forceinline__ u32 pen_count(const PenTable& t, int l) {
  const u32 bw = t.bits[l >> 5];
  if (!((bw >> (l & 31)) & 1u)) return 0u;
  return t.cnts[t.wpre[l >> 5] + __popc(bw & ((1u << (l & 31)) - 1u))];
}

// Count of `id` in an ascending LDS array of n ids.
__device__ __forceinline__ u32 count_sorted(const int* s, int n, int id) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int m = (lo + hi) >> 1;
    if (s[m] < id) lo = m + 1; else hi = m;
  }
  int lo2 = lo, hi2 = n;
  while (lo2 < hi2) {
    const int m = (lo2 + hi2) >> 1;
    if (s[m] <= id) lo2 = m + 1; else hi2 = m;
  }
  return (u32)(lo2 - lo);
}

// ---------------------------------------------------------------- single-workgroup exact path

struct SingleLds {
  u32 cnt[kBins];
  u64 mlo[kBins];
  u64 mhi[kBins];
};

template <int DT>
__device__ __forceinline__ float single_q(const Args& a, const RowParams& p, int row, int i, const int* sh, int Hs) {
  float z = load_logit<DT>(a, row, i);
  if (p.pen_on) {
    const u32 c = count_sorted(sh, Hs, i);
    if (c) z = apply_penalty(z, c, p.rep, p.pres, p.freq);
  }
  return z / p.T;
}

// Over nb bins scanned from the top bin down, the bin where the running
// count (by_count) or mass first exceeds `target`.  Writes the bin and the
// (count, mass) of the bins above it; bin -1 if the total does not exceed it.
__device__ __forceinline__ void find_bin(const SingleLds& L, bool by_count, u128 target, Scratch& s, int* out_bin, Acc* above) {
  constexpr int per = kBins / kThreads > 0 ? kBins / kThreads : 1;
  Acc loc = {0, 0, 0};
  for (int q = 0; q < per; ++q) {
    const int b = kBins - 1 - (threadIdx.x * per + q);
    if (b < 0) break;
    loc = acc_add(loc, acc_of(mk128(L.mlo[b], 0) + ((u128)L.mhi[b] << 32), L.cnt[b]));
  }
  if (threadIdx.x == 0) s.i[0] = -1;
  Acc tot;
  const Acc ex = block_scan_acc(loc, s, &tot);
  const u128 lo = by_count ? (u128)ex.c : acc_mass(ex);
  const u128 sz = by_count ? (u128)loc.c : acc_mass(loc);
  if (target >= lo && target < lo + sz) {
    Acc run = ex;
    for (int q = 0; q < per; ++q) {
      const int b = kBins - 1 - (threadIdx.x * per + q);
      if (b < 0) break;
      const Acc nxt = acc_add(run, acc_of(mk128(L.mlo[b], 0) + ((u128)L.mhi[b] << 32), L.cnt[b]));
      const u128 hv = by_count ? (u128)nxt.c : acc_mass(nxt);
      if (target < hv) {
        s.i[0] = b;
        s.w[3 * kWaves] = run.lo;
        s.w[3 * kWaves + 1] = run.hi;
        s.w[3 * kWaves + 2] = run.c;
        break;
      }
      run = nxt;
    }
  }
  __syncthreads();
  *out_bin = s.i[0];
  above->lo = s.w[3 * kWaves];
  above->hi = s.w[3 * kWaves + 1];
  above->c = (u32)s.w[3 * kWaves + 2];
  __syncthreads();
}

struct Found {
  u32 key;
  Acc above;  // keys above `key`
  Acc tie;    // tokens at `key`
  bool ok;
};

// Radix select (8-bit digits) over the row among keys >= key_lo, by rank
// (by_count) or by mass.
template <int DT>
__device__ __forceinline__ Found radix_find(const Args& a, const RowParams& p, int row, int N, u32 key_lo, bool by_count,
                            u128 target, SingleLds& L, const int* sh, int Hs, Scratch& s) {
  u32 prefix = 0u, mask = 0u;
  Acc above = {0, 0, 0}, tie = {0, 0, 0};
  for (int lv = 0; lv < 4; ++lv) {
    const int shift = 24 - 8 * lv;
    for (int i = threadIdx.x; i < kBins; i += kThreads) {
      L.cnt[i] = 0u;
      L.mlo[i] = 0ull;
      L.mhi[i] = 0ull;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.V; i += kThreads) {
      const float q = single_q<DT>(a, p, row, i, sh, Hs);
      const u32 k = skey(q);
      if (k < key_lo || (k & mask) != prefix) continue;
      const u32 d = (k >> shift) & 0xffu;
      atomicAdd(&L.cnt[d], 1u);
      const u64 w = weight_of(q, N);
      if (w) {
        atomicAdd(&L.mlo[d], w & 0xffffffffull);
        atomicAdd(&L.mhi[d], w >> 32);
      }
    }
    __syncthreads();
    int d;
    Acc ab;
    find_bin(L, by_count, target, s, &d, &ab);
    if (d < 0) {
      Found f = {0u, above, tie, false};
      return f;
    }
    above = acc_add(above, ab);
    target -= by_count ? (u128)ab.c : acc_mass(ab);
    prefix |= (u32)d << shift;
    mask |= 0xffu << shift;
    tie = acc_of(mk128(L.mlo[d], 0) + ((u128)L.mhi[d] << 32), L.cnt[d]);
    __syncthreads();
  }
  Found f = {prefix, above, tie, true};
  return f;
}

// Resolve one sampling row exactly with this workgroup alone, re-reading the
// row from global memory.  Returns the sampled id.
template <int DT>
__device__ __forceinline__ void resolve_single(const Args& a, const RowParams& p, int row, unsigned char* lds, Scratch& s) {
  SingleLds& L = *(SingleLds*)lds;
  int* sh = (int*)(lds + sizeof(SingleLds));
  int Hs = 0;
  if (p.pen_on) {
    Hs = a.Hpad;
    const int* h = a.hist + (size_t)row * a.H;
    for (int i = threadIdx.x; i < Hs; i += kThreads) {
      const int id = i < a.H ? h[i] : -1;
      sh[i] = (id >= 0 && id < a.V) ? id : 0x7fffffff;
    }
    __syncthreads();
    bitonic_i32(sh, Hs);
  }
  // row scale N
  u32 km = 0u;
  for (int i = threadIdx.x; i < a.V; i += kThreads) {
    const u32 k = skey(single_q<DT>(a, p, row, i, sh, Hs));
    km = k > km ? k : km;
  }
  km = block_max_u32(km, s);
  const int N = octave_of(f_of_key(km));
  // top-k
  u32 kappa_k = 0u;
  u128 S;
  if (p.topk_on) {
    const Found f = radix_find<DT>(a, p, row, N, 0u, true, (u128)(p.k - 1), L, sh, Hs, s);
    kappa_k = f.key;
    S = acc_mass(acc_add(f.above, f.tie));
  } else {
    Acc loc = {0, 0, 0};
    for (int i = threadIdx.x; i < a.V; i += kThreads)
      loc = acc_add(loc, acc_of((u128)weight_of(single_q<DT>(a, p, row, i, sh, Hs), N), 0u));
    S = acc_mass(block_sum_acc(loc, s));
  }
  u32 kappa_p = kappa_k, id_p = 0xffffffffu;
  u128 W = S;
  if (p.topp_on) {
    const u128 Tp = mul_frac(S, p.tp);
    const Found f = radix_find<DT>(a, p, row, N, kappa_k, false, Tp, L, sh, Hs, s);
    if (f.ok) {
      kappa_p = f.key;
      const u128 A = acc_mass(f.above);
      const u64 wk = weight_of(f_of_key(f.key), N);
      const u64 j = (wk && Tp >= A) ? div_small(Tp - A, wk) : 0ull;  // boundary member (0-based)
      if (j + 1 >= f.tie.c) {
        W = acc_mass(acc_add(f.above, f.tie));
      } else {
        W = A + (u128)wk * (u128)(j + 1);
        // id of the j-th tie member in ascending id
        const int Lr = (a.V + kThreads - 1) / kThreads;
        const int i0 = threadIdx.x * Lr, i1 = min(a.V, i0 + Lr);
        u32 c = 0;
        for (int i = i0; i < i1; ++i)
          if (skey(single_q<DT>(a, p, row, i, sh, Hs)) == kappa_p) ++c;
        if (threadIdx.x == 0) s.r[6] = 0xffffffffu;
        u32 tot;
        const u32 ex = block_scan_u32(c, s, &tot);
        if (j >= ex && j < (u64)ex + c) {
          u32 r = ex;
          for (int i = i0; i < i1; ++i) {
            if (skey(single_q<DT>(a, p, row, i, sh, Hs)) == kappa_p) {
              if (r == j) {
                s.r[6] = (u32)i;
                break;
              }
              ++r;
            }
          }
        }
        __syncthreads();
        id_p = s.r[6];
        __syncthreads();
      }
    }
  }
  // draw in ascending id over kept tokens
  const u128 t = mul_frac(W, p.u);
  const int Lr = (a.V + kThreads - 1) / kThreads;
  const int i0 = threadIdx.x * Lr, i1 = min(a.V, i0 + Lr);
  Acc loc = {0, 0, 0};
  for (int i = i0; i < i1; ++i) {
    const float q = single_q<DT>(a, p, row, i, sh, Hs);
    const u32 k = skey(q);
    if (k > kappa_p || (k == kappa_p && (u32)i <= id_p)) loc = acc_add(loc, acc_of((u128)weight_of(q, N), 0u));
  }
  Acc tot;
  const Acc ex = block_scan_acc(loc, s, &tot);
  if (threadIdx.x == 0) s.r[6] = 0xffffffffu;
  __syncthreads();
  {
    const u128 lo = acc_mass(ex);
    if (t >= lo && t < lo + acc_mass(loc)) {
      u128 run = lo;
      for (int i = i0; i < i1; ++i) {
        const float q = single_q<DT>(a, p, row, i, sh, Hs);
        const u32 k = skey(q);
        if (k > kappa_p || (k == kappa_p && (u32)i <= id_p)) {
          run += (u128)weight_of(q, N);
          if (run > t) {
            s.r[6] = (u32)i;
            break;
          }
        }
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) publish_result(a, row, (long long)s.r[6], N, W, kappa_p, id_p, false, 3u);
  __syncthreads();
}

// ---------------------------------------------------------------- top-k finish

// s[0, m): candidates (skey(z) << 32 | ~id), m <= kMergeCap; `zout` is the
// largest skey(z) of the row's tokens outside them (0 if none).  Resolves
// top-k, top-p and the draw with LDS radix selects (no sorting); false if the
// candidates cannot be proven to hold the top-k set.
__device__ __forceinline__ bool finish_topk(const Args& a, const RowParams& p, int row, u64* s, int m, u32 zout,
                                            SelLds& L, Scratch& sc) {
  if (m < p.k) return false;
  const int tid = threadIdx.x;
  // key q = z / T
  for (int i = tid; i < m; i += kThreads) {
    const u64 c = s[i];
    s[i] = ((u64)skey(f_of_key((u32)(c >> 32)) / p.T) << 32) | (u32)c;
  }
  __syncthreads();
  auto key = [&](int i) { return (u32)(s[i] >> 32); };
  auto idof = [&](int i) { return 0xffffffffu - (u32)s[i]; };
  auto all = [&](int) { return true; };
  auto nowt = [&](int) { return 0ull; };
  // k-th largest q
  const SelOut sk = lds_select<false, true>(m, key, all, nowt, (u128)(p.k - 1), L, sc);
  if (!sk.ok) return false;
  const u32 kqk = sk.val;
  QS_TR(6);
  // every token outside has z <= f_of_key(zout), so q <= that / T: it must be below q_k
  if (zout > 0u && skey(f_of_key(zout) / p.T) >= kqk) return false;
  u32 mx = 0u;
  for (int i = tid; i < m; i += kThreads) mx = key(i) > mx ? key(i) : mx;
  mx = block_max_u32(mx, sc);
  const int N = octave_of(f_of_key(mx));
  auto wt = [&](int i) { return weight_of(f_of_key(key(i)), N); };
  auto intop = [&](int i) { return key(i) >= kqk; };
  u128 sv = 0;
  for (int i = tid; i < m; i += kThreads)
    if (intop(i)) sv += (u128)wt(i);
  const u128 S = block_sum128(sv, sc);
  QS_TR(13);
  u32 kappa_p = kqk, id_p = 0xffffffffu;  // kept: key > kappa_p || (key == kappa_p && id <= id_p)
  u128 W = S;
  if (p.topp_on) {
    // the first token (q desc, id asc) whose inclusive mass exceeds floor(top_p * S)
    const u128 Tp = mul_frac(S, p.tp);
    const SelOut sp = lds_select<true, true>(m, key, intop, wt, Tp, L, sc);
    QS_TR(14);
    if (!sp.ok) return false;
    kappa_p = sp.val;
    const u128 A = acc_mass(sp.before);
    const u64 wk = weight_of(f_of_key(kappa_p), N);
    const u64 j = div_small(Tp - A, wk);  // 0-based boundary member among the ties (< sp.at.c)
    if (j + 1 >= sp.at.c) {
      W = A + acc_mass(sp.at);
    } else {
      W = A + (u128)wk * (u128)(j + 1);
      auto intie = [&](int i) { return key(i) == kappa_p; };
      const SelOut si = lds_select<false, false>(m, idof, intie, nowt, (u128)j, L, sc);
      if (!si.ok) return false;
      id_p = si.val;
    }
  }
  // draw: kept tokens in ascending id, the first whose inclusive mass exceeds floor(u * W)
  const u128 t = mul_frac(W, p.u);
  auto kept = [&](int i) {
    const u32 k = key(i);
    return k > kappa_p || (k == kappa_p && idof(i) <= id_p);
  };
  const SelOut sd = lds_select<true, false>(m, idof, kept, wt, t, L, sc);
  if (tid == 0)
    publish_result(a, row, sd.ok ? (long long)sd.val : -1ll, N, W, kappa_p, id_p, false, 1u);
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------- mass rows


struct MassLds {
  u64 h[kBins];             // local histogram (fixed-point mass >> 24)
  u64 g[kBins];             // merged histogram, read back
  u64 a_lo[kMaxChunks];     // per-chunk published mass (chunk mass or mass above the bracket)
  u64 a_hi[kMaxChunks];
  u32 nbv[kMaxChunks];      // per-chunk bracketed token count
  u32 pref[kMaxChunks];     // exclusive prefix of nbv
  u64 c_lo[kMaxChunks];     // per-chunk kept mass of bracketed tokens, lo 32-bit parts
  u64 c_hi[kMaxChunks];     //   hi parts
  u64 list[kBracketCap];    // bracketed tokens (key << 32 | ~id)
  SelLds sel;
};

__device__ __forceinline__ void load_slots(MassLds& M, const Slot* sl, int G) {
  for (int g = threadIdx.x; g < G; g += kThreads) {
    M.a_lo[g] = ldc(&sl[g].s_lo);
    M.a_hi[g] = ldc(&sl[g].s_hi);
    M.nbv[g] = ldc(&sl[g].nb);
  }
  __syncthreads();
}

// Bracket of bins [blo, bhi] that provably holds the top-p boundary (the first
// token, in descending order, whose inclusive mass exceeds Tp).  `g` holds,
// per bin, the sum over its tokens of (w >> 24); `above` is the same-units
// mass above the histogram's range and `err` bounds the truncation over all
// tokens counted (each loses less than one unit).  One bin per thread.
//   bhi: the lowest bin whose mass above it is provably <= Tp;
//   blo: the highest bin whose mass at or above it is provably > Tp.
__device__ __forceinline__ void bracket_bins(const u64* g, u64 above, u64 err, u128 Tp, Scratch& sc, int* blo,
                                             int* bhi) {
  static_assert(kBins == kThreads, "one histogram bin per thread");
  const int tid = threadIdx.x;
  const int b = kBins - 1 - tid;  // thread order = descending bins
  const u64 gb = g[b];
  Acc tot;
  const Acc ex = block_scan_acc(acc_of((u128)gb, 0u), sc, &tot);
  const u128 run = (u128)above + acc_mass(ex);  // lower bound of the mass above bin b
  if (tid == 0) {
    sc.r[6] = 0xffffffffu;  // min over bins satisfying the bhi condition
    sc.r[7] = 0u;           // max over bins satisfying the blo condition, +1
  }
  __syncthreads();
  if (((run + err) << 24) <= Tp) atomicMin(&sc.r[6], (u32)b);
  if (((run + gb) << 24) > Tp) atomicMax(&sc.r[7], (u32)b + 1u);
  __syncthreads();
  int hi = sc.r[6] == 0xffffffffu ? kBins - 1 : (int)sc.r[6];
  int lo = sc.r[7] == 0u ? 0 : (int)sc.r[7] - 1;
  __syncthreads();
  if (lo > hi) lo = hi;
  *blo = lo;
  *bhi = hi;
}

// ---------------------------------------------------------------- main kernel

// ROLE 0 resolves greedy, top-k and large-k rows (and mass rows when no mass
// launch follows); ROLE 1 resolves the mass rows only.
template <int DT, int EPT, int ROLE>
__global__ __launch_bounds__(kThreads) void k_sample(Args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ Scratch sc;
  __shared__ u32 tmax_s[kThreads];
  constexpr int VW = (DT == QS_DTYPE_F32) ? 4 : 8;
  constexpr int NV = EPT / VW;
  const int row = blockIdx.y, blk = blockIdx.x, tid = threadIdx.x;
  const int start = blk * a.CH;
  const int end = min(a.V, start + a.CH);
  const RowParams p = row_params(a, row);
  RowCtl* c = a.ctl + row;
  if (ROLE == 1 && p.kind != kMass) return;
  if (ROLE == 0 && p.kind == kMass && !(a.flags & QS_FLAG_NO_MASS_ROWS)) return;
  QS_TR(0);

  if (ROLE == 0 && (p.kind == kSingle || p.kind == kMass)) {
    if (blk == 0) {
      if (DT == QS_DTYPE_F32) resolve_single<QS_DTYPE_F32>(a, p, row, lds, sc);
      else resolve_single<QS_DTYPE_BF16>(a, p, row, lds, sc);
    }
    if (arrive_last(c, (u32)a.G, sc)) reset_row(a, row);
    return;
  }

  // ---- penalty table for the chunk, then the chunk into registers
  PenTable pt;
  pt.bits = (u32*)lds;
  pt.wpre = pt.bits + (a.CH >> 5);
  pt.cnts = pt.wpre + (a.CH >> 5);
  if (p.pen_on) pen_build(a, row, start, end, pt, sc);
  QS_TR(1);

  float z[EPT];
  {
    const bool vec = ((((uintptr_t)a.logits) | ((size_t)a.row_stride * (DT == QS_DTYPE_F32 ? 4 : 2))) & 15) == 0;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int e0 = start + (v * kThreads + tid) * VW;
      if (vec && e0 + VW <= end) {
        if (DT == QS_DTYPE_F32) {
          const float4 q = *(const float4*)((const float*)a.logits + (size_t)row * a.row_stride + e0);
          z[v * VW + 0] = q.x;
          z[v * VW + 1] = q.y;
          z[v * VW + 2] = q.z;
          z[v * VW + 3] = q.w;
        } else {
          const uint4 q = *(const uint4*)((const uint16_t*)a.logits + (size_t)row * a.row_stride + e0);
          const u32 w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            z[v * VW + 2 * j] = bf16_to_f32(w4[j] & 0xffffu);
            z[v * VW + 2 * j + 1] = bf16_to_f32(w4[j] >> 16);
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const int e = e0 + j;
          z[v * VW + j] = (e < end) ? load_logit<DT>(a, row, e) : 0.0f;
        }
      }
      if (p.pen_on) {
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const int e = e0 + j;
          if (e < end) {
            const u32 cnt = pen_count(pt, e - start);
            if (cnt) z[v * VW + j] = apply_penalty(z[v * VW + j], cnt, p.rep, p.pres, p.freq);
          }
        }
      }
    }
  }
  if (p.pen_on) __syncthreads();  // the LDS table is reused below

#define QS_FOR_ELEMS(...)                                   \
  _Pragma("unroll") for (int v = 0; v < NV; ++v) {          \
    _Pragma("unroll") for (int j = 0; j < VW; ++j) {        \
      const int e = start + (v * kThreads + tid) * VW + j;  \
      if (e < end) {                                        \
        float& zz = z[v * VW + j];                          \
        (void)zz;                                           \
        __VA_ARGS__                                         \
      }                                                     \
    }                                                       \
  }

  if constexpr (ROLE == 0) {
  // ================================================================ greedy
  if (p.kind == kGreedy) {
    u64 best = 0ull;
    QS_FOR_ELEMS({
      const u64 pk = ((u64)gkey(zz) << 32) | (0xffffffffu - (u32)e);
      best = pk > best ? pk : best;
    })
    best = block_max_u64(best, sc);
    QS_TR(2);
    if (tid == 0) maxc(&c->pack, best);
    if (arrive_last(c, (u32)a.G, sc)) {
      QS_TR(4);
      if (tid == 0) {
        const u64 pk = maxc(&c->pack, 0ull);
        publish_result(a, row, (long long)(0xffffffffu - (u32)pk), 0, 0, 0u, 0u, true, 0u);
      }
      reset_row(a, row);
    }
    return;
  }

  // ================================================================ top-k
  if (p.kind == kTopK) {
    u32 tm = 0u;
    QS_FOR_ELEMS({
      const u32 k = skey(zz);
      tm = k > tm ? k : tm;
    })
    // tau: at least kc tokens of the chunk are >= tau.  kc covers this chunk's
    // expected share of the row's top-k with a wide margin.  Each wave sorts
    // its 64 per-thread maxima (shuffles) and takes the ceil(kc/4)-th largest;
    // the workgroup takes the smallest of the four.
    const float mu = (float)p.k / (float)a.G;
    int kc = (int)ceilf(mu) + 4 * (int)ceilf(sqrtf(mu)) + 4;
    kc = min(kc, min(p.k, kThreads));
    const int kw = (kc + kWaves - 1) / kWaves;
    const int lane = tid & 63;
    u32 x = tm;
    for (int k2 = 2; k2 <= 64; k2 <<= 1) {
      for (int j = k2 >> 1; j > 0; j >>= 1) {
        const u32 o = __shfl_xor(x, j, 64);
        const bool take_small = ((lane & j) == 0) == ((lane & k2) != 0);
        x = take_small ? (o < x ? o : x) : (o > x ? o : x);
      }
    }
    const u32 tw = __shfl(x, kw - 1, 64);
    if (lane == 0) tmax_s[tid >> 6] = tw;
    __syncthreads();
    QS_TR(2);
    u32 tau = tmax_s[0];
    for (int w = 1; w < kWaves; ++w) tau = tmax_s[w] < tau ? tmax_s[w] : tau;
    u32 mine = 0, below = 0u;
    QS_FOR_ELEMS({
      const u32 k = skey(zz);
      if (k >= tau) ++mine;
      else below = k > below ? k : below;
    })
    below = block_max_u32(below, sc);
    u32 total;
    const u32 off = block_scan_u32(mine, sc, &total);
    const bool fits = total <= (u32)kBlockCand;
    if (fits) {
      u64* cd = a.cand + ((size_t)row * a.G + blk) * kBlockCand + off;
      u32 pos = 0;
      QS_FOR_ELEMS({
        const u32 k = skey(zz);
        if (k >= tau) {
          stc(&cd[pos], ((u64)k << 32) | (0xffffffffu - (u32)e));
          ++pos;
        }
      })
    }
    Slot* sl = a.slots + (size_t)row * a.G + blk;
    if (tid == 0) {
      stc(&sl->nb, fits ? total : 0xffffffffu);
      stc(&sl->pad[0], tau);
      stc(&sl->pad[1], below);
    }
    QS_TR(3);
    if (!arrive_last(c, (u32)a.G, sc)) {
      QS_TR(15);
      return;
    }
    QS_TR(4);
    // ---- the last workgroup merges and resolves the row
    u64* s = (u64*)lds;                    // merged candidates [kMergeCap]
    u32* offs = (u32*)(s + kMergeCap);     // per-workgroup candidate offsets [G]
    SelLds& SL = *(SelLds*)(offs + kMaxChunks);
    const Slot* slr = a.slots + (size_t)row * a.G;
    // per-workgroup counts, thresholds and maxima below them (one load each)
    const int gper = (a.G + kThreads - 1) / kThreads;
    u32 cnt_loc = 0, tstar_loc = 0, nout_loc = 0, ovf = 0;
    for (int q = 0; q < gper; ++q) {
      const int g = tid * gper + q;
      if (g < a.G) {
        const u32 cg = ldc(&slr[g].nb);
        const u32 tg = ldc(&slr[g].pad[0]);
        const u32 bg = ldc(&slr[g].pad[1]);
        if (cg == 0xffffffffu) ovf = 1u;
        offs[g] = (cg == 0xffffffffu) ? 0u : cg;
        tstar_loc = tg > tstar_loc ? tg : tstar_loc;
        nout_loc = bg > nout_loc ? bg : nout_loc;
      }
    }
    __syncthreads();
    QS_TR(11);
    for (int q = 0; q < gper; ++q) {
      const int g = tid * gper + q;
      if (g < a.G) cnt_loc += offs[g];
    }
    const u32 tstar = block_max_u32(tstar_loc, sc);
    const u32 nout = block_max_u32(nout_loc, sc);
    const bool overflow = block_max_u32(ovf, sc) != 0u;
    u32 M;
    {
      u32 run = block_scan_u32(cnt_loc, sc, &M);
      for (int q = 0; q < gper; ++q) {
        const int g = tid * gper + q;
        if (g < a.G) {
          const u32 cg = offs[g];
          offs[g] = run;
          run += cg;
        }
      }
    }
    if (tid == 0) {
      sc.r[3] = 0u;    // merged count
      sc.r[2] = nout;  // max key outside the merged set
    }
    __syncthreads();
    QS_TR(12);
    bool ok = !overflow;
    if (ok) {
      // each thread takes a contiguous run of the M emitted candidates (in
      // workgroup order); all its loads are issued before any is used
      const u64* cd = a.cand + (size_t)row * a.G * kBlockCand;
      const u32 per = (M + kThreads - 1) / kThreads;
      for (u32 base = 0; base < per; base += 16) {
        const u32 f0 = (u32)tid * per + base;
        u64 vals[16];
        int g = 0;
        if (f0 < M) {
          int lo = 0, hi = a.G - 1;  // last g with offs[g] <= f0
          while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (offs[mid] <= f0) lo = mid; else hi = mid - 1;
          }
          g = lo;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const u32 f = f0 + (u32)r;
          const bool valid = (base + (u32)r < per) && f < M;
          if (valid)
            while (g + 1 < a.G && offs[g + 1] <= f) ++g;
          vals[r] = valid ? ldc(&cd[(size_t)g * kBlockCand + (f - offs[g])]) : 0ull;
        }
        u32 outmax = 0u;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const u32 f = f0 + (u32)r;
          const bool valid = (base + (u32)r < per) && f < M;
          const u32 k = (u32)(vals[r] >> 32);
          const bool take = valid && k >= tstar;
          const u32 slot = wave_append(take, &sc.r[3]);
          if (take && slot < (u32)kMergeCap) s[slot] = vals[r];
          if (valid && !take) outmax = k > outmax ? k : outmax;
        }
        outmax = wave_max(outmax);
        if ((tid & 63) == 0 && outmax) atomicMax(&sc.r[2], outmax);
      }
      __syncthreads();
      const u32 m = sc.r[3];
      const u32 zout = sc.r[2];
      __syncthreads();
      QS_TR(5);
      ok = m <= (u32)kMergeCap && finish_topk(a, p, row, s, (int)m, zout, SL, sc);
    }
    if (!ok) {
      if (DT == QS_DTYPE_F32) resolve_single<QS_DTYPE_F32>(a, p, row, lds, sc);
      else resolve_single<QS_DTYPE_BF16>(a, p, row, lds, sc);
    }
    QS_TR(7);
    reset_row(a, row);
    QS_TR(15);
    return;
  }
  } else {
  // ================================================================ mass rows
  MassLds& M = *(MassLds*)lds;
  Slot* slots = a.slots + (size_t)row * a.G;
  // q = z / T; key range of the row
  u32 kmx = 0u, kmn = 0xffffffffu;
  QS_FOR_ELEMS({
    zz = zz / p.T;
    const u32 k = skey(zz);
    kmx = k > kmx ? k : kmx;
    kmn = k < kmn ? k : kmn;
  })
  kmx = block_max_u32(kmx, sc);
  kmn = ~block_max_u32(~kmn, sc);
  QS_TR(2);
  if (tid == 0) {
    maxc(&c->kmax, kmx);
    maxc(&c->nkmin, ~kmn);
  }
  QS_TR(3);
  row_barrier(c, (u32)a.G, 1u);
  QS_TR(4);
  const u32 rkmax = ldc(&c->kmax);
  const u32 rkmin = ~ldc(&c->nkmin);
  const float qmax = f_of_key(rkmax);
  const int N = octave_of(qmax);
  u128 W = 0;
  u32 kappa_p = 0u, id_p = 0xffffffffu;  // kept: key > kappa_p || (key == kappa_p && id <= id_p)
  bool failed = false;
  bool single_key = false;
  u32 bkey = 0u;
  u64 bw = 0ull;     // weight of the single bracket key
  u64 jkeep = 0ull;  // single key: bracketed tokens kept, in id order

  if (!p.topp_on) {
    // ---- plain draw: chunk masses
    u128 acc = 0;
    QS_FOR_ELEMS({ acc += (u128)weight_of(zz, N); })
    acc = block_sum128(acc, sc);
    if (tid == 0) {
      stc(&slots[blk].s_lo, (u64)acc);
      stc(&slots[blk].s_hi, (u64)(acc >> 64));
    }
    row_barrier(c, (u32)a.G, 2u);
    QS_TR(5);
    load_slots(M, slots, a.G);
    u128 v = 0;
    for (int g = tid; g < a.G; g += kThreads) v += mk128(M.a_lo[g], M.a_hi[g]);
    W = block_sum128(v, sc);
  } else {
    // ---- level 1: histogram over y in [ylo, yhi]
    const double yhi = y_of(qmax);
    double ylo = y_of(f_of_key(rkmin));
    if (ylo < (double)(N - kWindow)) ylo = (double)(N - kWindow);
    const double sc1 = (yhi > ylo) ? (double)kBins / (yhi - ylo) : 0.0;
    for (int i = tid; i < kBins; i += kThreads) M.h[i] = 0ull;
    __syncthreads();
    u128 acc = 0;
    QS_FOR_ELEMS({
      const double y = y_of(zz);
      const u64 w = weight_y(y, N);
      if (w) {
        acc += (u128)w;
        const int b = min(kBins - 1, (int)((y - ylo) * sc1));
        atomicAdd(&M.h[b], w >> 24);
      }
    })
    acc = block_sum128(acc, sc);  // its __syncthreads also orders the LDS atomics
    if (tid == 0) {
      stc(&slots[blk].s_lo, (u64)acc);
      stc(&slots[blk].s_hi, (u64)(acc >> 64));
    }
    u64* gh1 = a.mhist + (size_t)row * 2 * kBins;
    for (int i = tid; i < kBins; i += kThreads)
      if (M.h[i]) addc(&gh1[i], M.h[i]);
    row_barrier(c, (u32)a.G, 2u);
    QS_TR(5);
    // total mass S, the target, and the level-1 bracket
    load_slots(M, slots, a.G);
    u128 sv = 0;
    for (int g = tid; g < a.G; g += kThreads) sv += mk128(M.a_lo[g], M.a_hi[g]);
    const u128 S = block_sum128(sv, sc);
    const u128 Tp = mul_frac(S, p.tp);
    for (int i = tid; i < kBins; i += kThreads) M.g[i] = ldc(&gh1[i]);
    __syncthreads();
    const u64 err = (u64)a.V;  // each token truncates less than one unit
    int blo1, bhi1, blo2, bhi2;
    bracket_bins(M.g, 0ull, err, Tp, sc, &blo1, &bhi1);
    u64 above1;
    {
      const int b = kBins - 1 - tid;
      const u64 v = b > bhi1 ? M.g[b] : 0ull;
      above1 = (u64)acc_mass(block_sum_acc(acc_of((u128)v, 0u), sc));
    }
    // ---- level 2: histogram inside the level-1 bracket
    const double w1 = (sc1 > 0.0) ? 1.0 / sc1 : 0.0;
    const double ylo2 = ylo + (double)blo1 * w1;
    const double yhi2 = ylo + (double)(bhi1 + 1) * w1;
    const double sc2 = (sc1 > 0.0 && yhi2 > ylo2) ? (double)kBins / (yhi2 - ylo2) : 0.0;
    __syncthreads();
    for (int i = tid; i < kBins; i += kThreads) M.h[i] = 0ull;
    __syncthreads();
    QS_FOR_ELEMS({
      const double y = y_of(zz);
      const u64 w = weight_y(y, N);
      if (w) {
        const int b1 = min(kBins - 1, (int)((y - ylo) * sc1));
        if (b1 >= blo1 && b1 <= bhi1) {
          int b2 = (int)((y - ylo2) * sc2);
          b2 = b2 < 0 ? 0 : (b2 > kBins - 1 ? kBins - 1 : b2);
          atomicAdd(&M.h[b2], w >> 24);
        }
      }
    })
    __syncthreads();
    u64* gh2 = gh1 + kBins;
    for (int i = tid; i < kBins; i += kThreads)
      if (M.h[i]) addc(&gh2[i], M.h[i]);
    row_barrier(c, (u32)a.G, 3u);
    QS_TR(6);
    for (int i = tid; i < kBins; i += kThreads) M.g[i] = ldc(&gh2[i]);
    __syncthreads();
    bracket_bins(M.g, above1, err, Tp, sc, &blo2, &bhi2);
    __syncthreads();
    // ---- exact: mass above the bracket; bracketed tokens listed
    u128 accA = 0;
    u32 nb = 0, bkmx = 0u, bkmn = 0xffffffffu;
    QS_FOR_ELEMS({
      const double y = y_of(zz);
      const u64 w = weight_y(y, N);
      if (w) {
        const int b1 = min(kBins - 1, (int)((y - ylo) * sc1));
        bool above = b1 > bhi1, inside = false;
        if (b1 >= blo1 && b1 <= bhi1) {
          int b2 = (int)((y - ylo2) * sc2);
          b2 = b2 < 0 ? 0 : (b2 > kBins - 1 ? kBins - 1 : b2);
          above = b2 > bhi2;
          inside = b2 >= blo2 && b2 <= bhi2;
        }
        if (above) accA += (u128)w;
        if (inside) {
          const u32 k = skey(zz);
          ++nb;
          bkmx = k > bkmx ? k : bkmx;
          bkmn = k < bkmn ? k : bkmn;
        }
      }
    })
    accA = block_sum128(accA, sc);
    bkmx = block_max_u32(bkmx, sc);
    bkmn = ~block_max_u32(~bkmn, sc);
    u32 nbt;
    const u32 nboff = block_scan_u32(nb, sc, &nbt);
    if (tid == 0) {
      stc(&slots[blk].s_lo, (u64)accA);
      stc(&slots[blk].s_hi, (u64)(accA >> 64));
      stc(&slots[blk].nb, nbt);
      if (nbt) {
        maxc(&c->brk_kmax, bkmx);
        maxc(&c->brk_nkmin, ~bkmn);
        sc.r[4] = addc(&c->brk_n, nbt);
      }
    }
    __syncthreads();
    const u32 bbase = sc.r[4];
    if (nbt && (u64)bbase + nbt <= (u64)kBracketCap) {
      u64* bl = a.brk + (size_t)row * kBracketCap + bbase + nboff;
      u32 pos = 0;
      QS_FOR_ELEMS({
        const double y = y_of(zz);
        if (weight_y(y, N)) {
          const int b1 = min(kBins - 1, (int)((y - ylo) * sc1));
          if (b1 >= blo1 && b1 <= bhi1) {
            int b2 = (int)((y - ylo2) * sc2);
            b2 = b2 < 0 ? 0 : (b2 > kBins - 1 ? kBins - 1 : b2);
            if (b2 >= blo2 && b2 <= bhi2) {
              stc(&bl[pos], ((u64)skey(zz) << 32) | (0xffffffffu - (u32)e));
              ++pos;
            }
          }
        }
      })
    }
    row_barrier(c, (u32)a.G, 4u);
    QS_TR(7);
    // ---- every workgroup resolves the boundary from the published data
    load_slots(M, slots, a.G);
    u128 av = 0;
    for (int g = tid; g < a.G; g += kThreads) av += mk128(M.a_lo[g], M.a_hi[g]);
    const u128 A = block_sum128(av, sc);
    const u32 nbr = ldc(&c->brk_n);
    const u32 gkmx = ldc(&c->brk_kmax), gkmn = ~ldc(&c->brk_nkmin);
    const bool bottom = (blo1 == 0 && blo2 == 0);
    if (A > Tp || nbr == 0u) {
      failed = true;
    } else if (gkmx == gkmn) {
      // one key in the bracket: all bracketed tokens weigh the same
      single_key = true;
      bkey = gkmx;
      bw = weight_of(f_of_key(bkey), N);
      // bracketed tokens with exclusive mass <= Tp: floor((Tp - A) / bw) + 1, at most nbr
      u64 j = nbr;
      if (Tp - A < (u128)bw * nbr) j = div_small(Tp - A, bw) + 1ull;
      if (j >= nbr) {
        j = nbr;
        if (A + (u128)bw * nbr <= Tp && !bottom) failed = true;
      }
      jkeep = j;
      W = A + (u128)bw * j;
      kappa_p = bkey;
    } else if (nbr > (u32)kBracketCap) {
      failed = true;
    } else {
      // the bracketed tokens in LDS (loads issued before use), then radix
      // selects: the boundary by mass, the boundary member among ties by id
      const u64* bl = a.brk + (size_t)row * kBracketCap;
      const int nn = (int)nbr;
      {
        constexpr int kPerT = kBracketCap / kThreads;
        u64 tmp[kPerT];
#pragma unroll
        for (int q = 0; q < kPerT; ++q) {
          const int i = q * kThreads + tid;
          tmp[q] = i < nn ? ldc(&bl[i]) : 0ull;
        }
#pragma unroll
        for (int q = 0; q < kPerT; ++q) {
          const int i = q * kThreads + tid;
          if (i < nn) M.list[i] = tmp[q];
        }
      }
      __syncthreads();
      auto key = [&](int i) { return (u32)(M.list[i] >> 32); };
      auto idof = [&](int i) { return 0xffffffffu - (u32)M.list[i]; };
      auto all = [&](int) { return true; };
      auto nowt = [&](int) { return 0ull; };
      auto wt = [&](int i) { return weight_of(f_of_key(key(i)), N); };
      const SelOut sp = lds_select<true, true>(nn, key, all, wt, Tp - A, M.sel, sc);
      if (!sp.ok) {
        // every bracketed token is kept: only right if nothing with weight lies below
        if (!bottom) failed = true;
        kappa_p = 0u;
        id_p = 0xffffffffu;
      } else {
        kappa_p = sp.val;
        const u128 A2 = A + acc_mass(sp.before);
        const u64 wk = weight_of(f_of_key(kappa_p), N);
        const u64 j = div_small(Tp - A2, wk);  // 0-based boundary member among the ties
        if (j + 1 < sp.at.c) {
          auto intie = [&](int i) { return key(i) == kappa_p; };
          const SelOut si = lds_select<false, false>(nn, idof, intie, nowt, (u128)j, M.sel, sc);
          if (!si.ok) failed = true;
          id_p = si.val;
        }
      }
      if (!failed) {
        // per-chunk mass of the kept bracketed tokens
        for (int g = tid; g < a.G; g += kThreads) {
          M.c_lo[g] = 0ull;
          M.c_hi[g] = 0ull;
        }
        __syncthreads();
        for (int i = tid; i < nn; i += kThreads) {
          const u32 k = key(i), id = idof(i);
          if (k > kappa_p || (k == kappa_p && id <= id_p)) {
            const u64 w = wt(i);
            const int ch = (int)(id / (u32)a.CH);
            atomicAdd(&M.c_lo[ch], w & 0xffffffffull);
            atomicAdd(&M.c_hi[ch], w >> 32);
          }
        }
        __syncthreads();
        u128 wv = 0;
        for (int g = tid; g < a.G; g += kThreads) wv += mk128(M.c_lo[g], 0) + ((u128)M.c_hi[g] << 32);
        W = A + block_sum128(wv, sc);
      }
    }
  }

  if (failed) {
    QS_TR(9);
    if (blk == 0) {
      if (DT == QS_DTYPE_F32) resolve_single<QS_DTYPE_F32>(a, p, row, lds, sc);
      else resolve_single<QS_DTYPE_BF16>(a, p, row, lds, sc);
    }
    if (arrive_last(c, (u32)a.G, sc)) reset_row(a, row);
    return;
  }

  // ---- the draw: kept mass per chunk, the chunk holding the target, then
  // that workgroup locates the token in id order
  const u128 t = mul_frac(W, p.u);
  const bool need_rank = p.topp_on && single_key;
  {
    // one chunk per thread (G <= kMaxChunks <= kThreads)
    const int g = tid;
    u32 nbg = 0;
    u128 wg = 0;
    if (g < a.G) {
      wg = mk128(M.a_lo[g], M.a_hi[g]);
      nbg = need_rank ? M.nbv[g] : 0u;
    }
    u32 nbtot;
    const u32 before = block_scan_u32(nbg, sc, &nbtot);
    if (g < a.G) {
      M.pref[g] = before;
      if (p.topp_on) {
        if (single_key) {
          const u64 keep = jkeep > before ? min((u64)nbg, jkeep - before) : 0ull;
          wg += (u128)bw * keep;
        } else {
          wg += mk128(M.c_lo[g], 0) + ((u128)M.c_hi[g] << 32);
        }
      }
    }
    Acc tot;
    const Acc ex = block_scan_acc(acc_of(wg, 0u), sc, &tot);
    if (tid == 0) sc.r[5] = (u32)(a.G - 1);  // unreachable fallback: t < W
    __syncthreads();
    if (g < a.G && t >= acc_mass(ex) && t < acc_mass(ex) + wg) {
      sc.r[5] = (u32)g;
      const u128 tl = t - acc_mass(ex);
      sc.w[3 * kWaves] = (u64)tl;
      sc.w[3 * kWaves + 1] = (u64)(tl >> 64);
    }
    __syncthreads();
  }
  const int owner = (int)sc.r[5];
  const u128 tloc = (owner == (int)sc.r[5]) ? mk128(sc.w[3 * kWaves], sc.w[3 * kWaves + 1]) : 0;
  __syncthreads();
  // single key: this chunk's kept bracketed tokens are its first `kmine` members in id order
  u64 kmine = 0ull;
  bool idp_me = false;
  if (need_rank) {
    const u64 before = M.pref[blk];
    const u64 nbme = M.nbv[blk];
    kmine = jkeep > before ? min(nbme, jkeep - before) : 0ull;
    // the workgroup holding the last kept member records its id (for k_probs)
    idp_me = jkeep > before && jkeep <= before + nbme;
  }
  const bool owner_me = (owner == blk);
  QS_TR(8);
  if (owner_me || idp_me) {
    // One pass over the chunk in id order, which is (v, thread, j).  Per v:
    // ranks of the single bracket key's members (id order), the kept mass,
    // and, in the vector that holds the draw target, the drawn token.
    u128 rem = tloc;
    u32 members = 0;  // members of the bracket key in earlier vectors
    bool found = false;
    if (tid == 0) {
      sc.r[1] = 0xffffffffu;
      sc.r[2] = 0xffffffffu;
    }
    __syncthreads();
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      u32 rank = 0;
      if (need_rank) {
        u32 mc = 0;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const int e = start + (v * kThreads + tid) * VW + j;
          if (e < end && skey(z[v * VW + j]) == bkey && weight_of(z[v * VW + j], N)) ++mc;
        }
        u32 mtot;
        rank = members + block_scan_u32(mc, sc, &mtot);
        members += mtot;
      }
      // kept mass of this thread's tokens in vector v (and the boundary member for k_probs)
      u128 part = 0;
      {
        u32 r = rank;
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const int e = start + (v * kThreads + tid) * VW + j;
          if (e < end) {
            const float q = z[v * VW + j];
            const u32 k = skey(q);
            const u64 w = weight_of(q, N);
            bool kept;
            if (!p.topp_on) {
              kept = true;
            } else if (single_key) {
              if (k == bkey && w) {
                kept = (u64)r < kmine;
                if (idp_me && (u64)r + 1 == kmine) sc.r[2] = (u32)e;
                ++r;
              } else {
                kept = k > bkey;
              }
            } else {
              kept = k > kappa_p || (k == kappa_p && (u32)e <= id_p);
            }
            if (kept) part += (u128)w;
          }
        }
      }
      if (owner_me && !found) {
        Acc tot;
        const Acc ex = block_scan_acc(acc_of(part, 0u), sc, &tot);
        const u128 tv = acc_mass(tot);
        if (rem < tv) {
          found = true;
          const u128 lo = acc_mass(ex);
          if (rem >= lo && rem < lo + part) {
            u128 runm = lo;
            u32 r = rank;
#pragma unroll
            for (int j = 0; j < VW; ++j) {
              const int e = start + (v * kThreads + tid) * VW + j;
              if (e < end) {
                const float q = z[v * VW + j];
                const u32 k = skey(q);
                const u64 w = weight_of(q, N);
                bool kept;
                if (!p.topp_on) {
                  kept = true;
                } else if (single_key) {
                  if (k == bkey && w) {
                    kept = (u64)r < kmine;
                    ++r;
                  } else {
                    kept = k > bkey;
                  }
                } else {
                  kept = k > kappa_p || (k == kappa_p && (u32)e <= id_p);
                }
                if (kept) {
                  runm += (u128)w;
                  if (runm > rem && sc.r[1] == 0xffffffffu) sc.r[1] = (u32)e;
                }
              }
            }
          }
        } else {
          rem -= tv;
        }
      }
    }
    __syncthreads();
    if (tid == 0) {
      RowCtl* cc = a.ctl + row;
      if (idp_me) cc->id_p = sc.r[2];
      if (owner_me) {
        // a timed-out row barrier leaves the row unresolved: report an invalid id
        if (ldc(&c->status) & kStTimeout) sc.r[1] = 0xffffffffu;
        a.out_ids[row] = (sc.r[1] == 0xffffffffu) ? -1ll : (long long)sc.r[1];
        cc->chosen = (long long)sc.r[1];
        cc->n_max = N;
        cc->w_lo = (u64)W;
        cc->w_hi = (u64)(W >> 64);
        cc->greedy = 0u;
        cc->path = 2u;
        cc->kappa_p = single_key ? bkey : kappa_p;
        if (!single_key) cc->id_p = id_p;
      }
    }
    __syncthreads();
  }
  QS_TR(10);
  if (arrive_last(c, (u32)a.G, sc)) reset_row(a, row);
  QS_TR(15);
  }
#undef QS_FOR_ELEMS
}

// ---------------------------------------------------------------- probabilities

template <int DT>
__global__ __launch_bounds__(kThreads) void k_probs(Args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ Scratch sc;
  const int row = blockIdx.y, blk = blockIdx.x;
  const int start = blk * a.CH, end = min(a.V, start + a.CH);
  RowCtl* c = a.ctl + row;
  const RowParams p = row_params(a, row);
  PenTable pt;
  pt.bits = (u32*)lds;
  pt.wpre = pt.bits + (a.CH >> 5);
  pt.cnts = pt.wpre + (a.CH >> 5);
  if (p.pen_on && !p.greedy) pen_build(a, row, start, end, pt, sc);
  const long long chosen = c->chosen;
  u32 kept = 0;
  if (c->greedy) {
    for (int i = start + threadIdx.x; i < end; i += kThreads) {
      a.out_probs[(size_t)row * a.V + i] = (i == chosen) ? 1.0f : 0.0f;
      kept += (i == chosen);
    }
  } else {
    const int N = c->n_max;
    const u128 W = mk128(c->w_lo, c->w_hi);
    const double Wd = u128_to_double(W);
    const u32 kp = c->kappa_p, idp = c->id_p;
    for (int i = start + threadIdx.x; i < end; i += kThreads) {
      float z = load_logit<DT>(a, row, i);
      if (p.pen_on) {
        const u32 cnt = pen_count(pt, i - start);
        if (cnt) z = apply_penalty(z, cnt, p.rep, p.pres, p.freq);
      }
      const float q = z / p.T;
      const u32 k = skey(q);
      float pr = 0.0f;
      if (k > kp || (k == kp && (u32)i <= idp)) {
        const u64 w = weight_of(q, N);
        pr = (float)((double)w / Wd);
        kept += (w != 0ull);
      }
      a.out_probs[(size_t)row * a.V + i] = pr;
    }
  }
  for (int o = 32; o > 0; o >>= 1) kept += __shfl_xor(kept, o, 64);
  if ((threadIdx.x & 63) == 0 && kept) addc(&c->probs_kept, kept);
  wait_mem();
  __syncthreads();
  if (threadIdx.x == 0) sc.r[7] = (addc(&c->probs_arrive, 1u) == (u32)a.G - 1u) ? 1u : 0u;
  __syncthreads();
  if (!sc.r[7]) return;
  if (threadIdx.x == 0) {
    if (a.out_kept) a.out_kept[row] = (int)addc(&c->probs_kept, 0u);
    stc(&c->probs_kept, 0u);
    stc(&c->probs_arrive, 0u);
  }
}

__global__ void k_zero(u32* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// ---------------------------------------------------------------- host side

thread_local char g_err[512] = "";

int fail(const char* fmt, const char* detail = "") {
  snprintf(g_err, sizeof(g_err), fmt, detail);
  return -1;
}

struct Layout {
  int EPT, CH, G, seg_cap, Hpad;
  size_t off_ctl, off_cand, off_hist, off_brk, off_slots, total;
  size_t lds;
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Elements per thread: 32 once the batch has enough chunks to fill the chip,
// else 16 (shorter chunks, more workgroups per row).
int pick_ept(int B, int V) {
  const int g32 = (V + kThreads * 32 - 1) / (kThreads * 32);
  if ((long long)B * g32 >= 512) return 32;
  return 16;
}

Layout layout_for(int B, int V, int H) {
  Layout L;
  L.EPT = pick_ept(B, V);
  L.CH = kThreads * L.EPT;
  L.G = (V + L.CH - 1) / L.CH;
  L.seg_cap = H > 0 ? (H < L.CH ? H : L.CH) : 0;
  L.Hpad = 1;
  while (L.Hpad < H) L.Hpad <<= 1;
  size_t o = 0;
  L.off_ctl = o;
  o = align_up(o + (size_t)B * sizeof(RowCtl), 256);
  L.off_cand = o;
  o = align_up(o + (size_t)B * L.G * kBlockCand * 8, 256);
  L.off_hist = o;
  o = align_up(o + (size_t)B * 2 * kBins * 8, 256);
  L.off_brk = o;
  o = align_up(o + (size_t)B * kBracketCap * 8, 256);
  L.off_slots = o;
  o = align_up(o + (size_t)B * L.G * sizeof(Slot), 256);
  L.total = o;
  const size_t pen = H > 0 ? (size_t)(2 * (L.CH / 32) + L.seg_cap) * 4 : 0;
  const size_t merge = (size_t)kMergeCap * 8 + (size_t)kMaxChunks * 4 + sizeof(SelLds);
  const size_t single = sizeof(SingleLds) + (H > 0 ? (size_t)L.Hpad * 4 : 0);
  const size_t mass = sizeof(MassLds);
  L.lds = pen;
  if (merge > L.lds) L.lds = merge;
  if (single > L.lds) L.lds = single;
  if (mass > L.lds) L.lds = mass;
  return L;
}

template <int DT, int EPT, int ROLE>
hipError_t launch_sample(const Args& a, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((k_sample<DT, EPT, ROLE>), dim3(a.G, a.B), dim3(kThreads), lds, st, a);
  return hipGetLastError();
}

template <int DT, int ROLE>
hipError_t launch_dt(const Args& a, int ept, size_t lds, hipStream_t st) {
  if (ept == 32) return launch_sample<DT, 32, ROLE>(a, lds, st);
  return launch_sample<DT, 16, ROLE>(a, lds, st);
}

#ifdef QS_TRACE
u64* g_trace = nullptr;
#endif

// Per-device side stream (default priority) and fork/join events for the
// mass-row launch.  Created by qs_workspace_init, outside any graph capture.
struct SideStream {
  hipStream_t stream;
  hipEvent_t fork, join;
};
constexpr int kMaxDevices = 64;
SideStream g_side[kMaxDevices];
bool g_side_ok[kMaxDevices];

SideStream* side_stream() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  return g_side_ok[dev] ? &g_side[dev] : nullptr;
}

int init_side_stream() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
  if (g_side_ok[dev]) return 0;
  SideStream& sd = g_side[dev];
  if (hipStreamCreateWithFlags(&sd.stream, hipStreamNonBlocking) != hipSuccess) return -1;
  if (hipEventCreateWithFlags(&sd.fork, hipEventDisableTiming) != hipSuccess) return -1;
  if (hipEventCreateWithFlags(&sd.join, hipEventDisableTiming) != hipSuccess) return -1;
  g_side_ok[dev] = true;
  return 0;
}

int run(const void* logits, int64_t row_stride, int dtype, int B, int V, const float* temperature,
        const float* top_p, const int32_t* top_k, const float* rep, const float* pres, const float* freq,
        const int32_t* hist, int H, const float* uniforms, uint32_t flags, int64_t* out_ids, float* out_probs,
        int32_t* out_kept, void* ws, size_t ws_bytes, hipStream_t stream) {
  g_err[0] = 0;
  if (dtype != QS_DTYPE_F32 && dtype != QS_DTYPE_BF16) return fail("qs_sample: unknown logits dtype%s");
  if (B < 0 || V <= 0 || V >= (1 << 28)) return fail("qs_sample: bad shape (B >= 0, 0 < V < 2^28)%s");
  if (B > 65535) return fail("qs_sample: B above 65535%s");
  if (B == 0) return 0;
  if (row_stride < V) return fail("qs_sample: row_stride < V%s");
  if (!logits || !out_ids || !ws) return fail("qs_sample: null logits, out_ids or workspace%s");
  if (!(flags & QS_FLAG_ALL_GREEDY) && !temperature) return fail("qs_sample: temperature required%s");
  if (H < 0 || (H > 0 && !hist)) return fail("qs_sample: bad history arguments%s");
  if (H > kMaxHistory) return fail("qs_sample: history longer than QS_MAX_HISTORY%s");
  if (out_kept && !out_probs) return fail("qs_sample: out_kept requires out_probs%s");
  const int Heff = hist ? H : 0;
  const Layout L = layout_for(B, V, Heff);
  if (ws_bytes < L.total) return fail("qs_sample: workspace too small (see qs_workspace_bytes)%s");
  if (((uintptr_t)ws) % 256) return fail("qs_sample: workspace must be 256-byte aligned%s");
  const bool all_greedy = (flags & QS_FLAG_ALL_GREEDY) != 0;
  if (!all_greedy && !uniforms) return fail("qs_sample: uniforms required unless all rows are greedy%s");
  if (L.G > kMaxChunks) return fail("qs_sample: V too large for the chunking%s");
  if (L.lds > 64 * 1024) return fail("qs_sample: LDS budget exceeded%s");

  Args a;
  memset(&a, 0, sizeof(a));
  a.logits = logits;
  a.row_stride = row_stride;
  a.B = B;
  a.V = V;
  a.H = Heff;
  a.G = L.G;
  a.CH = L.CH;
  a.seg_cap = L.seg_cap;
  a.Hpad = L.Hpad;
  a.flags = flags;
  a.temperature = temperature;
  a.top_p = top_p;
  a.top_k = top_k;
  a.rep = rep;
  a.pres = pres;
  a.freq = freq;
  a.hist = Heff ? hist : nullptr;
  a.uniforms = uniforms;
  a.out_ids = (long long*)out_ids;
  a.out_probs = out_probs;
  a.out_kept = out_kept;
  char* base = (char*)ws;
  a.ctl = (RowCtl*)(base + L.off_ctl);
  a.cand = (u64*)(base + L.off_cand);
  a.mhist = (u64*)(base + L.off_hist);
  a.brk = (u64*)(base + L.off_brk);
  a.slots = (Slot*)(base + L.off_slots);
#ifdef QS_TRACE
  a.trace = g_trace;
#endif

  const bool mass = !(flags & (QS_FLAG_ALL_GREEDY | QS_FLAG_NO_MASS_ROWS));
  SideStream* side = nullptr;
  hipError_t e;
  if (mass) {
    // the mass-row launch runs beside the other rows' launch: fork and join
    // through events on a side stream (capturable into a HIP graph)
    side = side_stream();
    if (!side) return fail("qs_sample: no side stream (call qs_workspace_init first)%s");
    e = hipEventRecord(side->fork, stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(side->stream, side->fork, 0);
    if (e != hipSuccess) return fail("qs_sample: fork failed: %s", hipGetErrorString(e));
  }
  e = dtype == QS_DTYPE_F32 ? launch_dt<QS_DTYPE_F32, 0>(a, L.EPT, L.lds, stream)
                            : launch_dt<QS_DTYPE_BF16, 0>(a, L.EPT, L.lds, stream);
  if (e != hipSuccess) return fail("qs_sample: kernel launch failed: %s", hipGetErrorString(e));
  if (mass) {
    e = dtype == QS_DTYPE_F32 ? launch_dt<QS_DTYPE_F32, 1>(a, L.EPT, L.lds, side->stream)
                              : launch_dt<QS_DTYPE_BF16, 1>(a, L.EPT, L.lds, side->stream);
    if (e != hipSuccess) return fail("qs_sample: mass kernel launch failed: %s", hipGetErrorString(e));
    e = hipEventRecord(side->join, side->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(stream, side->join, 0);
    if (e != hipSuccess) return fail("qs_sample: join failed: %s", hipGetErrorString(e));
  }
  if (out_probs) {
    const size_t plds = Heff > 0 ? (size_t)(2 * (L.CH / 32) + L.seg_cap) * 4 : 16;
    if (dtype == QS_DTYPE_F32)
      hipLaunchKernelGGL(k_probs<QS_DTYPE_F32>, dim3(a.G, B), dim3(kThreads), plds, stream, a);
    else
      hipLaunchKernelGGL(k_probs<QS_DTYPE_BF16>, dim3(a.G, B), dim3(kThreads), plds, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return fail("qs_sample: probs kernel launch failed: %s", hipGetErrorString(e));
  }
  return 0;
}

}  // namespace

extern "C" {

int qs_version(void) { return 200; }

#ifdef QS_TRACE
// Trace builds only: device buffer of [B, G, 16] u64 wall-clock stamps.
void qs_debug_set_trace(void* buf) { g_trace = (u64*)buf; }
#endif

const char* qs_last_error(void) { return g_err; }

size_t qs_workspace_bytes(int B, int V, int logits_dtype, int H) {
  (void)logits_dtype;
  if (B <= 0 || V <= 0) return 256;
  return layout_for(B, V, H > 0 ? H : 0).total;
}

int qs_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream) {
  g_err[0] = 0;
  if (!workspace) return fail("qs_workspace_init: null workspace%s");
  if (init_side_stream() != 0) return fail("qs_workspace_init: cannot create the side stream%s");
  const size_t n = workspace_bytes / 4;
  hipLaunchKernelGGL(k_zero, dim3(1024), dim3(256), 0, stream, (u32*)workspace, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("qs_workspace_init: %s", hipGetErrorString(e));
  return 0;
}

int qs_sample(const void* logits, int64_t row_stride, int logits_dtype, int B, int V, const float* temperature,
              const float* top_p, const int32_t* top_k, const float* rep_pen, const float* pres_pen,
              const float* freq_pen, const int32_t* hist_ids, int H, const float* uniforms, uint32_t flags,
              int64_t* out_ids, float* out_probs, int32_t* out_kept, void* workspace, size_t workspace_bytes,
              hipStream_t stream) {
  return run(logits, row_stride, logits_dtype, B, V, temperature, top_p, top_k, rep_pen, pres_pen, freq_pen,
             hist_ids, H, uniforms, flags, out_ids, out_probs, out_kept, workspace, workspace_bytes, stream);
}

int qs_argmax(const void* logits, int64_t row_stride, int logits_dtype, int B, int V, int64_t* out_ids,
              void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return run(logits, row_stride, logits_dtype, B, V, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
             nullptr, 0, nullptr, QS_FLAG_ALL_GREEDY, out_ids, nullptr, nullptr, workspace, workspace_bytes,
             stream);
}

}  // extern "C"
