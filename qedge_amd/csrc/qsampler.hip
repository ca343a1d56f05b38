// qsampler: decode-step token sampler for MI355X (gfx950).
//
// Replaces BatchSampler.forward (src/compute/sampler.py:25-41) behind the
// ModelRunner._sample_gpu call site (src/compute/model_runner.py:77-93) and the
// greedy argmax sites (src/compute/model_runner.py:85,353).  The arithmetic
// contract is stated in include/qsampler.h; ids are exact integers.
//
// Grid (G chunks, B rows), 256 threads (4 waves of 64); each workgroup streams
// one chunk of 8192 logits of a row into registers once (16-byte loads) and
// applies the history penalties from an LDS table.  Two launches run side by
// side (the second on a side stream):
//   main launch  greedy rows: local argmax, one 64-bit atomic max per
//                workgroup, the last workgroup to arrive publishes the id.
//                top-k rows (0 < k <= QS_TOPK_FAST_MAX): every workgroup
//                writes the tokens at or above a threshold taken from its
//                per-thread maxima, in id order, to its own region; the last
//                workgroup gathers the regions into registers (eight tokens per
//                thread, still in id order) and resolves top-k, top-p and the
//                draw with register radix selects over 256-bin LDS histograms.
//   mass launch  rows with top-k off.  Every workgroup writes the tokens
//                within 40 octaves of its own maximum; one row barrier
//                exchanges the row maximum and the counts.  A peaked row (few
//                such tokens) is then resolved by one workgroup like a top-k
//                row.  A flat row stays cooperative: exact weights, per-bin
//                masses, a second row barrier for the global histogram and the
//                total mass, the bracket of bins holding the top-p boundary,
//                the bracketed tokens listed; the last workgroup to arrive
//                resolves the boundary exactly, finds the chunk holding the
//                draw and re-reads that chunk to locate the token in id order.
//   fallback     a single workgroup resolves the row exactly from global
//                memory (large k, a candidate overflow, an incomplete
//                candidate set, a bracket overflow).  Slow, rare on real logits.
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
constexpr int kEPT = 32;                          // logits per thread
constexpr int kCH = kThreads * kEPT;              // logits per chunk (workgroup)
constexpr int kWindow = 40;
constexpr double kYClamp = 1073741824.0;  // 2^30
constexpr double kLog2e = 1.4426950408889634074;
constexpr int kTopkFast = QS_TOPK_FAST_MAX;
constexpr int kGatherPer = 16;                    // region entries one finishing thread loads
constexpr int kRegionTotal = 8192;                // G * R <= this (the entries written stay <= kThreads * kGatherPer)
constexpr int kStageCap = 1024;
constexpr int kHoffBytes = 2048;                  // finish_row: region offsets ahead of the histogram                   // region entries staged in LDS by one workgroup
constexpr int kFinPer = 16;                       // merged candidates per thread
constexpr int kFinCap = kThreads * kFinPer;       // merged candidates per row
constexpr int kBins = 256;                        // histogram bins
constexpr int kWideBits = 11;                     // finishing histogram: 2048 bins
constexpr int kWide = 1 << kWideBits;
constexpr int kWidePer = kWide / kThreads;        // bins per thread
constexpr int kListCap = kFinCap;                 // bracket entries per row (flat mass rows)
constexpr int kHash = 1024;
constexpr int kStage2 = 2048;                      // bracketed tokens staged per chunk (flat mass rows)
constexpr int kSegEnt = 512;                      // (key, segment) entries per chunk (flat mass rows)
constexpr int kSegs = 32;                          // segments per chunk (vector x wave), at most                       // bracketed tokens per chunk (flat mass rows)
constexpr int kMaxChunks = 256;                   // chunks per row (G)
constexpr int kMaxHistory = QS_MAX_HISTORY;
constexpr u32 kSpinLimit = 1u << 21;

enum : u32 { kStFallback = 1u, kStTimeout = 2u, kStOverflow = 4u, kStList = 8u };
// Reasons for a fallback to resolve_single, recorded in RowCtl::why.
enum : u32 {
  kWhyRegion = 1u,      // a workgroup's region overflowed
  kWhyMerge = 2u,       // more merged candidates than kFinCap
  kWhyFewer = 3u,       // fewer merged candidates than k
  kWhyKSelect = 4u,     // the k-select found no value
  kWhyIncomplete = 5u,  // a token left out could be in the top-k set
  kWhyTopP = 6u,        // the top-p select found no value
  kWhyList = 11u,       // flat row: more bracketed tokens than kListCap
  kWhyAbove = 12u,      // flat row: mass above the bracket exceeds the target
  kWhyBracket = 13u,    // flat row: the boundary is not inside the bracket
  kWhyTie = 14u,        // flat row: the tie select found no value
  kWhyOwner = 15u,      // flat row: no chunk holds the draw target
  kWhyTimeout = 16u,    // a row barrier gave up waiting
  kWhyLargeK = 17u,     // top_k above QS_TOPK_FAST_MAX
};

// Per-row control block.  The first 64 bytes are counters that every call
// leaves at zero; the rest holds the last call's result for k_probs.
struct __attribute__((aligned(256))) RowCtl {
  u64 pack;        // greedy: max of (gkey << 32 | ~id)
  u32 arrive;      // workgroups done
  u32 bar;         // row barrier counter
  u32 kmax;        // mass rows: max key(q)
  u32 nkmin;       // mass rows: ~min key(q) over non-NaN tokens
  u32 status;      // kSt* flags
  u32 cand_n;      // mass rows: tokens written to the regions
  u32 list_n;      // mass rows: bracketed tokens listed
  u32 probs_arrive;
  u32 probs_kept;
  u32 pad0[5];
  long long chosen;
  u64 w_lo, w_hi;  // kept mass W
  u64 tp_lo, tp_hi;  // flat mass rows: floor(top_p * S)
  int n_max;       // row scale N
  u32 kappa_p, id_p;  // kept iff key > kappa_p || (key == kappa_p && id <= id_p)
  u32 greedy;
  u32 path;        // 0 greedy, 1 top-k, 2 flat mass row, 3 single workgroup, 4 peaked mass row
  u32 flat_blo;    // flat mass rows: lowest bin of the bracket
  u32 why;         // why the last fallback to resolve_single was taken (kWhy*), 0 if none
  u32 pad1[31];
};
static_assert(sizeof(RowCtl) == 256, "row control block is 256 bytes");
constexpr int kCtlZeroWords = 16;

// Per-(row, workgroup) published values.
struct __attribute__((aligned(64))) Slot {
  u64 s_lo, s_hi;  // mass rows: exact mass of the chunk
  u64 a_lo, a_hi;  // flat mass rows: exact mass of the chunk's tokens above the bracket
  u32 nb;          // tokens written to the region (0xffffffff: more than fit)
  u32 tau;         // top-k rows: the region's threshold (z key)
  u32 below;       // top-k rows: largest z key below tau in the chunk
  u32 nbr;         // flat mass rows: bracketed tokens of the chunk
  u32 nse;         // flat mass rows: (key, segment) entries of the chunk (0xffffffff: more than fit)
  u32 pad[3];
};
static_assert(sizeof(Slot) == 64, "slot is 64 bytes");

struct Args {
  const void* logits;
  long long row_stride;
  int B, V, H, G, R, logR, seg_cap, Hpad;
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
  uint4* cand; // [B, G, R] region entries {id, q key, exp2 mantissa M, octave n}
  u64* mhist;  // [B, kBins] global mass histogram (flat mass rows)
  u64* list;   // [B, kListCap] bracket entries (key << 32 | chunk << 16 | count), flat mass rows
  u64* sent;   // [B, G, kSegEnt] per chunk: bracket entries (key << 32 | segment << 16 | count), flat mass rows
  u64* segm;   // [B, G, kSegs, 2] flat mass rows: exact mass per segment (above the bracket with top-p), lo, hi
  Slot* slots; // [B, G]
  u64* trace;  // per-workgroup phase timestamps (trace builds only)
};

#ifdef QS_TRACE
#define QS_TR(i)                                                             \
  do {                                                                       \
    if (a.trace && threadIdx.x == 0) a.trace[(size_t)sc.tslot * 16 + (i)] = wall_clock64(); \
  } while (0)
#else
#define QS_TR(i) \
  do {           \
  } while (0)
#endif

// ---------------------------------------------------------------- memory model

// Workgroup barrier for LDS traffic only: outstanding global loads stay in flight.
__device__ __forceinline__ void lds_sync() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt left at their maxima
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
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
// The weight packed in 32 bits: (n - N + 40) << 24 | M, 0 for weight 0.
__device__ __forceinline__ u32 wpack_y(double y, int N) {
  const double fl = floor(y);
  const int n = (int)fl;
  if (n < N - kWindow) return 0u;
  return ((u32)(n - N + kWindow) << 24) | mant24(exp2_poly((float)(y - fl)));
}
__device__ __forceinline__ u32 wpack(float q, int N) { return wpack_y(y_of(q), N); }
__device__ __forceinline__ u64 wunpack(u32 wp) { return wp ? (u64)(wp & 0xffffffu) << (wp >> 24) : 0ull; }
// Smallest non-NaN key whose octave floor(y) is at least n0 (keys at or above
// it are exactly the tokens inside a window that starts at octave n0).
__device__ __forceinline__ u32 window_key(int n0) {
  if ((double)n0 <= -kYClamp) return 1u;
  if ((double)n0 > kYClamp) return 0xffffffffu;
  u32 k = skey((float)((double)n0 / kLog2e));
  if (k == 0u) k = 1u;
  for (int it = 0; it < 64 && k > 1u && floor(y_of(f_of_key(k - 1u))) >= (double)n0; ++it) --k;
  for (int it = 0; it < 64 && k < 0xffffffffu && floor(y_of(f_of_key(k))) < (double)n0; ++it) ++k;
  return k;
}
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
// Values the same in every lane, moved to scalar registers.
__device__ __forceinline__ u32 uni(u32 v) { return (u32)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ u64 uni64(u64 v) { return ((u64)uni((u32)(v >> 32)) << 32) | uni((u32)v); }
__device__ __forceinline__ u128 uni128(u128 v) { return mk128(uni64((u64)v), uni64((u64)(v >> 64))); }
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
  u64 w[20];              // [12, 15]: find_bin results; [8, 20): select results
  u64 fw[12];             // wide_find results: [0, 6) slot 0, [6, 12) slot 1
  u32 u[8];               // finish_row: key range of a bin
  u32 v[kWaves][8];       // per-wave partials of the block collectives
  int i[8];               // find_bin
  u32 r[16];              // results and counters of the callers
  u32 tslot;              // trace builds: this workgroup's row of time stamps
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
// Sum over the wave, returned to every lane.
__device__ __forceinline__ u32 wave_sum(u32 v) { return (u32)__builtin_amdgcn_readlane((int)wave_incl_scan(v), 63); }
// Exact sum over the wave of lo + hi * 2^64 (hi < 2^22), in 22-bit limbs.
__device__ __forceinline__ u128 wave_sum128(u64 lo, u32 hi) {
  const u32 l0 = wave_sum((u32)lo & 0x3fffffu);
  const u32 l1 = wave_sum((u32)(lo >> 22) & 0x3fffffu);
  const u32 l2 = wave_sum((u32)(lo >> 44));
  const u32 l3 = wave_sum(hi);
  return (u128)l0 + ((u128)l1 << 22) + ((u128)l2 << 44) + ((u128)l3 << 64);
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

// Exclusive scan of v in thread order (total in *total) and the maxima of
// x[0..NX) over the workgroup (returned in x): one LDS exchange.
template <int NX>
__device__ __forceinline__ u32 block_scan_max(u32 v, u32 (&x)[NX], Scratch& s, u32* total) {
  static_assert(NX <= 7, "per-wave slots");
  const int wv = threadIdx.x >> 6;
  const u32 inc = wave_incl_scan(v);
  u32 mx[NX];
#pragma unroll
  for (int i = 0; i < NX; ++i) mx[i] = wave_max(x[i]);
  if (lane_id() == 63) s.v[wv][0] = inc;
  if (lane_id() == 0) {
#pragma unroll
    for (int i = 0; i < NX; ++i) s.v[wv][1 + i] = mx[i];
  }
  __syncthreads();
  u32 base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < NX; ++i) x[i] = 0u;
  for (int w = 0; w < kWaves; ++w) {
    const u32 c = s.v[w][0];
    base += (w < wv) ? c : 0u;
    tot += c;
#pragma unroll
    for (int i = 0; i < NX; ++i) x[i] = s.v[w][1 + i] > x[i] ? s.v[w][1 + i] : x[i];
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

// Maxima of up to three u32 over the workgroup, one LDS exchange.
__device__ __forceinline__ void block_max3(u32& a0, u32& a1, u32& a2, Scratch& s) {
  a0 = wave_max(a0);
  a1 = wave_max(a1);
  a2 = wave_max(a2);
  const int wv = threadIdx.x >> 6;
  if (lane_id() == 0) {
    s.v[wv][0] = a0;
    s.v[wv][1] = a1;
    s.v[wv][2] = a2;
  }
  __syncthreads();
  u32 r0 = 0, r1 = 0, r2 = 0;
  for (int i = 0; i < kWaves; ++i) {
    r0 = s.v[i][0] > r0 ? s.v[i][0] : r0;
    r1 = s.v[i][1] > r1 ? s.v[i][1] : r1;
    r2 = s.v[i][2] > r2 ? s.v[i][2] : r2;
  }
  __syncthreads();
  a0 = r0;
  a1 = r1;
  a2 = r2;
}

// ---------------------------------------------------------------- register radix select

struct SelLds {  // one 8-bit digit level of a radix select
  u32 cnt[256];
  u64 mlo[256];  // sums of the low 32 bits of the weights
  u64 mhi[256];  // sums of the high 32 bits
};

struct WideLds {  // the finishing histogram: count and mass per bin
  u32 cnt[kWide];
  u64 mlo[kWide];
  u64 mhi[kWide];
};

__device__ __forceinline__ Acc wide_bin(const WideLds& W, int b) {
  return acc_of(mk128(W.mlo[b], 0) + ((u128)W.mhi[b] << 32), W.cnt[b]);
}

// Thread t holds the kWidePer bins kWide - 1 - (t * kWidePer + i), i.e. the
// bins in descending order: bin[i] their (count, mass), `ex` the sum of all
// bins before its first.  The bin where the running count (or, by_mass, mass)
// first exceeds `target`: *bin (-1 if none), *before the (count, mass) of the
// bins before it, *at its own.  Result slot `slot` (0 or 1): the caller has set
// sc.i[1 + slot] = -1 before a barrier that every thread has passed since.
// All threads call it.
__device__ __forceinline__ void wide_find(const Acc (&bin)[kWidePer], Acc ex, bool by_mass, u128 target, Scratch& sc,
                                          int slot, int* bout, Acc* before, Acc* at) {
  const int tid = threadIdx.x;
  Acc run = ex;
  bool found = false;
#pragma unroll
  for (int i = 0; i < kWidePer; ++i) {
    const Acc x = bin[i];
    const u128 lo = by_mass ? acc_mass(run) : (u128)run.c;
    const u128 sz = by_mass ? acc_mass(x) : (u128)x.c;
    if (!found && sz > 0 && target >= lo && target < lo + sz) {
      found = true;
      sc.i[1 + slot] = kWide - 1 - (tid * kWidePer + i);
      u64* f = sc.fw + 6 * slot;
      f[0] = run.lo;
      f[1] = run.hi;
      f[2] = run.c;
      f[3] = x.lo;
      f[4] = x.hi;
      f[5] = x.c;
    }
    run = acc_add(run, x);
  }
  __syncthreads();
  const u64* f = sc.fw + 6 * slot;
  *bout = sc.i[1 + slot];
  *before = Acc{uni64(f[0]), uni64(f[1]), uni((u32)f[2])};
  *at = Acc{uni64(f[3]), uni64(f[4]), uni((u32)f[5])};
}

struct SelOut {
  u32 val;      // the selected 32-bit value
  Acc before;   // members ordered before it (count, mass)
  Acc at;       // members equal to it
  bool ok;      // false if the target is not below the members' total
};

// Over the members (bit j of memb) of every thread's E values val[j], ordered
// by value descending, the value at which the running count (or, BY_MASS, the
// running weight wunpack(wp[j])) first exceeds `target`.  With CNT, member j
// stands for mult[j] tokens of that value.  8-bit digits from the highest bit
// where members differ; the histogram alternates between the two buffers
// L[0], L[1].  All threads call it.
template <bool BY_MASS, int E, bool CNT = false>
__device__ __forceinline__ SelOut reg_select(const u32 (&val)[E], u32 memb, const u32 (&wp)[E], u128 target,
                                             SelLds* L, Scratch& sc, const u32* mult = nullptr) {
  static_assert(kThreads == 256, "one digit bin per thread");
  const int tid = threadIdx.x;
  u32 mx = 0u, nmn = 0u, any = memb ? 1u : 0u;
#pragma unroll
  for (int j = 0; j < E; ++j) {
    if ((memb >> j) & 1u) {
      mx = val[j] > mx ? val[j] : mx;
      nmn = ~val[j] > nmn ? ~val[j] : nmn;
    }
  }
  block_max3(mx, nmn, any, sc);
  mx = uni(mx);
  nmn = uni(nmn);
  any = uni(any);
  target = uni128(target);
  SelOut out;
  out.before = Acc{0, 0, 0};
  out.at = Acc{0, 0, 0};
  out.val = ~nmn;
  out.ok = any != 0u;
  if (!any) return out;
  const u32 first = ~nmn, diff = mx ^ first;
  if (diff == 0u) {
    // one value: every member is at it
    Acc loc = {0, 0, 0};
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const u32 n = CNT ? mult[j] : 1u;
      if ((memb >> j) & 1u) loc = acc_add(loc, acc_of(BY_MASS ? (u128)wunpack(wp[j]) * n : (u128)0, n));
    }
    out.at = block_sum_acc(loc, sc);
    const u128 sz = BY_MASS ? acc_mass(out.at) : (u128)out.at.c;
    out.ok = target < sz;
    return out;
  }
  int top = 31;
  while (!((diff >> top) & 1u)) --top;
  u32 prefix = (top == 31) ? 0u : (first & ~((2u << top) - 1u));
  u32 mask = (top == 31) ? 0u : ~((2u << top) - 1u);
  int hi = top;
  for (int lv = 0;; ++lv) {
    SelLds& H = L[lv & 1];
    const int lo = hi >= 7 ? hi - 7 : 0;
    const u32 dmask = (1u << (hi - lo + 1)) - 1u;
    H.cnt[tid] = 0u;
    if (BY_MASS) {
      H.mlo[tid] = 0ull;
      H.mhi[tid] = 0ull;
    }
    // result slots alternate with the level, so no barrier is needed between
    // one level's reads and the next level's writes
    const int rs = 2 * (lv & 1), ws = 8 + 6 * (lv & 1);
    if (tid == 0) sc.r[rs] = 0xffffffffu;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if (((memb >> j) & 1u) && (val[j] & mask) == prefix) {
        const u32 d = (val[j] >> lo) & dmask;
        const u32 n = CNT ? mult[j] : 1u;
        atomicAdd(&H.cnt[d], n);
        if (BY_MASS) {
          // unpacked here, not hoisted out of the level loop (registers)
          u32 wj = wp[j];
          asm volatile("" : "+v"(wj));
          const u64 w = wunpack(wj);
          if (w) {
            atomicAdd(&H.mlo[d], (w & 0xffffffffull) * n);
            atomicAdd(&H.mhi[d], (w >> 32) * n);
          }
        }
      }
    }
    __syncthreads();
    // scan the bins from the top: thread t takes bin 255 - t
    const int b = 255 - tid;
    const bool live = b <= (int)dmask;
    Acc mine = {0, 0, 0};
    if (live) {
      mine.c = H.cnt[b];
      if (BY_MASS) mine = acc_of(mk128(H.mlo[b], 0) + ((u128)H.mhi[b] << 32), H.cnt[b]);
    }
    Acc ex;
    if (BY_MASS) {
      Acc tot;
      ex = block_scan_acc(mine, sc, &tot);
    } else {
      u32 tot;
      ex = acc_of(0, block_scan_u32(mine.c, sc, &tot));
    }
    const u128 lo_m = BY_MASS ? acc_mass(ex) : (u128)ex.c;
    const u128 sz = BY_MASS ? acc_mass(mine) : (u128)mine.c;
    if (live && sz > 0 && target >= lo_m && target < lo_m + sz) {
      sc.r[rs] = (u32)b;
      sc.r[rs + 1] = mine.c;
      sc.w[ws] = ex.lo;
      sc.w[ws + 1] = ex.hi;
      sc.w[ws + 2] = ex.c;
      sc.w[ws + 3] = mine.lo;
      sc.w[ws + 4] = mine.hi;
    }
    __syncthreads();
    const u32 d = uni(sc.r[rs]);
    const u32 dcnt = uni(sc.r[rs + 1]);
    const Acc bex = {uni64(sc.w[ws]), uni64(sc.w[ws + 1]), uni((u32)sc.w[ws + 2])};
    const Acc bat = {uni64(sc.w[ws + 3]), uni64(sc.w[ws + 4]), dcnt};
    if (d == 0xffffffffu) {
      __syncthreads();
      out.ok = false;
      return out;
    }
    out.before = acc_add(out.before, bex);
    target -= BY_MASS ? acc_mass(bex) : (u128)bex.c;
    prefix |= d << lo;
    mask |= dmask << lo;
    if (lo == 0) {
      out.at = bat;
      __syncthreads();
      break;
    }
    if (dcnt == 1u) {
      // a single member left: its value
      __syncthreads();
#pragma unroll
      for (int j = 0; j < E; ++j)
        if (((memb >> j) & 1u) && (val[j] & mask) == prefix) sc.r[4] = val[j];
      __syncthreads();
      prefix = uni(sc.r[4]);
      out.at = bat;
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

// Called by the last workgroup of the row: counters (and the row's mass
// histogram, if it was used) to zero.
__device__ __forceinline__ void reset_row(const Args& a, int row, bool hist = false) {
  u32* w = (u32*)(a.ctl + row);
  if (threadIdx.x < kCtlZeroWords) stc(&w[threadIdx.x], 0u);
  if (hist) {
    u64* h = a.mhist + (size_t)row * kBins;
    for (int i = threadIdx.x; i < kBins; i += kThreads) stc(&h[i], 0ull);
  }
}

__device__ __forceinline__ bool give_up(const Args& a, int row, u32 why) {
  if (threadIdx.x == 0) a.ctl[row].why = why;
  return false;
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
  constexpr int kB = 8;                 // history ids per thread and batch
  constexpr int kBatch = kB * kThreads;
  const int nw = kCH >> 5;
  for (int i = threadIdx.x; i < nw; i += kThreads) t.bits[i] = 0u;
  for (int i = threadIdx.x; i < a.seg_cap; i += kThreads) t.cnts[i] = 0u;
  // the row's history ids in this chunk, chunk-relative (-1 otherwise); the
  // first batch stays in registers for the counting pass
  const int* h = a.hist + (size_t)row * a.H;
  int loc[kB];
#pragma unroll
  for (int q = 0; q < kB; ++q) {
    const int i = q * kThreads + threadIdx.x;
    loc[q] = i < a.H ? h[i] : -1;
  }
#pragma unroll
  for (int q = 0; q < kB; ++q) loc[q] = (loc[q] >= start && loc[q] < end) ? loc[q] - start : -1;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kB; ++q)
    if (loc[q] >= 0) atomicOr(&t.bits[loc[q] >> 5], 1u << (loc[q] & 31));
  for (int b0 = kBatch; b0 < a.H; b0 += kBatch) {
    int l2[kB];
#pragma unroll
    for (int q = 0; q < kB; ++q) {
      const int i = b0 + q * kThreads + threadIdx.x;
      l2[q] = i < a.H ? h[i] : -1;
    }
#pragma unroll
    for (int q = 0; q < kB; ++q)
      if (l2[q] >= start && l2[q] < end) atomicOr(&t.bits[(l2[q] - start) >> 5], 1u << ((l2[q] - start) & 31));
  }
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
  for (int q = 0; q < kB; ++q) {
    const int l = loc[q];
    if (l >= 0) {
      const u32 bw = t.bits[l >> 5];
      atomicAdd(&t.cnts[t.wpre[l >> 5] + __popc(bw & ((1u << (l & 31)) - 1u))], 1u);
    }
  }
  for (int b0 = kBatch; b0 < a.H; b0 += kBatch) {
    int l2[kB];
#pragma unroll
    for (int q = 0; q < kB; ++q) {
      const int i = b0 + q * kThreads + threadIdx.x;
      l2[q] = i < a.H ? h[i] : -1;
    }
#pragma unroll
    for (int q = 0; q < kB; ++q) {
      if (l2[q] >= start && l2[q] < end) {
        const int l = l2[q] - start;
        const u32 bw = t.bits[l >> 5];
        atomicAdd(&t.cnts[t.wpre[l >> 5] + __popc(bw & ((1u << (l & 31)) - 1u))], 1u);
      }
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

// ---------------------------------------------------------------- chunk loads

// The chunk's logits, 16-byte vectors: thread t holds, for v < NV, the VW
// logits from start + (v * 256 + t) * VW.  Loads are issued here and consumed
// by unpack_chunk, so they stay in flight across the penalty table's build.
template <int DT>
struct ChunkLoad {
  static constexpr int VW = (DT == QS_DTYPE_F32) ? 4 : 8;
  static constexpr int NV = kEPT / VW;
  static constexpr int ESZ = (DT == QS_DTYPE_F32) ? 4 : 2;
  uint4 raw[NV];
  bool vec;
};

template <int DT>
__device__ __forceinline__ void issue_chunk(const Args& a, int row, int start, int end, ChunkLoad<DT>& L) {
  using CL = ChunkLoad<DT>;
  const char* rp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * CL::ESZ;
  L.vec = ((((uintptr_t)a.logits) | ((size_t)a.row_stride * CL::ESZ)) & 15) == 0;
  if (L.vec && end - start == kCH) {
#pragma unroll
    for (int v = 0; v < CL::NV; ++v) {
      const int e0 = start + (v * kThreads + (int)threadIdx.x) * CL::VW;
      L.raw[v] = *(const uint4*)(rp + (size_t)e0 * CL::ESZ);
    }
  }
}

template <int DT>
__device__ __forceinline__ void unpack_chunk(const Args& a, int row, int start, int end, const ChunkLoad<DT>& L,
                                             float (&z)[kEPT]) {
  using CL = ChunkLoad<DT>;
  if (L.vec && end - start == kCH) {
    // every vector of the chunk was loaded
#pragma unroll
    for (int v = 0; v < CL::NV; ++v) {
      const u32 w4[4] = {L.raw[v].x, L.raw[v].y, L.raw[v].z, L.raw[v].w};
      if (DT == QS_DTYPE_F32) {
#pragma unroll
        for (int j = 0; j < 4; ++j) z[v * 4 + j] = __uint_as_float(w4[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          z[v * 8 + 2 * j] = bf16_to_f32(w4[j] & 0xffffu);
          z[v * 8 + 2 * j + 1] = bf16_to_f32(w4[j] >> 16);
        }
      }
    }
    return;
  }
  // the last chunk of a row, or an unaligned row: element loads
  const char* rp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * CL::ESZ;
#pragma unroll
  for (int v = 0; v < CL::NV; ++v) {
#pragma unroll
    for (int j = 0; j < CL::VW; ++j) {
      const int e = start + (v * kThreads + (int)threadIdx.x) * CL::VW + j;
      const int ec = e < end ? e : end - 1;
      const float x = (DT == QS_DTYPE_F32) ? ((const float*)rp)[ec] : bf16_to_f32(((const uint16_t*)rp)[ec]);
      z[v * CL::VW + j] = e < end ? x : 0.0f;
    }
  }
}

// ---------------------------------------------------------------- region writes

// Writes the chunk's tokens whose key kz is at least `thr` to the
// workgroup's region, in id order (the id start + (v * 256 + t) * VW + j is
// ordered by (v, t, j)), as {id, key of q, M, n}: q = f_of_key(key) / T for
// z keys (ZKEYS) or f_of_key(key) for q keys, and exp(q) = M * 2^(n - 23) as
// in the weights.  The tokens are first staged in LDS as (chunk index, key) at
// their final positions; the entries are then computed one per thread and
// stored contiguously.  Returns their number (the same in every thread) and,
// in *below, the largest key under `thr`.  Nothing is written when they do not
// fit the region (more than a.R).  The entries are read by k_finish, a later
// kernel.  `lds` holds kStageCap uint2 and is free on return.
template <int DT, bool ZKEYS>
__device__ __forceinline__ u32 emit_region(const Args& a, int row, int blk, int start, const u32 (&kz)[kEPT], u32 thr,
                                           float T, unsigned char* lds, Scratch& sc, u32* below_out) {
  constexpr int VW = (DT == QS_DTYPE_F32) ? 4 : 8;
  constexpr int NV = kEPT / VW;
  constexpr int NW = (NV + 1) / 2;  // counts per vector packed two to a word (16-bit fields)
  const int tid = threadIdx.x, wv = tid >> 6;
  if (thr == 0u) thr = 1u;  // key 0 (NaN, or past the end of the row) is never written
  u32 pk[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) pk[w] = 0u;
  u32 below = 0u;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      const u32 k = kz[v * VW + j];
      const bool in = k >= thr;
      pk[v >> 1] += (in ? 1u : 0u) << (16 * (v & 1));
      below = in ? below : (k > below ? k : below);
    }
  }
  u32 inc[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) inc[w] = wave_incl_scan(pk[w]);
  const u32 bw = wave_max(below);
  if (lane_id() == 63) {
#pragma unroll
    for (int w = 0; w < NW; ++w) sc.v[wv][w] = inc[w];
  }
  if (lane_id() == 0) sc.v[wv][7] = bw;
  __syncthreads();
  u32 base[NW], tot[NW], bmax = 0u;
#pragma unroll
  for (int w = 0; w < NW; ++w) base[w] = tot[w] = 0u;
  for (int i = 0; i < kWaves; ++i) {
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const u32 x = sc.v[i][w];
      base[w] += (i < wv) ? x : 0u;
      tot[w] += x;
    }
    bmax = sc.v[i][7] > bmax ? sc.v[i][7] : bmax;
  }
  __syncthreads();
  u32 total = 0u;
#pragma unroll
  for (int v = 0; v < NV; ++v) total += (tot[v >> 1] >> (16 * (v & 1))) & 0xffffu;
  *below_out = bmax;
  if (total > (u32)a.R) return total;
  // stage (chunk index, key) at the final positions
  u32* stg_i = (u32*)lds;           // [kStageCap] chunk index
  u32* stg_k = stg_i + kStageCap;   // [kStageCap] key
  u32 run = 0u;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int sh = 16 * (v & 1);
    u32 pos = run + (((base[v >> 1] + inc[v >> 1] - pk[v >> 1]) >> sh) & 0xffffu);
    const u32 l0 = (u32)((v * kThreads + tid) * VW);
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      u32 k = kz[v * VW + j];
      asm volatile("" : "+v"(k));  // compared again here: keeping 32 lane masks costs registers
      if (k >= thr) {
        stg_i[pos] = l0 + (u32)j;
        stg_k[pos] = k;
        ++pos;
      }
    }
    run += (tot[v >> 1] >> sh) & 0xffffu;
  }
  __syncthreads();
  // the entries, one per thread
  uint4* rg = a.cand + ((size_t)row * a.G + blk) * a.R;
  for (u32 i = (u32)tid; i < total; i += kThreads) {
    const uint2 s = make_uint2(stg_i[i], stg_k[i]);
    const float q = ZKEYS ? f_of_key(s.y) / T : f_of_key(s.y);
    const double y = y_of(q);
    const double fl = floor(y);
    rg[i] = make_uint4((u32)start + s.x, skey(q), mant24(exp2_poly((float)(y - fl))), (u32)(int)fl);
  }
  __syncthreads();
  return total;
}

// ---------------------------------------------------------------- finishing a row from its regions

// finish_row with at most 256 members, in id order in LDS (st: ids, keys,
// packed weights, kThreads each): one per thread.  Each candidate's rank in (q desc,
// id asc) order is counted directly, the candidates are placed in that order,
// and one prefix sum in it gives the top-k set, its mass and the top-p
// boundary; a second, in id order, gives the draw.
template <bool TOPK>
__device__ __forceinline__ bool finish_small(const Args& a, const RowParams& p, int row, u32 m, int N, u32 nout,
                                             u32* st, Scratch& sc) {
  const int tid = threadIdx.x;
  u32* st_id = st;
  u32* st_key = st_id + kThreads;
  u32* st_wp = st_key + kThreads;
  const bool have = (u32)tid < m;
  const u32 mkey = have ? st_key[tid] : 0u, mid = have ? st_id[tid] : 0u, mwp = have ? st_wp[tid] : 0u;
  // rank: members with a larger key, or the same key and a smaller id (an earlier slot)
  u32 rank = 0u;
  if (have) {
    u32 j = 0u;
    for (; j + 4u <= m; j += 4u) {
      const uint4 k4 = *(const uint4*)&st_key[j];
      rank += (k4.x > mkey || (k4.x == mkey && j < (u32)tid)) ? 1u : 0u;
      rank += (k4.y > mkey || (k4.y == mkey && j + 1u < (u32)tid)) ? 1u : 0u;
      rank += (k4.z > mkey || (k4.z == mkey && j + 2u < (u32)tid)) ? 1u : 0u;
      rank += (k4.w > mkey || (k4.w == mkey && j + 3u < (u32)tid)) ? 1u : 0u;
    }
    for (; j < m; ++j) {
      const u32 kj = st_key[j];
      rank += (kj > mkey || (kj == mkey && j < (u32)tid)) ? 1u : 0u;
    }
  }
  __syncthreads();
  if (have) {
    st_key[rank] = mkey;
    st_wp[rank] = mwp;
    st_id[rank] = mid;
  }
  __syncthreads();
  // thread i now holds the candidate of rank i
  const u32 rkey = have ? st_key[tid] : 0u, rwp = have ? st_wp[tid] : 0u, rid = have ? st_id[tid] : 0u;
  u32 kappa = 0u;
  if (TOPK) {
    if (m < (u32)p.k) return give_up(a, row, kWhyFewer);
    kappa = st_key[p.k - 1];
    // every token left out has a q key <= nout: it must be below the k-th
    if (nout > 0u && nout >= kappa) return give_up(a, row, kWhyIncomplete);
  }
  QS_TR(6);
  const bool intop = have && rkey >= kappa;
  const u128 rw = intop ? (u128)wunpack(rwp) : (u128)0;
  Acc tot;
  const Acc ex = block_scan_acc(acc_of(rw, intop ? 1u : 0u), sc, &tot);
  const u128 S = acc_mass(tot);
  QS_TR(13);
  u32 kp = kappa, idp = 0xffffffffu;  // kept: key > kp || (key == kp && id <= idp)
  u128 W = S;
  if (p.topp_on) {
    // the first candidate in this order whose inclusive mass exceeds floor(top_p * S)
    const u128 Tp = mul_frac(S, p.tp);
    if (tid == 0) sc.r[5] = 0xffffffffu;
    __syncthreads();
    if (intop && Tp >= acc_mass(ex) && Tp < acc_mass(ex) + rw) {
      sc.r[5] = (u32)tid;
      sc.w[6] = (u64)(acc_mass(ex) + rw);
      sc.w[7] = (u64)((acc_mass(ex) + rw) >> 64);
    }
    __syncthreads();
    const u32 c = sc.r[5];
    if (c == 0xffffffffu) return give_up(a, row, kWhyTopP);
    kp = st_key[c];
    idp = st_id[c];
    W = mk128(sc.w[6], sc.w[7]);
    __syncthreads();
  }
  QS_TR(7);
  // ---- the draw: kept candidates in id order, which is the order of the slots
  const u128 t = mul_frac(W, p.u);
  const bool kept = have && (mkey > kp || (mkey == kp && mid <= idp));
  const u128 mw = kept ? (u128)wunpack(mwp) : (u128)0;
  if (tid == 0) sc.r[6] = 0xffffffffu;
  const Acc dx = block_scan_acc(acc_of(mw, 0u), sc, &tot);
  if (kept && t >= acc_mass(dx) && t < acc_mass(dx) + mw) sc.r[6] = mid;
  __syncthreads();
  const u32 chosen = sc.r[6];
  __syncthreads();
  QS_TR(9);
  (void)rid;
  if (tid == 0)
    publish_result(a, row, chosen == 0xffffffffu ? -1ll : (long long)chosen, N, W, kp, idp, false, TOPK ? 1u : 4u);
  __syncthreads();
  return true;
}


// Resolves a row from the regions of all its workgroups: the last workgroup of
// a top-k row (TOPK: entries hold z keys; k-select, then a proof that no token
// left out could be in the top-k set) or the first workgroup of a peaked mass
// row (entries hold q keys; `kthr` drops those outside the row's window).
// The regions are gathered in id order into registers: thread t holds the
// concatenated entries [t * per, t * per + per), so register order is id
// order.  At most 256 members go through finish_small; more are resolved over
// one 2048-bin histogram of their keys (count and mass per bin), whose single
// scan places the k-th key and the top-p boundary in their bins.
// False if the candidates cannot be proven to hold the answer; the caller then
// resolves the row with resolve_single.
template <bool TOPK>
__device__ __forceinline__ bool finish_row(const Args& a, const RowParams& p, int row, u32 kthr, unsigned char* lds,
                                           Scratch& sc) {
  const int tid = threadIdx.x;
  const Slot* sl = a.slots + (size_t)row * a.G;
  const uint4* cd = a.cand + (size_t)row * a.G * a.R;
  // (written by k_sample, an earlier kernel on this stream: plain loads see it)
  u32* hoff = (u32*)lds;  // [kMaxChunks + 1] start of each region's entries in the concatenation
  WideLds& WL = *(WideLds*)(lds + kHoffBytes);
  SelLds* SL = (SelLds*)(lds + kHoffBytes + sizeof(WideLds));
  // ---- the regions' headers: one region per thread (G <= 256)
  u32 cnt = 0u, hx[3] = {0u, 0u, 0u};  // tau, overflow, below
  if (tid < a.G) {
    cnt = sl[tid].nb;
    if (TOPK) {
      hx[0] = sl[tid].tau;
      hx[2] = sl[tid].below;
    }
  }
  if (cnt == 0xffffffffu) {
    hx[1] = 1u;
    cnt = 0u;
  }
  u32 m0;
  const u32 coff = block_scan_max<3>(cnt, hx, sc, &m0);
  const u32 tstar = hx[0], below = hx[2];
  if (tid < a.G) hoff[tid] = coff;
  if (tid == 0) hoff[a.G] = m0;
  __syncthreads();
  QS_TR(11);
  if (hx[1]) return give_up(a, row, kWhyRegion);
  if (m0 > (u32)(kThreads * kGatherPer)) return give_up(a, row, kWhyMerge);
  // ---- this thread's share of the concatenated entries (id order): flat
  // indices [f0, f0 + per); all loads issued before any is used
  const u32 per = (m0 + kThreads - 1) / kThreads;  // <= kGatherPer
  const u32 f0 = (u32)tid * per;
  int g = 0;
  if (f0 < m0) {
    int lo = 0, hi = a.G - 1;  // the last region starting at or before f0
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (hoff[mid] <= f0) lo = mid; else hi = mid - 1;
    }
    g = lo;
  }
  uint4 ent[kGatherPer];
#pragma unroll
  for (int q = 0; q < kGatherPer; ++q) {
    const u32 f = f0 + (u32)q;
    ent[q] = make_uint4(0u, 0u, 0u, 0u);
    if ((u32)q < per && f < m0) {
      while (hoff[g + 1] <= f) ++g;
      ent[q] = cd[(size_t)g * a.R + (f - hoff[g])];
    }
  }
  // the histogram is cleared while the loads are in flight (the exchange
  // below orders it before its use)
  for (int i = tid; i < kWide; i += kThreads) {
    WL.cnt[i] = 0u;
    WL.mlo[i] = 0ull;
    WL.mhi[i] = 0ull;
  }
  if (tid == 0) {
    sc.i[1] = -1;  // wide_find result slots
    sc.i[2] = -1;
    sc.u[0] = sc.u[1] = sc.u[2] = sc.u[3] = 0u;  // key range of the k-th's and the boundary's bins
  }
  // ---- members: entries at or above the threshold.  One exchange gives
  // their number and positions, the row scale N (their largest octave), the
  // largest q key of the tokens left out, and their key range.
  const u32 thr = TOPK ? skey(f_of_key(tstar) / p.T) : kthr;
  u32 memb = 0u, npass = 0u, dropmax = 0u, kmx = 0u, nkmn = 0u;
  int nmax = (int)0x80000000u;
#pragma unroll
  for (int q = 0; q < kGatherPer; ++q) {
    if ((u32)q < per && f0 + (u32)q < m0) {
      const u32 k = ent[q].y;
      if (k >= thr) {
        memb |= 1u << q;
        ++npass;
        nmax = (int)ent[q].w > nmax ? (int)ent[q].w : nmax;
        kmx = k > kmx ? k : kmx;
        nkmn = ~k > nkmn ? ~k : nkmn;
      } else {
        dropmax = k > dropmax ? k : dropmax;
      }
    }
  }
  QS_TR(1);
  u32 sx[4] = {dropmax, (u32)nmax ^ 0x80000000u, kmx, nkmn};
  if (TOPK) {
    // largest q key of the tokens left out: dropped entries, and below each region's threshold
    const u32 bq = below ? skey(f_of_key(below) / p.T) : 0u;
    sx[0] = dropmax > bq ? dropmax : bq;
  }
  u32 m;
  const u32 off = block_scan_max<4>(npass, sx, sc, &m);
#ifdef QS_TRACE
  if (a.trace && tid == 0) {
    ((u32*)(a.ctl + row))[40] = m0;
    ((u32*)(a.ctl + row))[41] = m;
  }
#endif
  const u32 nout = TOPK ? sx[0] : 0u;
  const int N = (int)(sx[1] ^ 0x80000000u);
  if (TOPK && m < (u32)p.k) return give_up(a, row, kWhyFewer);
  u32 key[kGatherPer], id[kGatherPer], wp[kGatherPer];
#pragma unroll
  for (int q = 0; q < kGatherPer; ++q) {
    const int r = (int)ent[q].w - N + kWindow;
    key[q] = ent[q].y;
    id[q] = ent[q].x;
    wp[q] = (((memb >> q) & 1u) && r >= 0) ? ((u32)r << 24) | ent[q].z : 0u;
  }
  if (m <= (u32)kThreads) {
    // few members: one per thread, in id order, through LDS
    u32* st = (u32*)(lds + kHoffBytes);  // [3][kThreads] ids, keys, packed weights
    u32 pos = off;
#pragma unroll
    for (int q = 0; q < kGatherPer; ++q) {
      if ((memb >> q) & 1u) {
        st[pos] = id[q];
        st[kThreads + pos] = key[q];
        st[2 * kThreads + pos] = wp[q];
        ++pos;
      }
    }
    __syncthreads();
    QS_TR(2);
    return finish_small<TOPK>(a, p, row, m, N, nout, st, sc);
  }
  // ---- the histogram: bits [lob, lob + 11) of the key.  Bits above hib are
  // common to all members, so the digit is monotone in the key; with lob == 0
  // a bin holds a single key, (kfirst & ~(kWide - 1)) | bin.
  const u32 kfirst = ~sx[3], kdiff = sx[2] ^ kfirst;
  const int hib = kdiff ? 31 - __clz(kdiff) : 0;
  const int lob = hib >= kWideBits - 1 ? hib - (kWideBits - 1) : 0;
  auto digit = [&](u32 k) { return (int)((k >> lob) & (u32)(kWide - 1)); };
#pragma unroll
  for (int q = 0; q < kGatherPer; ++q) {
    if ((memb >> q) & 1u) {
      const int d = digit(key[q]);
      atomicAdd(&WL.cnt[d], 1u);
      u32 wj = wp[q];
      asm volatile("" : "+v"(wj));
      const u64 w = wunpack(wj);
      if (w) {
        atomicAdd(&WL.mlo[d], w & 0xffffffffull);
        atomicAdd(&WL.mhi[d], w >> 32);
      }
    }
  }
  __syncthreads();
  QS_TR(4);
  Acc wbin[kWidePer], wmine = {0, 0, 0};
#pragma unroll
  for (int i = 0; i < kWidePer; ++i) {
    wbin[i] = wide_bin(WL, kWide - 1 - (tid * kWidePer + i));
    wmine = acc_add(wmine, wbin[i]);
  }
  Acc wtot;
  const Acc wex = block_scan_acc(wmine, sc, &wtot);
  QS_TR(8);
  // the key range of bin b's members (r0, r1 in sc.u) is a single key iff it
  // collapses: one LDS max per member of the bin, one barrier
  auto bin_single = [&](int b, int r0, u32* kv) {
#pragma unroll
    for (int q = 0; q < kGatherPer; ++q) {
      if (((memb >> q) & 1u) && digit(key[q]) == b) {
        atomicMax(&sc.u[r0], key[q]);
        atomicMax(&sc.u[r0 + 1], ~key[q]);
      }
    }
    __syncthreads();
    const u32 hi = sc.u[r0], nlo = sc.u[r0 + 1];
    *kv = hi;
    return hi == ~nlo;
  };
  // ---- top-k: the k-th largest q, and the proof that the candidates hold the top-k set
  u32 kappa = 0u;
  int bk = -1;
  Acc kb = {0, 0, 0}, ka = {0, 0, 0};  // bins above kappa's, kappa's bin
  bool ksingle = true;                 // kappa's bin holds kappa only
  u128 S;
  if (TOPK) {
    wide_find(wbin, wex, false, (u128)(p.k - 1), sc, 0, &bk, &kb, &ka);
    QS_TR(10);
    if (bk < 0) return give_up(a, row, kWhyKSelect);
    if (lob == 0) {
      kappa = (kfirst & ~(u32)(kWide - 1)) | (u32)bk;
    } else if (bin_single(bk, 0, &kappa)) {
      // kappa: the bin's single key
    } else {
      u32 mk = 0u;
#pragma unroll
      for (int q = 0; q < kGatherPer; ++q)
        if (((memb >> q) & 1u) && digit(key[q]) == bk) mk |= 1u << q;
      {
        ksingle = false;
        const SelOut sk = reg_select<false>(key, mk, wp, (u128)(p.k - 1 - kb.c), SL, sc);
        if (!sk.ok) return give_up(a, row, kWhyKSelect);
        kappa = sk.val;
      }
    }
    QS_TR(6);
    // every token left out has a q key <= nout: it must be below the k-th
    if (nout > 0u && nout >= kappa) return give_up(a, row, kWhyIncomplete);
    if (ksingle) {
      S = acc_mass(kb) + acc_mass(ka);
    } else {
      u128 sv = 0;
#pragma unroll
      for (int q = 0; q < kGatherPer; ++q)
        if (((memb >> q) & 1u) && key[q] >= kappa) sv += (u128)wunpack(wp[q]);
      S = uni128(block_sum128(sv, sc));
    }
  } else {
    S = acc_mass(wtot);
  }
  QS_TR(13);
  u32 kp = kappa, idp = 0xffffffffu;  // kept: key > kp || (key == kp && id <= idp)
  u128 W = S;
  if (p.topp_on) {
    // the first token (q desc, id asc) whose inclusive mass exceeds floor(top_p * S)
    const u128 Tp = uni128(mul_frac(S, p.tp));
    u128 A;
    Acc at;
    if (TOPK && Tp >= acc_mass(kb)) {
      // the boundary lies in kappa's bin, among its keys >= kappa
      if (ksingle) {
        kp = kappa;
        A = acc_mass(kb);
        at = ka;
      } else {
        u32 mp = 0u;
#pragma unroll
        for (int q = 0; q < kGatherPer; ++q)
          if (((memb >> q) & 1u) && digit(key[q]) == bk && key[q] >= kappa) mp |= 1u << q;
        const SelOut sp = reg_select<true>(key, mp, wp, Tp - acc_mass(kb), SL, sc);
        if (!sp.ok) return give_up(a, row, kWhyTopP);
        kp = sp.val;
        A = acc_mass(kb) + acc_mass(sp.before);
        at = sp.at;
      }
    } else {
      int bp;
      Acc pb, pa;
      wide_find(wbin, wex, true, Tp, sc, 1, &bp, &pb, &pa);
      QS_TR(12);
      if (bp < 0) return give_up(a, row, kWhyTopP);
      u32 bkey = 0u;
      if (lob == 0) {
        kp = (kfirst & ~(u32)(kWide - 1)) | (u32)bp;
        A = acc_mass(pb);
        at = pa;
      } else if (bin_single(bp, 2, &bkey)) {
        kp = bkey;
        A = acc_mass(pb);
        at = pa;
      } else {
        u32 mp = 0u;
#pragma unroll
        for (int q = 0; q < kGatherPer; ++q)
          if (((memb >> q) & 1u) && digit(key[q]) == bp) mp |= 1u << q;
        {
          const SelOut sp = reg_select<true>(key, mp, wp, Tp - acc_mass(pb), SL, sc);
          if (!sp.ok) return give_up(a, row, kWhyTopP);
          kp = sp.val;
          A = acc_mass(pb) + acc_mass(sp.before);
          at = sp.at;
        }
      }
    }
    QS_TR(14);
    const u64 wk = wunpack(wpack(f_of_key(kp), N));
    const u64 jb = div_small(Tp - A, wk);  // 0-based boundary member among the ties (< at.c)
    if (jb + 1 >= at.c) {
      W = A + acc_mass(at);
    } else {
      W = A + (u128)wk * (u128)(jb + 1);
      // the boundary member: tie member jb in id order, which is register order
      u32 c = 0u;
#pragma unroll
      for (int q = 0; q < kGatherPer; ++q) c += (((memb >> q) & 1u) && key[q] == kp) ? 1u : 0u;
      if (tid == 0) sc.r[5] = 0xffffffffu;
      u32 ct;
      const u32 ex = block_scan_u32(c, sc, &ct);
      if (jb >= ex && jb < (u64)ex + c) {
        u32 r = ex;
#pragma unroll
        for (int q = 0; q < kGatherPer; ++q) {
          if (((memb >> q) & 1u) && key[q] == kp) {
            if (r == (u32)jb) sc.r[5] = id[q];
            ++r;
          }
        }
      }
      __syncthreads();
      idp = sc.r[5];
      __syncthreads();
    }
  }
  QS_TR(7);
  // ---- the draw: kept tokens in id order (register order), the first whose
  // inclusive mass exceeds floor(u * W)
  const u128 t = mul_frac(W, p.u);
  u32 keptm = 0u;
  u128 mine = 0;
#pragma unroll
  for (int q = 0; q < kGatherPer; ++q) {
    if (((memb >> q) & 1u) && (key[q] > kp || (key[q] == kp && id[q] <= idp))) {
      keptm |= 1u << q;
      mine += (u128)wunpack(wp[q]);
    }
  }
  if (tid == 0) sc.r[6] = 0xffffffffu;
  Acc tot;
  const Acc ex = block_scan_acc(acc_of(mine, 0u), sc, &tot);
  {
    const u128 lo = acc_mass(ex);
    if (t >= lo && t < lo + mine) {
      u128 run = lo;
      bool found = false;
#pragma unroll
      for (int q = 0; q < kGatherPer; ++q) {
        if (!found && ((keptm >> q) & 1u)) {
          run += (u128)wunpack(wp[q]);
          if (run > t) {
            sc.r[6] = id[q];
            found = true;
          }
        }
      }
    }
  }
  __syncthreads();
  const u32 chosen = sc.r[6];
  __syncthreads();
  QS_TR(9);
  if (tid == 0)
    publish_result(a, row, chosen == 0xffffffffu ? -1ll : (long long)chosen, N, W, kp, idp, false, TOPK ? 1u : 4u);
  __syncthreads();
  return true;
}

// ---------------------------------------------------------------- flat mass rows

// Bracket of bins [blo, bhi] that provably holds the top-p boundary (the first
// token, in descending order, whose inclusive mass exceeds Tp).  g[b] is the
// sum over bin b's tokens of (w >> shift); each token truncates less than one
// unit, so `err` (the number of tokens) bounds the error of any sum of bins.
// One bin per thread.
//   bhi: the lowest bin whose mass above it is provably <= Tp;
//   blo: the highest bin whose mass at or above it is provably > Tp.
__device__ __forceinline__ void bracket_bins(const u64* g, u64 err, u128 Tp, int shift, Scratch& sc, int* blo,
                                             int* bhi) {
  static_assert(kBins == kThreads, "one histogram bin per thread");
  const int tid = threadIdx.x;
  const int b = kBins - 1 - tid;  // thread order = descending bins
  const u64 gb = g[b];
  if (tid == 0) {
    sc.r[10] = 0xffffffffu;  // min over bins meeting the bhi condition
    sc.r[11] = 0u;           // max over bins meeting the blo condition, +1
  }
  Acc tot;
  const Acc ex = block_scan_acc(acc_of((u128)gb, 0u), sc, &tot);
  const u128 run = acc_mass(ex);  // lower bound of the mass above bin b, in units
  if (((run + err) << shift) <= Tp) atomicMin(&sc.r[10], (u32)b);
  if (((run + gb) << shift) > Tp) atomicMax(&sc.r[11], (u32)b + 1u);
  __syncthreads();
  int hi = sc.r[10] == 0xffffffffu ? kBins - 1 : (int)sc.r[10];
  int lo = sc.r[11] == 0u ? 0 : (int)sc.r[11] - 1;
  __syncthreads();
  if (lo > hi) lo = hi;
  *blo = lo;
  *bhi = hi;
}

// Histogram bins of a flat mass row, linear in q from q0 with scale s:
// bin(q) = (int)clamp((q - q0) * s, 0, kBins - 1) in fp32, non-decreasing in q
// and so in the key.
struct QBins {
  float q0, s;
  __device__ __forceinline__ int bin(float q) const {
    const float x = fminf(fmaxf((q - q0) * s, 0.0f), (float)(kBins - 1));
    return (int)x;
  }
  // The smallest key in [1, key(+inf)] whose bin is at least b (b <= kBins - 1).
  __device__ __forceinline__ u32 first_key(int b) const {
    u32 lo = 1u, hi = 0xff800000u;
    while (lo < hi) {
      const u32 mid = lo + ((hi - lo) >> 1);
      if (bin(f_of_key(mid)) >= b) hi = mid; else lo = mid + 1u;
    }
    return lo;
  }
};
__device__ __forceinline__ QBins qbins_of(float qlo, float qhi) {
  QBins r;
  r.q0 = qlo;
  r.s = qhi > qlo ? (float)kBins / (qhi - qlo) : 0.0f;
  return r;
}

// Per segment (vector v, this wave) of a k_sample workgroup: the exact sum of
// the lanes' lo + hi * 2^64, written to sgm[2 * (v * kWaves + wave)].
template <int NV>
__device__ __forceinline__ void store_segments(u64* sgm, const u64 (&lo)[NV], const u32 (&hi)[NV]) {
  const int wv = threadIdx.x >> 6;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const u128 m = wave_sum128(lo[v], hi[v]);
    if (lane_id() == 0) {
      sgm[2 * (v * kWaves + wv)] = (u64)m;
      sgm[2 * (v * kWaves + wv) + 1] = (u64)(m >> 64);
    }
  }
}

// Segment s of chunk g, s = v * kWaves + w: the tokens that wave w of the
// chunk's k_sample workgroup held in vector v, the ids
// [seg_first(g, s), seg_first(g, s) + 64 * VW) (clipped at the row's end).
template <int DT>
__device__ __forceinline__ int seg_first(int g, int s) {
  constexpr int VW = ChunkLoad<DT>::VW;
  return g * kCH + ((s / kWaves) * kThreads + (s % kWaves) * 64) * VW;
}

// Re-reads segment s of chunk g (one or two tokens per thread, in id order).
// DRAW: the id of the first kept token (key > kp || (key == kp && id <= idp))
// whose inclusive mass within the segment exceeds tl.  Otherwise: the id of
// the token of rank `rank` (0-based, id order) among those whose key is kp.
// 0xffffffff if there is none.  `plds` holds the chunk's penalty table.
template <int DT, bool DRAW>
__device__ __forceinline__ u32 seg_locate(const Args& a, const RowParams& p, int row, int g, int s, int N, u32 kp,
                                          u32 idp, u128 tl, u32 rank, unsigned char* plds, Scratch& sc) {
  constexpr int VW = ChunkLoad<DT>::VW;
  constexpr int E = 64 * VW / kThreads;  // tokens per thread
  const int tid = threadIdx.x;
  const int start = g * kCH, end = min(a.V, start + kCH);
  PenTable pt;
  pt.bits = (u32*)plds;
  pt.wpre = pt.bits + (kCH >> 5);
  pt.cnts = pt.wpre + (kCH >> 5);
  if (p.pen_on) pen_build(a, row, start, end, pt, sc);
  const int e0 = seg_first<DT>(g, s) + tid * E;
  float q[E];
  u32 k[E];
#pragma unroll
  for (int j = 0; j < E; ++j) {
    const int e = e0 + j;
    float zz = e < end ? load_logit<DT>(a, row, e) : 0.0f;
    if (p.pen_on && e < end) {
      const u32 cn = pen_count(pt, e - start);
      if (cn) zz = apply_penalty(zz, cn, p.rep, p.pres, p.freq);
    }
    q[j] = zz / p.T;
    k[j] = e < end ? skey(q[j]) : 0u;
  }
  if (tid == 0) sc.r[9] = 0xffffffffu;
  if (DRAW) {
    u64 w[E];
    u128 mine = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
      const bool kept = k[j] && (k[j] > kp || (k[j] == kp && (u32)(e0 + j) <= idp));
      w[j] = kept ? weight_of(q[j], N) : 0ull;
      mine += (u128)w[j];
    }
    Acc tot;
    const Acc ex = block_scan_acc(acc_of(mine, 0u), sc, &tot);
    u128 run = acc_mass(ex);
    if (tl >= run && tl < run + mine) {
      bool found = false;
#pragma unroll
      for (int j = 0; j < E; ++j) {
        run += (u128)w[j];
        if (!found && run > tl) {
          sc.r[9] = (u32)(e0 + j);
          found = true;
        }
      }
    }
  } else {
    u32 c = 0u;
#pragma unroll
    for (int j = 0; j < E; ++j) c += (k[j] && k[j] == kp) ? 1u : 0u;
    u32 ct;
    const u32 ex = block_scan_u32(c, sc, &ct);
    if (rank >= ex && rank < ex + c) {
      u32 r = ex;
#pragma unroll
      for (int j = 0; j < E; ++j) {
        if (k[j] && k[j] == kp) {
          if (r == rank) sc.r[9] = (u32)(e0 + j);
          ++r;
        }
      }
    }
  }
  __syncthreads();
  const u32 id = sc.r[9];
  __syncthreads();
  return id;
}

// LDS of the flat-row resolver: two select buffers; per chunk, the kept mass
// of its bracket entries above the boundary key and its count of tokens at
// it; per segment of the owner chunk, the same, and per segment of the chunk
// holding the boundary token, its count of tokens at the boundary key.
struct FlatLds {
  SelLds sel[2];
  u64 clo[kMaxChunks];
  u64 chi[kMaxChunks];
  u32 ckp[kMaxChunks];
  u64 slo[kSegs];
  u64 shi[kSegs];
  u32 skp[kSegs];
  u32 bkp[kSegs];
};

// A flat mass row after k_sample: the top-p boundary from the bracket entries
// (topp) or none; the kept mass per chunk and the chunk holding the draw
// target; within it, the kept mass per segment and the segment holding the
// target; the token inside that segment.  With `topp` false every token is
// kept and the masses are the chunks' and segments' totals.
template <int DT>
__device__ __forceinline__ bool resolve_flat(const Args& a, const RowParams& p, int row, int N, bool topp, u128 Tp,
                                             bool bottom, unsigned char* lds, Scratch& sc) {
  constexpr int NSEG = ChunkLoad<DT>::NV * kWaves;
  const int tid = threadIdx.x;
  const Slot* sl = a.slots + (size_t)row * a.G;
  RowCtl* c = a.ctl + row;
  FlatLds& F = *(FlatLds*)lds;
  unsigned char* plds = lds + sizeof(FlatLds);
  // per-chunk mass above the bracket (topp) or of the whole chunk
  u128 ag = 0;
  if (tid < a.G) ag = topp ? mk128(ldc(&sl[tid].a_lo), ldc(&sl[tid].a_hi)) : mk128(ldc(&sl[tid].s_lo), ldc(&sl[tid].s_hi));
  u32 kp = 0u, idp = 0xffffffffu;  // kept: key > kp || (key == kp && id <= idp)
  u64 wk = 0ull;                   // weight of a token at kp
  u32 J = 0u;                      // tokens at kp kept (in id order), if they are split
  bool split = false;
  if (tid < kMaxChunks) {
    F.clo[tid] = 0ull;
    F.chi[tid] = 0ull;
    F.ckp[tid] = 0u;
  }
  if (tid < kSegs) {
    F.slo[tid] = 0ull;
    F.shi[tid] = 0ull;
    F.skp[tid] = 0u;
    F.bkp[tid] = 0u;
  }
  // bracket entries: key, count, chunk
  u32 key[kFinPer], cnt[kFinPer], wp[kFinPer], cs[kFinPer], memb = 0u;
  if (topp) {
    const u32 m = ldc(&c->list_n);
    const u32 st = ldc(&c->status);
    const u64* lst = a.list + (size_t)row * kListCap;
    const u32 P = (min(m, (u32)kListCap) + kThreads - 1) / kThreads;  // entries per thread, <= kFinPer
#pragma unroll
    for (int j = 0; j < kFinPer; ++j) {
      const u32 i = (u32)tid * P + (u32)j;
      const bool in = (u32)j < P && i < m && i < (u32)kListCap;
      const u64 e = in ? ldc(&lst[i]) : 0ull;
      key[j] = (u32)(e >> 32);
      cnt[j] = (u32)e & 0xffffu;
      cs[j] = ((u32)e >> 16) & 0xffu;
      if (in) memb |= 1u << j;
    }
    const u128 A = block_sum128(ag, sc);
    QS_TR(1);
    if (m > (u32)kListCap || (st & kStList)) return give_up(a, row, kWhyList);
    if (A > Tp) return give_up(a, row, kWhyAbove);
#pragma unroll
    for (int j = 0; j < kFinPer; ++j) wp[j] = ((memb >> j) & 1u) ? wpack(f_of_key(key[j]), N) : 0u;
    const SelOut sp = reg_select<true, kFinPer, true>(key, memb, wp, Tp - A, F.sel, sc, cnt);
    QS_TR(2);
    if (!sp.ok) {
      // every bracketed token is kept: right only if nothing with weight lies below
      if (!bottom) return give_up(a, row, kWhyBracket);
    } else {
      kp = sp.val;
      const u128 A2 = A + acc_mass(sp.before);
      wk = wunpack(wpack(f_of_key(kp), N));
      const u64 jb = div_small(Tp - A2, wk);  // 0-based boundary member among the tokens at kp
      if (jb + 1 < sp.at.c) {
        split = true;
        J = (u32)jb + 1u;
      }
    }
    // per chunk: mass of the entries above kp, tokens at kp
#pragma unroll
    for (int j = 0; j < kFinPer; ++j) {
      if ((memb >> j) & 1u) {
        const u32 ch = cs[j];
        if (key[j] > kp) {
          const u64 w = wunpack(wp[j]);
          atomicAdd(&F.clo[ch], (w & 0xffffffffull) * cnt[j]);
          atomicAdd(&F.chi[ch], (w >> 32) * cnt[j]);
        } else if (key[j] == kp) {
          atomicAdd(&F.ckp[ch], cnt[j]);
        }
      }
    }
    __syncthreads();
  }
  // kept mass per chunk (one chunk per thread); tokens at kp are kept in id
  // order, chunk by chunk, until J of them
  u32 kpc = (tid < a.G) ? F.ckp[tid] : 0u;
  u32 kpt;
  const u32 kpre = block_scan_u32(kpc, sc, &kpt);
  u32 keep = kpc;
  if (split) keep = J > kpre ? min(kpc, J - kpre) : 0u;
  if (tid == 0) {
    sc.r[8] = 0xffffffffu;
    sc.r[14] = 0xffffffffu;
  }
  u128 kg = 0;
  if (tid < a.G) kg = ag + mk128(F.clo[tid], 0) + ((u128)F.chi[tid] << 32) + (u128)wk * keep;
  Acc tot;
  const Acc ex = block_scan_acc(acc_of(kg, 0u), sc, &tot);  // its barriers order the writes below after the ones above
  // the chunk holding the boundary token (the J-th at kp) and its rank there
  if (split && tid < a.G && J - 1u >= kpre && J - 1u < kpre + kpc) {
    sc.r[14] = (u32)tid;
    sc.r[15] = J - 1u - kpre;
  }
  const u128 W = acc_mass(tot);
  const u128 t = mul_frac(W, p.u);
  if (tid < a.G && t >= acc_mass(ex) && t < acc_mass(ex) + kg) {
    sc.r[8] = (u32)tid;
    const u128 tl = t - acc_mass(ex);
    sc.w[16] = (u64)tl;
    sc.w[17] = (u64)(tl >> 64);
  }
  __syncthreads();
  const int owner = (int)sc.r[8];
  const u128 tl = mk128(sc.w[16], sc.w[17]);
  const int gb = (int)sc.r[14];
  const u32 rb = sc.r[15];
  __syncthreads();
  QS_TR(3);
  if (owner < 0 || owner >= a.G) return give_up(a, row, kWhyOwner);
  if (split && (gb < 0 || gb >= a.G)) return give_up(a, row, kWhyTie);
  // ---- segments: tokens at kp per segment of chunk gb (for the boundary
  // token) and the kept bracket entries per segment of the owner chunk, from
  // those chunks' own (key, segment) lists
  if (topp) {
    const u32 no = ldc(&sl[owner].nse);
    const u32 nb2 = split ? ldc(&sl[gb].nse) : 0u;
    if (no == 0xffffffffu || nb2 == 0xffffffffu) return give_up(a, row, kWhyList);
    const u64* so = a.sent + ((size_t)row * a.G + owner) * kSegEnt;
    const u64* sbp = a.sent + ((size_t)row * a.G + (split ? gb : 0)) * kSegEnt;
    for (u32 i = tid; i < no; i += kThreads) {
      const u64 e = so[i];
      const u32 k = (u32)(e >> 32), sg = ((u32)e >> 16) & 31u, n = (u32)e & 0xffffu;
      if (k > kp) {
        const u64 w = wunpack(wpack(f_of_key(k), N));
        atomicAdd(&F.slo[sg], (w & 0xffffffffull) * n);
        atomicAdd(&F.shi[sg], (w >> 32) * n);
      } else if (k == kp) {
        atomicAdd(&F.skp[sg], n);
      }
    }
    for (u32 i = tid; i < nb2; i += kThreads) {
      const u64 e = sbp[i];
      if ((u32)(e >> 32) == kp) atomicAdd(&F.bkp[((u32)e >> 16) & 31u], (u32)e & 0xffffu);
    }
  }
  const u64* sgm = a.segm + ((size_t)row * a.G + owner) * (2 * kSegs);
  u128 ms = 0;
  if (tid < NSEG) ms = mk128(sgm[2 * tid], sgm[2 * tid + 1]);
  __syncthreads();
  int sb = -1;
  u32 rbs = 0u;
  if (split) {
    // the boundary token: rank rb among chunk gb's tokens at kp, by segment
    const u32 bc = tid < NSEG ? F.bkp[tid] : 0u;
    if (tid == 0) sc.r[13] = 0xffffffffu;
    u32 bt;
    const u32 bx = block_scan_u32(bc, sc, &bt);
    if (tid < NSEG && rb >= bx && rb < bx + bc) {
      sc.r[13] = (u32)tid;
      sc.r[12] = rb - bx;
    }
    __syncthreads();
    sb = (int)sc.r[13];
    rbs = sc.r[12];
    __syncthreads();
    if (sb < 0 || sb >= NSEG) return give_up(a, row, kWhyTie);
    idp = seg_locate<DT, false>(a, p, row, gb, sb, N, kp, 0u, 0, rbs, plds, sc);
    if (idp == 0xffffffffu) return give_up(a, row, kWhyTie);
  }
  QS_TR(8);
  // kept mass per segment of the owner chunk (one segment per thread)
  u128 km = 0;
  if (tid < NSEG) {
    u32 ks = F.skp[tid];  // tokens at kp in the segment, kept in id order up to the boundary token
    if (split) {
      if (owner > gb || (owner == gb && tid > sb)) ks = 0u;
      else if (owner == gb && tid == sb) ks = rbs + 1u;
    }
    km = ms + mk128(F.slo[tid], 0) + ((u128)F.shi[tid] << 32) + (u128)wk * ks;
  }
  if (tid == 0) sc.r[11] = 0xffffffffu;
  Acc stot;
  const Acc sx = block_scan_acc(acc_of(km, 0u), sc, &stot);
  if (tid < NSEG && tl >= acc_mass(sx) && tl < acc_mass(sx) + km) {
    sc.r[11] = (u32)tid;
    const u128 t2 = tl - acc_mass(sx);
    sc.w[16] = (u64)t2;
    sc.w[17] = (u64)(t2 >> 64);
  }
  __syncthreads();
  const int os = (int)sc.r[11];
  const u128 tl2 = mk128(sc.w[16], sc.w[17]);
  __syncthreads();
  if (os < 0 || os >= NSEG) return give_up(a, row, kWhyOwner);
  const u32 chosen = seg_locate<DT, true>(a, p, row, owner, os, N, kp, idp, tl2, 0u, plds, sc);
  QS_TR(10);
  if (tid == 0)
    publish_result(a, row, chosen == 0xffffffffu ? -1ll : (long long)chosen, N, W, kp, idp, false, 2u);
  __syncthreads();
  return true;
}

// The chunk of a row into registers, history penalties applied: thread t
// holds z[v * VW + j] = logit start + (v * 256 + t) * VW + j.
template <int DT>
__device__ __forceinline__ void load_chunk_pen(const Args& a, const RowParams& p, int row, int start, int end,
                                               float (&z)[kEPT], unsigned char* lds, Scratch& sc) {
  constexpr int VW = ChunkLoad<DT>::VW;
  constexpr int NV = ChunkLoad<DT>::NV;
  const int tid = threadIdx.x;
  PenTable pt;
  pt.bits = (u32*)lds;
  pt.wpre = pt.bits + (kCH >> 5);
  pt.cnts = pt.wpre + (kCH >> 5);
  ChunkLoad<DT> cl;
  // bf16: the loads overlap the table's build; fp32 chunks are twice the
  // registers, so they are loaded after it
  if (DT == QS_DTYPE_BF16) issue_chunk<DT>(a, row, start, end, cl);
  if (p.pen_on) pen_build(a, row, start, end, pt, sc);
  QS_TR(8);
  if (DT == QS_DTYPE_F32) issue_chunk<DT>(a, row, start, end, cl);
  unpack_chunk<DT>(a, row, start, end, cl, z);
  QS_TR(9);
  if (p.pen_on) {
    // one bitmap word per vector (its VW tokens are aligned inside one word);
    // counts are looked up only for the tokens present in the history
    u32 pres[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int o = (v * kThreads + tid) * VW;  // chunk-relative
      pres[v] = o < end - start ? (pt.bits[o >> 5] >> (o & 31)) & ((1u << VW) - 1u) : 0u;
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      if (pres[v]) {  // rare: a vector with a history token
        const int o = (v * kThreads + tid) * VW;
        const u32 bw = pt.bits[o >> 5];
        const u32 base = pt.wpre[o >> 5];
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          if ((pres[v] >> j) & 1u) {
            const int l = o + j;
            const u32 cnt = pt.cnts[base + __popc(bw & ((1u << (l & 31)) - 1u))];
            z[v * VW + j] = apply_penalty(z[v * VW + j], cnt, p.rep, p.pres, p.freq);
          }
        }
      }
    }
    __syncthreads();  // the LDS table is reused after
  }
}

// ---------------------------------------------------------------- streaming kernel

// One workgroup per (chunk, row).  ROLE 0: greedy rows (resolved here by the
// last workgroup to arrive) and the regions of top-k rows; ROLE 1: mass rows
// (regions, the row maximum, and for flat rows the bin masses, the bracket and
// the bracketed tokens).  k_finish resolves the other rows afterwards.
template <int DT, int ROLE>
__global__ __launch_bounds__(kThreads) void k_sample(Args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ Scratch sc;
  constexpr int VW = ChunkLoad<DT>::VW;
  constexpr int NV = ChunkLoad<DT>::NV;
  const int row = blockIdx.y, blk = blockIdx.x, tid = threadIdx.x;
  const int start = blk * kCH;
  const int end = min(a.V, start + kCH);
  const RowParams p = row_params(a, row);
  RowCtl* c = a.ctl + row;
  if (ROLE == 1 && p.kind != kMass) return;
  if (ROLE == 0 && (p.kind == kMass || p.kind == kSingle)) return;
#ifdef QS_TRACE
  if (tid == 0) sc.tslot = (u32)(row * a.G + blk);
#endif
  QS_TR(0);

  // token (v, j) of this thread is start + (v * 256 + tid) * VW + j, inside the
  // row iff j < lim[v]
  int lim[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) lim[v] = (end - start) - (v * kThreads + tid) * VW;

  if constexpr (ROLE == 0) {
    // ================================================================ greedy
    if (p.kind == kGreedy) {
      float z[kEPT];
      load_chunk_pen<DT>(a, p, row, start, end, z, lds, sc);
      QS_TR(1);
      // this thread's tokens in increasing id: the first of the largest keys
      u32 bk = 0u;
      int bi = -1;
#pragma unroll
      for (int i = 0; i < kEPT; ++i) {
        const u32 gk = gkey(z[i]);
        const bool take = (i % VW) < lim[i / VW] && (bi < 0 || gk > bk);
        bk = take ? gk : bk;
        bi = take ? i : bi;
      }
      const u32 be = (u32)(start + ((bi / VW) * kThreads + tid) * VW + (bi % VW));
      u64 best = bi < 0 ? 0ull : (((u64)bk << 32) | (0xffffffffu - be));
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
    // tau: at least kc tokens of the chunk are >= tau, kc covering this chunk's
    // expected share of the row's top-k with a wide margin.  Each wave takes
    // the ceil(kc/4)-th largest of its 64 per-thread maxima (a bit-by-bit
    // search on ballot counts); the workgroup takes the smallest of the four.
    float z[kEPT];
    load_chunk_pen<DT>(a, p, row, start, end, z, lds, sc);
    QS_TR(1);
    // z keys without the NaN and -0 cases of skey (3 operations): they only
    // choose which tokens are written, and a NaN or -0 among them can only make
    // the written set look incomplete to k_finish (whose entries carry exact
    // keys of q), never wrong
    u32 kz[kEPT];
#pragma unroll
    for (int i = 0; i < kEPT; ++i) {
      const u32 u = __float_as_uint(z[i]);
      kz[i] = u ^ ((u32)((int)u >> 31) | 0x80000000u);
    }
    if (end - start < kCH) {  // the row's last chunk: tokens past the end get key 0
#pragma unroll
      for (int i = 0; i < kEPT; ++i) kz[i] = ((i % VW) < lim[i / VW]) ? kz[i] : 0u;
    }
    u32 tm = 0u;
#pragma unroll
    for (int i = 0; i < kEPT; ++i) tm = kz[i] > tm ? kz[i] : tm;
    const float mu = (float)p.k / (float)a.G;
    int kc = (int)ceilf(mu) + 4 * (int)ceilf(sqrtf(mu)) + 4;
    kc = min(kc, min(p.k, kThreads));
    const u32 kw = (u32)((kc + kWaves - 1) / kWaves);
    u32 tw = 0u;  // the largest value with at least kw thread maxima at or above it
    for (int b = 31; b >= 0; --b) {
      const u32 cand = tw | (1u << b);
      if ((u32)__popcll(__ballot(tm >= cand)) >= kw) tw = cand;
    }
    if (lane_id() == 0) sc.v[tid >> 6][6] = tw;
    __syncthreads();
    QS_TR(2);
    u32 tau = sc.v[0][6];
    for (int w = 1; w < kWaves; ++w) tau = sc.v[w][6] < tau ? sc.v[w][6] : tau;
    u32 below;
    u32 total = emit_region<DT, true>(a, row, blk, start, kz, tau, p.T, lds, sc, &below);
    if (total > (u32)a.R) {
      // too many tokens at the threshold (ties): leave those at tau out
      if (tau != 0xffffffffu) ++tau;
      total = emit_region<DT, true>(a, row, blk, start, kz, tau, p.T, lds, sc, &below);
    }
    if (tid == 0) {
      Slot* sl = a.slots + (size_t)row * a.G + blk;
      stc(&sl->nb, total <= (u32)a.R ? total : 0xffffffffu);
      stc(&sl->tau, tau);
      stc(&sl->below, below);
    }
    QS_TR(3);
    return;
  } else {
    // ================================================================ mass rows
    Slot* slots = a.slots + (size_t)row * a.G;
    // the chunk is kept as the keys of q = z / T (q = f_of_key(key) up to the
    // sign of zero); its tokens within 40 octaves of its own maximum go to its
    // region
    float z[kEPT];
    load_chunk_pen<DT>(a, p, row, start, end, z, lds, sc);
    QS_TR(1);
    u32 kz[kEPT];
    u32 kmx = 0u, nkmn = 0u, dummy = 0u;
#pragma unroll
    for (int i = 0; i < kEPT; ++i) {
      const u32 k = ((i % VW) < lim[i / VW]) ? skey(z[i] / p.T) : 0u;
      kz[i] = k;
      kmx = k > kmx ? k : kmx;
      nkmn = (k && ~k > nkmn) ? ~k : nkmn;
    }
    block_max3(kmx, nkmn, dummy, sc);
    const u32 kthr_l = window_key(octave_of(f_of_key(kmx)) - kWindow);
    u32 below;
    const u32 total = emit_region<DT, false>(a, row, blk, start, kz, kthr_l, 1.0f, lds, sc, &below);
    QS_TR(2);
    if (tid == 0) {
      const bool fits = total <= (u32)a.R;
      stc(&slots[blk].nb, fits ? total : 0xffffffffu);
      maxc(&c->kmax, kmx);
      maxc(&c->nkmin, nkmn);
      if (fits) addc(&c->cand_n, total);
      else orc(&c->status, kStOverflow);
    }
    QS_TR(3);
    row_barrier(c, (u32)a.G, 1u);
    QS_TR(4);
    const u32 rkmax = ldc(&c->kmax);
    const u32 rnkmin = ldc(&c->nkmin);
    const u32 candn = ldc(&c->cand_n);
    const u32 st = ldc(&c->status);
    const int N = octave_of(f_of_key(rkmax));
    // a timed-out barrier, or a peaked row: k_finish resolves it
    if ((st & kStTimeout) || (!(st & kStOverflow) && candn <= (u32)kFinCap)) return;
    // ---- flat row: exact weights, kept packed in registers; the chunk's mass,
    // its bin masses (high 32-bit parts) and, without top-p, its segment masses
    const float qhi = f_of_key(rkmax);
    const double yhi = y_of(qhi);
    double ylo = rnkmin ? y_of(f_of_key(~rnkmin)) : yhi;
    if (ylo < (double)(N - kWindow)) ylo = (double)(N - kWindow);
    const QBins qb = qbins_of((float)(ylo / kLog2e), qhi);
    u64* bh = (u64*)lds;        // [kBins] sums of w >> 32 per bin
    u64* gmh = bh + kBins;      // [kBins] the row's histogram, read back
    bh[tid] = 0ull;
    __syncthreads();
    u64 vlo[NV];
    u32 vhi[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      vlo[v] = 0ull;
      vhi[v] = 0u;
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const int i = v * VW + j;
        u32 ki = kz[i];
        asm volatile("" : "+v"(ki));
        const float q = f_of_key(ki);
        const u64 w = ki ? wunpack(wpack(q, N)) : 0ull;
        vlo[v] += w;
        vhi[v] += vlo[v] < w ? 1u : 0u;
        if (p.topp_on && (w >> 32)) atomicAdd(&bh[qb.bin(q)], w >> 32);
      }
    }
    u128 tsum = 0;
#pragma unroll
    for (int v = 0; v < NV; ++v) tsum += mk128(vlo[v], vhi[v]);
    const u128 acc = block_sum128(tsum, sc);  // its barriers also order the LDS atomics
    if (tid == 0) {
      stc(&slots[blk].s_lo, (u64)acc);
      stc(&slots[blk].s_hi, (u64)(acc >> 64));
    }
    QS_TR(5);
    u64* sgm = a.segm + ((size_t)row * a.G + blk) * (2 * kSegs);
    if (!p.topp_on) {
      // plain draw: the segment masses let k_finish find the token
      store_segments<NV>(sgm, vlo, vhi);
      return;
    }
    u64* gh = a.mhist + (size_t)row * kBins;
    if (bh[tid]) addc(&gh[tid], bh[tid]);
    row_barrier(c, (u32)a.G, 2u);
    QS_TR(6);
    // every workgroup: the total mass, the target and the bracket of bins
    u128 sv = 0;
    if (tid < a.G) sv = mk128(ldc(&slots[tid].s_lo), ldc(&slots[tid].s_hi));
    gmh[tid] = ldc(&gh[tid]);
    const u128 S = block_sum128(sv, sc);  // its barriers also publish gmh
    const u128 Tp = mul_frac(S, p.tp);
    int blo, bhi;
    bracket_bins(gmh, (u64)a.V, Tp, 32, sc, &blo, &bhi);
    if (blk == 0 && tid == 0) {
      stc(&c->tp_lo, (u64)Tp);
      stc(&c->tp_hi, (u64)(Tp >> 64));
      stc(&c->flat_blo, (u32)blo);
    }
    const u32 kwin = window_key(N - kWindow);  // the tokens with weight: keys >= kwin
    // this chunk: exact mass above the bracket per segment; its bracketed
    // tokens, aggregated by (key, segment), appended to the row's list.  Each
    // wave stages its bracketed tokens in its own quarter of `stg` (ballot
    // positions, no atomics).
    u64* stg = (u64*)(gmh + kBins);  // [kStage2] key << 32 | segment + 1
    u64* hk = stg + kStage2;         // [kHash] hash table: key << 32 | segment + 1
    u32* hc = (u32*)(hk + kHash);    //                     count
    for (int i = tid; i < kHash; i += kThreads) {
      hk[i] = 0ull;
      hc[i] = 0u;
    }
    constexpr u32 kQ = kStage2 / kWaves;
    const u32 wbase = (u32)(tid >> 6) * kQ;
    u32 run = 0u;  // this wave's bracketed tokens so far
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      vlo[v] = 0ull;
      vhi[v] = 0u;
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const int i = v * VW + j;
        u32 ki = kz[i];
        asm volatile("" : "+v"(ki));  // recomputed here: keeping 32 weights from the last pass costs registers
        const float q = f_of_key(ki);
        const int b = qb.bin(q);
        const u64 w = (ki >= kwin && b > bhi) ? wunpack(wpack(q, N)) : 0ull;
        vlo[v] += w;
        vhi[v] += vlo[v] < w ? 1u : 0u;
        const bool in = ki >= kwin && b >= blo && b <= bhi;
        const u64 bal = __ballot(in);
        if (bal) {
          const u32 r = run + __builtin_amdgcn_mbcnt_hi((u32)(bal >> 32), __builtin_amdgcn_mbcnt_lo((u32)bal, 0u));
          if (in && r < kQ) stg[wbase + r] = ((u64)ki << 32) | (u32)(v * kWaves + (tid >> 6) + 1);
          run += (u32)__popcll(bal);
        }
      }
    }
    store_segments<NV>(sgm, vlo, vhi);
    u128 asum = 0;
#pragma unroll
    for (int v = 0; v < NV; ++v) asum += mk128(vlo[v], vhi[v]);
    if (lane_id() == 0) sc.v[tid >> 6][5] = run;  // read after block_sum128's first barrier
    const u128 above = block_sum128(asum, sc);  // its barriers also publish the staging
    u32 nbt = 0u, sovf = 0u;
    for (int w = 0; w < kWaves; ++w) {
      const u32 n = sc.v[w][5];
      nbt += n;
      sovf |= n > kQ ? 1u : 0u;
    }
    for (int w = 0; w < kWaves; ++w) {
      const u32 n = min(sc.v[w][5], kQ);
      for (u32 t = tid; t < n; t += kThreads) {
        const u64 hkey = stg[w * kQ + t];
        u32 h = (((u32)(hkey >> 32)) ^ ((u32)hkey << 27)) * 0x9E3779B1u >> 22;  // kHash = 1024 slots
        for (int probe = 0; probe < kHash; ++probe) {
          const u64 prev = atomicCAS((unsigned long long*)&hk[h], 0ull, (unsigned long long)hkey);
          if (prev == 0ull || prev == hkey) {
            atomicAdd(&hc[h], 1u);
            break;
          }
          h = (h + 1u) & (u32)(kHash - 1);
        }
      }
    }
    __syncthreads();
    // (key, segment) counts: this chunk's own list, read by k_finish for the
    // chunk holding the draw or the boundary token
    u32 ne = 0u;
#pragma unroll
    for (int q = 0; q < kHash / kThreads; ++q) ne += hc[tid * (kHash / kThreads) + q] ? 1u : 0u;
    u32 nes;
    u32 o = block_scan_u32(ne, sc, &nes);
    const bool sfit = !sovf && nes <= (u32)kSegEnt;
    u64* sent = a.sent + ((size_t)row * a.G + blk) * kSegEnt;
    // then per key (the staging area becomes a second table): the row's list
    u64* hk2 = stg;                 // [kHash] key + 1... as key << 32 | 1
    u32* hc2 = (u32*)(hk2 + kHash); // [kHash] count
    for (int i = tid; i < kHash; i += kThreads) {
      hk2[i] = 0ull;
      hc2[i] = 0u;
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kHash / kThreads; ++q) {
      const int h = tid * (kHash / kThreads) + q;
      const u32 n = hc[h];
      if (n) {
        const u64 hkey = hk[h];
        const u32 key = (u32)(hkey >> 32);
        if (sfit) sent[o++] = ((u64)key << 32) | ((((u32)hkey - 1u) & 31u) << 16) | n;
        const u64 k2 = ((u64)key << 32) | 1u;
        u32 h2 = (key * 0x9E3779B1u) >> 22;  // kHash = 1024 slots
        for (int probe = 0; probe < kHash; ++probe) {
          const u64 prev = atomicCAS((unsigned long long*)&hk2[h2], 0ull, (unsigned long long)k2);
          if (prev == 0ull || prev == k2) {
            atomicAdd(&hc2[h2], n);
            break;
          }
          h2 = (h2 + 1u) & (u32)(kHash - 1);
        }
      }
    }
    __syncthreads();
    u32 nk = 0u;
#pragma unroll
    for (int q = 0; q < kHash / kThreads; ++q) nk += hc2[tid * (kHash / kThreads) + q] ? 1u : 0u;
    u32 net;
    const u32 neoff = block_scan_u32(nk, sc, &net);
    if (tid == 0) {
      stc(&slots[blk].a_lo, (u64)above);
      stc(&slots[blk].a_hi, (u64)(above >> 64));
      stc(&slots[blk].nbr, nbt);
      stc(&slots[blk].nse, sfit ? nes : 0xffffffffu);
      if (sovf) orc(&c->status, kStList);
      sc.r[12] = net ? addc(&c->list_n, net) : 0u;
    }
    __syncthreads();
    const u32 base = sc.r[12];
    if (net && !sovf && (u64)base + net <= (u64)kListCap) {
      u64* lst = a.list + (size_t)row * kListCap + base + neoff;
      u32 o2 = 0u;
#pragma unroll
      for (int q = 0; q < kHash / kThreads; ++q) {
        const int h = tid * (kHash / kThreads) + q;
        const u32 n = hc2[h];
        if (n) {
          u32* ent = (u32*)&lst[o2];
          stc(&ent[0], ((u32)blk << 16) | n);
          stc(&ent[1], (u32)(hk2[h] >> 32));
          ++o2;
        }
      }
    }
    QS_TR(7);
  }
}

// ---------------------------------------------------------------- finishing kernel

// One workgroup per row, after k_sample of the same ROLE: resolves the rows
// k_sample left open and returns their counters to zero.
//   ROLE 0: top-k rows from the regions; rows with large k, and mass rows when
//           no mass launch runs, by resolve_single.
//   ROLE 1: mass rows: peaked rows from the regions, flat rows from the
//           bracketed tokens and the chunk holding the draw.
template <int DT, int ROLE>
__global__ __launch_bounds__(kThreads) void k_finish(Args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ Scratch sc;
  const int row = blockIdx.x;
  const RowParams p = row_params(a, row);
  RowCtl* c = a.ctl + row;
#ifdef QS_TRACE
  if (threadIdx.x == 0) sc.tslot = (u32)(a.B * a.G + row);
#endif
  if (ROLE == 0) {
    if (p.kind == kGreedy || (p.kind == kMass && !(a.flags & QS_FLAG_NO_MASS_ROWS))) return;
    QS_TR(0);
    if (p.kind == kTopK) {
      if (!finish_row<true>(a, p, row, 0u, lds, sc)) resolve_single<DT>(a, p, row, lds, sc);
    } else {
      give_up(a, row, kWhyLargeK);
      resolve_single<DT>(a, p, row, lds, sc);
    }
    reset_row(a, row);
    QS_TR(15);
    return;
  }
  if (p.kind != kMass) return;
  QS_TR(0);
  const u32 st = ldc(&c->status);
  const u32 candn = ldc(&c->cand_n);
  const int N = octave_of(f_of_key(ldc(&c->kmax)));
  bool hist = false;
  if (st & kStTimeout) {
    give_up(a, row, kWhyTimeout);
    resolve_single<DT>(a, p, row, lds, sc);
  } else if (!(st & kStOverflow) && candn <= (u32)kFinCap) {
    if (!finish_row<false>(a, p, row, window_key(N - kWindow), lds, sc)) resolve_single<DT>(a, p, row, lds, sc);
  } else {
    hist = p.topp_on;
    const u128 Tp = p.topp_on ? mk128(ldc(&c->tp_lo), ldc(&c->tp_hi)) : (u128)0;
    const bool bottom = !p.topp_on || ldc(&c->flat_blo) == 0u;
    if (!resolve_flat<DT>(a, p, row, N, p.topp_on, Tp, bottom, lds, sc)) resolve_single<DT>(a, p, row, lds, sc);
  }
  reset_row(a, row, hist);
  QS_TR(15);
}

// ---------------------------------------------------------------- probabilities

template <int DT>
__global__ __launch_bounds__(kThreads) void k_probs(Args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ Scratch sc;
  const int row = blockIdx.y, blk = blockIdx.x;
  const int start = blk * kCH, end = min(a.V, start + kCH);
  RowCtl* c = a.ctl + row;
  const RowParams p = row_params(a, row);
  PenTable pt;
  pt.bits = (u32*)lds;
  pt.wpre = pt.bits + (kCH >> 5);
  pt.cnts = pt.wpre + (kCH >> 5);
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
  int G, R, logR, seg_cap, Hpad;
  size_t off_ctl, off_cand, off_hist, off_list, off_slots, off_segm, off_sent, total;
  size_t lds_sample, lds_finish;
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

Layout layout_for(int B, int V, int H) {
  Layout L;
  L.G = (V + kCH - 1) / kCH;
  // region capacity: the largest power of two with G * R <= kRegionTotal and
  // R <= kStageCap (a region is staged in LDS before it is written)
  L.R = 1;
  L.logR = 0;
  while (L.G * (L.R * 2) <= kRegionTotal && L.R * 2 <= kStageCap) {
    L.R *= 2;
    ++L.logR;
  }
  L.seg_cap = H > 0 ? (H < kCH ? H : kCH) : 0;
  L.Hpad = 1;
  while (L.Hpad < H) L.Hpad <<= 1;
  size_t o = 0;
  L.off_ctl = o;
  o = align_up(o + (size_t)B * sizeof(RowCtl), 256);
  L.off_cand = o;
  o = align_up(o + (size_t)B * L.G * L.R * 16, 256);
  L.off_hist = o;
  o = align_up(o + (size_t)B * kBins * 8, 256);
  L.off_list = o;
  o = align_up(o + (size_t)B * kListCap * 8, 256);
  L.off_slots = o;
  o = align_up(o + (size_t)B * L.G * sizeof(Slot), 256);
  L.off_segm = o;
  o = align_up(o + (size_t)B * L.G * kSegs * 16, 256);
  L.off_sent = o;
  o = align_up(o + (size_t)B * L.G * kSegEnt * 8, 256);
  L.total = o;
  const size_t pen = H > 0 ? (size_t)(2 * (kCH / 32) + L.seg_cap) * 4 : 0;
  const size_t fin = kHoffBytes + sizeof(WideLds) + 2 * sizeof(SelLds);  // finish_row
  const size_t flat = sizeof(FlatLds) + pen;  // the penalty table follows FlatLds
  const size_t single = sizeof(SingleLds) + (H > 0 ? (size_t)L.Hpad * 4 : 0);
  size_t bins = (size_t)2 * kBins * 8 + (size_t)kStage2 * 8 + (size_t)kHash * (8 + 4);  // flat mass rows in k_sample
  if ((size_t)L.R * 8 > bins) bins = (size_t)L.R * 8;                // region staging
  L.lds_sample = pen > bins ? pen : bins;
  L.lds_finish = pen;
  if (fin > L.lds_finish) L.lds_finish = fin;
  if (flat > L.lds_finish) L.lds_finish = flat;
  if (single > L.lds_finish) L.lds_finish = single;
  return L;
}

// k_sample then, unless every row is greedy, k_finish, on one stream.
template <int DT, int ROLE>
hipError_t launch_role(const Args& a, const Layout& L, bool finish, hipStream_t st) {
  hipLaunchKernelGGL((k_sample<DT, ROLE>), dim3(a.G, a.B), dim3(kThreads), L.lds_sample, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !finish) return e;
  hipLaunchKernelGGL((k_finish<DT, ROLE>), dim3(a.B), dim3(kThreads), L.lds_finish, st, a);
  return hipGetLastError();
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
  if ((V + kCH - 1) / kCH > kMaxChunks) return fail("qs_sample: V too large for the chunking%s");
  const Layout L = layout_for(B, V, Heff);
  if (ws_bytes < L.total) return fail("qs_sample: workspace too small (see qs_workspace_bytes)%s");
  if (((uintptr_t)ws) % 256) return fail("qs_sample: workspace must be 256-byte aligned%s");
  const bool all_greedy = (flags & QS_FLAG_ALL_GREEDY) != 0;
  if (!all_greedy && !uniforms) return fail("qs_sample: uniforms required unless all rows are greedy%s");
  if (L.lds_sample > 64 * 1024 || L.lds_finish > 64 * 1024) return fail("qs_sample: LDS budget exceeded%s");

  Args a;
  memset(&a, 0, sizeof(a));
  a.logits = logits;
  a.row_stride = row_stride;
  a.B = B;
  a.V = V;
  a.H = Heff;
  a.G = L.G;
  a.R = L.R;
  a.logR = L.logR;
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
  a.cand = (uint4*)(base + L.off_cand);
  a.mhist = (u64*)(base + L.off_hist);
  a.list = (u64*)(base + L.off_list);
  a.slots = (Slot*)(base + L.off_slots);
  a.segm = (u64*)(base + L.off_segm);
  a.sent = (u64*)(base + L.off_sent);
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
    e = dtype == QS_DTYPE_F32 ? launch_role<QS_DTYPE_F32, 1>(a, L, true, side->stream)
                              : launch_role<QS_DTYPE_BF16, 1>(a, L, true, side->stream);
    if (e != hipSuccess) return fail("qs_sample: mass kernel launch failed: %s", hipGetErrorString(e));
  }
  e = dtype == QS_DTYPE_F32 ? launch_role<QS_DTYPE_F32, 0>(a, L, !all_greedy, stream)
                            : launch_role<QS_DTYPE_BF16, 0>(a, L, !all_greedy, stream);
  if (e != hipSuccess) return fail("qs_sample: kernel launch failed: %s", hipGetErrorString(e));
  if (mass) {
    e = hipEventRecord(side->join, side->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(stream, side->join, 0);
    if (e != hipSuccess) return fail("qs_sample: join failed: %s", hipGetErrorString(e));
  }
  if (out_probs) {
    const size_t plds = Heff > 0 ? (size_t)(2 * (kCH / 32) + L.seg_cap) * 4 : 16;
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

int qs_version(void) { return 300; }

#ifdef QS_TRACE
// Trace builds only: device buffer of [B * G + B, 16] u64 wall-clock stamps
// (k_sample workgroups, then k_finish rows).
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
