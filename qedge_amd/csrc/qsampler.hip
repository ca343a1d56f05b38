// qsampler: decode-step token sampler for MI355X (gfx950).
//
// Replaces BatchSampler.forward (src/compute/sampler.py:25-41) behind the
// ModelRunner._sample_gpu call site (src/compute/model_runner.py:77-93) and the
// greedy argmax sites (src/compute/model_runner.py:85,353).  The arithmetic
// contract is stated in include/qsampler.h; ids are exact integers.
//
// Grid (G chunks, rows); each workgroup streams one chunk of 8192 logits of a
// row (2048 in batches of at most 8 rows) into registers once (16-byte loads)
// and applies the history penalties from an LDS table.  Rows are greedy,
// top-k (0 < k <= QS_TOPK_FAST_MAX) or mass rows (top-k off).  A batch of at
// most 64 rows with mass rows is one streaming launch (k_sample_all, at 512
// threads: grid rows for the mass rows first, then the batch's own rows) and
// one finishing launch (k_finish_all, one workgroup per row), on the caller's
// stream; small batches finish each row inside the streaming launch (its
// last workgroup to arrive).  Larger batches run the mass rows and the other
// rows as two launches on two streams (k_sample then k_finish, per role).
//   greedy rows  local argmax, one 64-bit atomic max per workgroup, the last
//                workgroup to arrive publishes the id.
//   top-k rows   every workgroup writes the tokens at or above a threshold
//                taken from its per-thread maxima, in id order, to its own
//                region; the finisher gathers the regions into registers
//                (still in id order) and resolves top-k, top-p and the draw
//                with register radix selects over LDS histograms.
//   mass rows    every workgroup writes the tokens within 40 octaves of its
//                own maximum; one row barrier exchanges the row maximum and
//                the counts.  A peaked row (few such tokens) is then resolved
//                by one workgroup like a top-k row.  A flat row stays
//                cooperative: exact weights, per-bin masses, a second row
//                barrier for the global histogram and the total mass, the
//                bracket of bins holding the top-p boundary, the bracketed
//                tokens listed; the finisher resolves the boundary exactly,
//                finds the chunk holding the draw and re-reads one segment of
//                it to locate the token in id order.
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

constexpr int kCHLarge = 8192;                    // logits per chunk (one k_sample workgroup)
constexpr int kCHSmall = 2048;                    // the same for batches of at most kSmallChunkMaxB rows
constexpr int kSmallChunkMaxB = 8;
constexpr int kWindow = 40;
constexpr double kYClamp = 1073741824.0;  // 2^30
constexpr double kLog2e = 1.4426950408889634074;
constexpr int kTopkFast = QS_TOPK_FAST_MAX;
constexpr int kRegionTotal = 8192;                // G * R <= this
constexpr int kStageCap = 1024;                   // region entries staged in LDS by one workgroup
constexpr int kHoffBytes = 2048;                  // finish_row: region offsets ahead of the histogram
constexpr int kFinCap = 4096;                     // region entries gathered per row; bracket entries per row
constexpr int kSmallMax = 256;                    // finish_small: members, one per thread
constexpr int kSmallPre = 64;                     // top-k rows with more members are pre-filtered
constexpr int kFusedMaxB = 8;                     // batches up to this size finish rows inside k_sample
constexpr int kOneLaunchMaxB = 64;                // batches up to this size with mass rows: one k_sample_all launch
constexpr int kMassSlots = 8;                     // k_sample_all: grid rows for mass rows ahead of the batch's rows
constexpr int kBins = 256;                        // histogram bins
constexpr int kWBins = 1024;                      // flat mass rows: packed-weight bins
constexpr int kWideBits = 11;                     // finishing histogram: 2048 bins
constexpr int kWide = 1 << kWideBits;
constexpr int kListCap = kFinCap;                 // bracket entries per row (flat mass rows)
constexpr int kHash = 1024;                       // (key, segment) hash slots per chunk (flat mass rows)
constexpr int kStage2 = 2048;                     // bracketed tokens staged per chunk (flat mass rows)
constexpr int kSegEnt = 512;                      // (key, segment) entries per chunk (flat mass rows)
constexpr int kSegs = 32;                         // segments per chunk, at most (64 * VW tokens each)
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
  u32 arrive;      // arrival lines all of whose workgroups are done (see arrive_last)
  u32 bar_unused;  // (row barriers count in Args::bars)
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
  u32 flat_blo;    // flat mass rows: 1 if tokens with weight lie below the boundary's bin
  u32 why;         // why the last fallback to resolve_single was taken (kWhy*), 0 if none
  u32 pad1[31];
};
static_assert(sizeof(RowCtl) == 256, "row control block is 256 bytes");
constexpr int kCtlZeroWords = 16;
constexpr int kSubLines = 8;  // cache lines a row's barrier and arrival counters are spread over

// Per-(row, workgroup) published values.
struct __attribute__((aligned(64))) Slot {
  u64 s_lo, s_hi;  // mass rows: exact mass of the chunk
  u64 a_lo, a_hi;  // flat mass rows: exact mass of the chunk's tokens above the bracket
  u32 nb;          // tokens written to the region (0xffffffff: more than fit)
  u32 tau;         // top-k rows: the region's threshold (z key)
  u32 below;       // top-k rows: largest z key below tau in the chunk
  u32 nbr;         // flat mass rows: bracketed tokens of the chunk
  u32 nse;         // flat mass rows: (key, segment) entries of the chunk (0xffffffff: more than fit)
  u32 kmx;         // mass rows: the chunk's largest key of q
  u32 nkmn;        // mass rows: ~ its smallest key of q (over tokens with a key)
  u32 pad;
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
  u64* cand;   // [B, G, R] region entries (key of q) << 32 | id
  u64* mhist;  // [B, kWBins] flat mass rows: the row's sums of mantissas per bin
  u64* list;   // [B, kListCap] bracket entries (key << 32 | chunk << 16 | count), flat mass rows
  u64* sent;   // [B, G, kSegEnt] per chunk: bracket entries (key << 32 | segment << 16 | count), flat mass rows
  u64* segm;   // [B, G, kSegs, 2] flat mass rows: exact mass per segment (above the bracket with top-p), lo, hi
  Slot* slots; // [B, G]
  u32* bars;    // [B, 2, kSubLines, 32]: row-barrier and arrival counters, one per cache line
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
// A 16-byte entry as two device-coherent 8-byte accesses.
__device__ __forceinline__ void stc_u4(uint4* p, uint4 v) {
  stc((u64*)p, ((u64)v.y << 32) | v.x);
  stc((u64*)p + 1, ((u64)v.w << 32) | v.z);
}
__device__ __forceinline__ uint4 ldc_u4(const uint4* p) {
  const u64 a = ldc((const u64*)p), b = ldc((const u64*)p + 1);
  return make_uint4((u32)a, (u32)(a >> 32), (u32)b, (u32)(b >> 32));
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
// wpack without branches (selects only), so that the streaming passes can
// interleave the fp64 chains of their 32 tokens; `valid` false gives 0.  Same
// value as wpack for every input.
__device__ __forceinline__ u32 wpack_nb(float q, int N, bool valid) {
  double y = (double)q * kLog2e;
  y = (y >= -kYClamp) ? y : -kYClamp;  // also NaN -> -kYClamp, as y_of
  y = (y > kYClamp) ? kYClamp : y;
  const double fl = floor(y);
  const int n = (int)fl;
  float pf = exp2_poly((float)(y - fl));
  pf = fminf(fmaxf(pf, 1.0f), __uint_as_float(0x3fffffffu));  // mant24's clamps
  const u32 wp = ((u32)(n - N + kWindow) << 24) | (0x800000u | (__float_as_uint(pf) & 0x7fffffu));
  return (valid && n >= N - kWindow) ? wp : 0u;
}
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
// z / b for a row-constant b, with r = 1 / b (correctly rounded): Markstein's
// correction of q0 = z * r by the exact residual fma(-q0, b, z).  It equals
// the correctly rounded z / b whenever div_fast_ok holds (|z| and |q0| in
// [2^-100, 2^100)): checked against the division for every fp32 z and 23
// divisors from 1.2e-36 to 3.4e37, and for 1e9 random (z, b) pairs.
__device__ __forceinline__ float div_fast(float z, float b, float r) {
  const float q0 = z * r;
  const float e = __builtin_fmaf(-q0, b, z);
  return __builtin_fmaf(e, r, q0);
}
__device__ __forceinline__ bool div_fast_ok(float z, float r) {
  const u32 aq = __float_as_uint(z * r) & 0x7fffffffu, az = __float_as_uint(z) & 0x7fffffffu;
  return (aq - 0x0d800000u) < (0x71800000u - 0x0d800000u) && (az - 0x0d800000u) < (0x71800000u - 0x0d800000u);
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

// The device code, written against the workgroup width kThreads (every
// launch uses 256 threads: 4 waves of 64, 32 logits per thread).
namespace w256 {
constexpr int kCH = kCHLarge;
constexpr int kThreads = 256;
#include "qsampler_body.inc"
}  // namespace w256
// Small batches: four times the workgroups per row, a quarter of the logits
// per thread (the same code).
namespace n2k {
constexpr int kCH = kCHSmall;
constexpr int kThreads = 256;
#include "qsampler_body.inc"
}  // namespace n2k
// The same chunks as w256 with twice the threads (16 logits per thread), for
// launches with few busy workgroups per row, whose phases are latency chains:
// the mass rows' cooperative passes and the one-workgroup-per-row finishers.
namespace w512 {
constexpr int kCH = kCHLarge;
constexpr int kThreads = 512;
#include "qsampler_body.inc"
}  // namespace w512

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

// Device-code builds: chunk size and workgroup width.
enum Ns : int { kNsW256 = 0, kNsN2K = 1, kNsW512 = 2 };
constexpr int ns_threads(int ns) { return ns == kNsW512 ? 512 : 256; }

struct Layout {
  bool small;  // kCHSmall chunks (the n2k kernels)
  int kch, G, R, logR, seg_cap, Hpad;
  size_t off_ctl, off_cand, off_hist, off_list, off_slots, off_segm, off_sent, off_bars, total;
  size_t lds_sample0, lds_sample1;  // k_sample of greedy and top-k rows, of mass rows
  int ns_sample[2], ns_finish[2];  // builds of k_sample and k_finish, per role
  size_t lds_finish[3];                   // k_finish (and a fused k_sample's tail), per build
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Small batches whose rows fit kMaxChunks small chunks use them.
bool small_chunks(int B, int V) { return B <= kSmallChunkMaxB && (V + kCHSmall - 1) / kCHSmall <= kMaxChunks; }

template <typename NS_WIDE, typename NS_SEL, typename NS_FLAT, typename NS_SINGLE>
struct LdsSizes {
  static constexpr size_t wide = sizeof(NS_WIDE), sel = sizeof(NS_SEL), flat = sizeof(NS_FLAT),
                          single = sizeof(NS_SINGLE);
};
using LdsLarge = LdsSizes<w256::WideLds, w256::SelLds, w256::FlatLds, w256::SingleLds>;
using LdsSmall = LdsSizes<n2k::WideLds, n2k::SelLds, n2k::FlatLds, n2k::SingleLds>;
using LdsW512 = LdsSizes<w512::WideLds, w512::SelLds, w512::FlatLds, w512::SingleLds>;

// LDS of the finishing code of build `ns` (finish_row, resolve_flat,
// resolve_single), with `pen` bytes of penalty table and a history of Hpad ids.
template <typename LS>
size_t finish_lds(size_t pen, int H, int Hpad) {
  const size_t fin = kHoffBytes + LS::wide + 2 * LS::sel;  // finish_row
  const size_t flat = LS::flat + pen;                      // the penalty table follows FlatLds
  const size_t single = LS::single + (H > 0 ? (size_t)Hpad * 4 : 0);
  size_t r = pen;
  if (fin > r) r = fin;
  if (flat > r) r = flat;
  if (single > r) r = single;
  return r;
}

Layout layout_for(int B, int V, int H) {
  Layout L;
  L.small = small_chunks(B, V);
  L.kch = L.small ? kCHSmall : kCHLarge;
  L.G = (V + L.kch - 1) / L.kch;
  // region capacity: the largest power of two with G * R <= kRegionTotal and
  // R <= kStageCap (a region is staged in LDS before it is written)
  L.R = 1;
  L.logR = 0;
  while (L.G * (L.R * 2) <= kRegionTotal && L.R * 2 <= kStageCap) {
    L.R *= 2;
    ++L.logR;
  }
  L.seg_cap = H > 0 ? (H < L.kch ? H : L.kch) : 0;
  L.Hpad = 1;
  while (L.Hpad < H) L.Hpad <<= 1;
  size_t o = 0;
  L.off_ctl = o;
  o = align_up(o + (size_t)B * sizeof(RowCtl), 256);
  L.off_cand = o;
  o = align_up(o + (size_t)B * L.G * L.R * 8, 256);
  L.off_hist = o;
  o = align_up(o + (size_t)B * kWBins * 8, 256);
  L.off_list = o;
  o = align_up(o + (size_t)B * kListCap * 8, 256);
  L.off_slots = o;
  o = align_up(o + (size_t)B * L.G * sizeof(Slot), 256);
  L.off_segm = o;
  o = align_up(o + (size_t)B * L.G * kSegs * 16, 256);
  L.off_sent = o;
  o = align_up(o + (size_t)B * L.G * kSegEnt * 8, 256);
  L.off_bars = o;
  o = align_up(o + (size_t)B * 2 * kSubLines * 128, 256);
  L.total = o;
  const size_t pen = H > 0 ? (size_t)L.kch * 2 : 0;  // 16-bit history counts of one chunk
  L.lds_finish[kNsW256] = finish_lds<LdsLarge>(pen, H, L.Hpad);
  L.lds_finish[kNsN2K] = finish_lds<LdsSmall>(pen, H, L.Hpad);
  L.lds_finish[kNsW512] = finish_lds<LdsW512>(pen, H, L.Hpad);
  // Builds of the per-role launches (batches with mass rows of at most
  // kOneLaunchMaxB rows use k_sample_all instead).  Small batches: small
  // chunks throughout.  Otherwise the streaming passes keep 32 logits per
  // thread (many workgroups, loads in flight), while the top-k finisher (one
  // workgroup per row) runs twice as many threads.
  L.ns_sample[0] = L.small ? kNsN2K : kNsW256;
  L.ns_sample[1] = L.small ? kNsN2K : kNsW256;
  L.ns_finish[0] = L.small ? kNsN2K : kNsW512;
  L.ns_finish[1] = L.small ? kNsN2K : kNsW256;
  size_t bins = (size_t)kWBins * 8 + (size_t)kStage2 * 8 + (size_t)kHash * (8 + 4);  // flat mass rows in k_sample
  if ((size_t)L.R * 8 > bins) bins = (size_t)L.R * 8;                // region staging
  const size_t stage = (size_t)L.R * 8;  // region staging
  L.lds_sample0 = pen > stage ? pen : stage;
  L.lds_sample1 = L.lds_sample0 > bins ? L.lds_sample0 : bins;
  return L;
}

// The builds a per-role launch can use: k_sample n2k or w256; k_finish of
// top-k rows n2k or w512, of mass rows n2k or w256.
template <int DT, int ROLE, bool FUSED>
const void* sample_kernel(int ns) {
  if (ns == kNsN2K) return (const void*)n2k::k_sample<DT, ROLE, FUSED>;
  return (const void*)w256::k_sample<DT, ROLE, FUSED>;
}
template <int DT, int ROLE>
const void* finish_kernel(int ns) {
  if (ns == kNsN2K) return (const void*)n2k::k_finish<DT, ROLE>;
  if constexpr (ROLE == 1) return (const void*)w256::k_finish<DT, ROLE>;
  else return (const void*)w512::k_finish<DT, ROLE>;
}
template <int DT>
const void* probs_kernel(int ns) {
  if (ns == kNsN2K) return (const void*)n2k::k_probs<DT>;
  return (const void*)w256::k_probs<DT>;
}

hipError_t launch(const void* fn, dim3 grid, int ns, size_t lds, hipStream_t st, const Args& a) {
  void* args[] = {(void*)&a};
  return hipLaunchKernel(fn, grid, dim3(ns_threads(ns)), args, lds, st);
}

// k_sample then, unless every row is greedy, k_finish, on one stream; with
// `fused` (small batches) k_sample's last workgroup of each row finishes it
// instead, which saves the second launch.  256-thread workgroups.
template <int DT, int ROLE>
hipError_t launch_role(const Args& a, const Layout& L, bool finish, bool fused, hipStream_t st) {
  const size_t lds = ROLE == 0 ? L.lds_sample0 : L.lds_sample1;
  const int ns = L.ns_sample[ROLE];
  if constexpr (ROLE == 0) {  // mass rows are fused only inside k_sample_all
    if (fused) {
      const size_t lf = lds > L.lds_finish[ns] ? lds : L.lds_finish[ns];
      return launch(sample_kernel<DT, ROLE, true>(ns), dim3(a.G, a.B), ns, lf, st, a);
    }
  }
  hipError_t e = launch(sample_kernel<DT, ROLE, false>(ns), dim3(a.G, a.B), ns, lds, st, a);
  if (e != hipSuccess || !finish) return e;
  const int nf = L.ns_finish[ROLE];
  return launch(finish_kernel<DT, ROLE>(nf), dim3(a.B), nf, L.lds_finish[nf], st, a);
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

// The mass rows on the caller's stream beside the other rows on the side
// stream (fork and join through events), or the other rows alone.
int launch_two(const Args& a, const Layout& L, int dtype, bool mass, bool fused, bool all_greedy,
               hipStream_t stream) {
  SideStream* side = nullptr;
  hipError_t e;
  if (mass) {
    // the mass-row launch (the longer chain of the two) goes first, on the
    // caller's stream; the other rows' launch runs beside it on a side stream,
    // forked and joined through events (capturable into a HIP graph).  A
    // launch behind the fork's event wait starts some microseconds later.
    side = side_stream();
    if (!side) return fail("qs_sample: no side stream (call qs_workspace_init first)%s");
    e = hipEventRecord(side->fork, stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(side->stream, side->fork, 0);
    if (e != hipSuccess) return fail("qs_sample: fork failed: %s", hipGetErrorString(e));
    e = dtype == QS_DTYPE_F32 ? launch_role<QS_DTYPE_F32, 1>(a, L, true, false, stream)
                              : launch_role<QS_DTYPE_BF16, 1>(a, L, true, false, stream);
    if (e != hipSuccess) return fail("qs_sample: mass kernel launch failed: %s", hipGetErrorString(e));
  }
  hipStream_t st0 = mass ? side->stream : stream;
  e = dtype == QS_DTYPE_F32 ? launch_role<QS_DTYPE_F32, 0>(a, L, !all_greedy, fused, st0)
                            : launch_role<QS_DTYPE_BF16, 0>(a, L, !all_greedy, fused, st0);
  if (e != hipSuccess) return fail("qs_sample: kernel launch failed: %s", hipGetErrorString(e));
  if (mass) {
    e = hipEventRecord(side->join, side->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(stream, side->join, 0);
    if (e != hipSuccess) return fail("qs_sample: join failed: %s", hipGetErrorString(e));
  }
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
  if ((V + kCHLarge - 1) / kCHLarge > kMaxChunks) return fail("qs_sample: V too large for the chunking%s");
  const Layout L = layout_for(B, V, Heff);
  if (ws_bytes < L.total) return fail("qs_sample: workspace too small (see qs_workspace_bytes)%s");
  if (((uintptr_t)ws) % 256) return fail("qs_sample: workspace must be 256-byte aligned%s");
  const bool all_greedy = (flags & QS_FLAG_ALL_GREEDY) != 0;
  if (!all_greedy && !uniforms) return fail("qs_sample: uniforms required unless all rows are greedy%s");
  for (int ns = 0; ns < 3; ++ns)
    if (L.lds_sample1 > 64 * 1024 || L.lds_finish[ns] > 64 * 1024) return fail("qs_sample: LDS budget exceeded%s");

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
  a.cand = (u64*)(base + L.off_cand);
  a.mhist = (u64*)(base + L.off_hist);
  a.list = (u64*)(base + L.off_list);
  a.slots = (Slot*)(base + L.off_slots);
  a.segm = (u64*)(base + L.off_segm);
  a.sent = (u64*)(base + L.off_sent);
  a.bars = (u32*)(base + L.off_bars);
#ifdef QS_TRACE
  a.trace = g_trace;
#endif

  const bool mass = !(flags & (QS_FLAG_ALL_GREEDY | QS_FLAG_NO_MASS_ROWS));
  const bool fused = B <= kFusedMaxB;  // greedy and top-k rows without mass rows
  // Batches of at most kOneLaunchMaxB rows with mass rows: one streaming
  // launch for all rows (mass rows first in its grid), on the caller's stream.
  // Small chunks finish the rows inside it; large chunks run it at 512
  // threads, followed by one finishing launch for all rows.  (Two launches on
  // two streams would overlap too, but their fork and join cost ~7 us per
  // call inside a HIP graph.)
  const bool one = mass && B <= kOneLaunchMaxB;
  hipError_t e;
  if (one && L.small) {
    size_t lds = L.lds_sample0 > L.lds_sample1 ? L.lds_sample0 : L.lds_sample1;
    if (L.lds_finish[kNsN2K] > lds) lds = L.lds_finish[kNsN2K];
    e = launch(dtype == QS_DTYPE_F32 ? (const void*)n2k::k_sample_all<QS_DTYPE_F32, true>
                                     : (const void*)n2k::k_sample_all<QS_DTYPE_BF16, true>,
               dim3(a.G, B + (B < kMassSlots ? B : kMassSlots)), kNsN2K, lds, stream, a);
    if (e != hipSuccess) return fail("qs_sample: kernel launch failed: %s", hipGetErrorString(e));
  } else if (one) {
    const size_t lds = L.lds_sample0 > L.lds_sample1 ? L.lds_sample0 : L.lds_sample1;
    e = launch(dtype == QS_DTYPE_F32 ? (const void*)w512::k_sample_all<QS_DTYPE_F32, false>
                                     : (const void*)w512::k_sample_all<QS_DTYPE_BF16, false>,
               dim3(a.G, B + (B < kMassSlots ? B : kMassSlots)), kNsW512, lds, stream, a);
    if (e == hipSuccess)
      e = launch(dtype == QS_DTYPE_F32 ? (const void*)w512::k_finish_all<QS_DTYPE_F32>
                                       : (const void*)w512::k_finish_all<QS_DTYPE_BF16>,
                 dim3(B), kNsW512, L.lds_finish[kNsW512], stream, a);
    if (e != hipSuccess) return fail("qs_sample: kernel launch failed: %s", hipGetErrorString(e));
  } else {
    if (launch_two(a, L, dtype, mass, fused, all_greedy, stream) != 0) return -1;
  }
  if (out_probs) {
    const size_t plds = Heff > 0 ? (size_t)L.kch * 2 : 16;
    const int pns = L.small ? kNsN2K : kNsW256;
    e = launch(dtype == QS_DTYPE_F32 ? probs_kernel<QS_DTYPE_F32>(pns) : probs_kernel<QS_DTYPE_BF16>(pns),
               dim3(a.G, B), pns, plds, stream, a);
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
