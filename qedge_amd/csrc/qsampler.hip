// qsampler: decode-step token sampler for MI355X (gfx950).
//
// Replaces BatchSampler.forward (src/compute/sampler.py:25-41) behind the
// ModelRunner._sample_gpu call site (src/compute/model_runner.py:77-93) and the
// greedy argmax sites (src/compute/model_runner.py:85,353).  The arithmetic
// contract is stated in include/qsampler.h; ids are exact integers.
//
// Kernels, all wave64, no MFMA (nothing here is a contraction):
//   k_main      grid (chunks, rows), 256 threads.  Streams each row chunk once
//               into registers (16-byte loads), applies history penalties from
//               an LDS bitmap, publishes the row maximum with a 64-bit atomic,
//               and for top-k rows (k <= QS_TOPK_FAST_MAX) selects the chunk's
//               local top candidates by an LDS radix select.  The last
//               workgroup of a row (arrival counter) finishes greedy rows and
//               top-k rows: merge, bitonic sort, exact top-k/top-p cut, draw.
//   k_resolve   grid (rows), 1024 threads.  Every row the main kernel could
//               not finish (top-p without a small top-k, full-vocabulary draws,
//               candidate overflow): exact radix select over the row with
//               128-bit masses, then the id-order draw.
//   k_probs     optional verification output (post-filter probabilities).
// The last kernel of a call returns the row state to zero, so the workspace
// is reusable by the next call without a memset.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/qsampler.h"

typedef unsigned __int128 u128;

namespace {

constexpr int kWindow = 40;
constexpr double kYClamp = 1073741824.0;  // 2^30
constexpr double kLog2e = 1.4426950408889634074;
constexpr int kCap = 4096;                // candidates per row (global)
constexpr int kMergeCap = 2048;           // candidates merged in LDS
constexpr int kMainThreads = 256;
constexpr int kResolveThreads = 1024;

enum : uint32_t { kPending = 0, kDone = 1, kNeedsResolve = 2 };

struct __attribute__((aligned(256))) RowState {
  unsigned long long maxpack;  // (key << 32) | (0xffffffff - id), atomicMax
  unsigned int arrive_main;
  unsigned int arrive_probs;
  unsigned int cand_count;
  unsigned int tau_max;
  unsigned int status;
  unsigned int all_emitted;
  int n_max;
  unsigned int kappa_p;  // kept: key > kappa_p || (key == kappa_p && id <= id_p)
  unsigned int id_p;
  unsigned int kept_count;
  unsigned long long w_lo, w_hi;
  long long chosen;
  unsigned int greedy;
  unsigned int pad[43];
};
static_assert(sizeof(RowState) == 256, "row state is 256 bytes");

struct Args {
  const void* logits;
  long long row_stride;
  int B, V, H, G, CH, seg_cap, nwords;
  unsigned int flags;
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
  RowState* rs;
  unsigned long long* cand;  // [B, kCap]
  unsigned int* pbits;       // [B, nwords]
  unsigned int* pwpre;       // [B, nwords], prefix within the chunk
  unsigned int* pcnt;        // [B, G, seg_cap]
  int last_kernel;           // 1 main, 2 resolve, 3 probs
};

// ---------------------------------------------------------------- contract

__device__ __forceinline__ uint32_t skey(float z) {
  if (z != z) return 0u;
  if (z == 0.0f) z = 0.0f;
  uint32_t u = __float_as_uint(z);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint32_t gkey(float z) {
  if (z != z) return 0xffffffffu;
  return skey(z);
}
__device__ __forceinline__ float z_of_key(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}
__device__ __forceinline__ double y_of(float z, double c) {
  if (z != z) return -kYClamp;
  double y = (double)z * c;
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
__device__ __forceinline__ uint32_t mant24(float p) {
  if (!(p >= 1.0f)) p = 1.0f;
  if (p >= 2.0f) p = __uint_as_float(0x3fffffffu);
  return 0x800000u | (__float_as_uint(p) & 0x7fffffu);
}
// Octave of exp(z/T): floor(y).
__device__ __forceinline__ int octave_of(float z, double c) { return (int)floor(y_of(z, c)); }
// u64 weight relative to the row scale N (0 outside the window).
__device__ __forceinline__ unsigned long long weight_of(float z, double c, int N) {
  double y = y_of(z, c);
  double fl = floor(y);
  int n = (int)fl;
  if (n < N - kWindow) return 0ull;
  uint32_t m = mant24(exp2_poly((float)(y - fl)));
  return (unsigned long long)m << (n - N + kWindow);
}
__device__ __forceinline__ u128 mul_frac(u128 x, float f) {
  if (!(f > 0.0f)) return 0;
  uint32_t b = __float_as_uint(f);
  uint32_t e = (b >> 23) & 0xffu;
  uint32_t m = b & 0x7fffffu;
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
// floor(d / w) for a quotient below 2^53 (no 128-bit division on the device).
__device__ __forceinline__ unsigned long long div_small(u128 d, unsigned long long w) {
  unsigned long long q = (unsigned long long)((double)(unsigned long long)(d >> 64) * 0x1p64 /
                                                  (double)w +
                                              (double)(unsigned long long)d / (double)w);
  while (q > 0 && (u128)q * w > d) --q;
  while ((u128)(q + 1) * w <= d) ++q;
  return q;
}
__device__ __forceinline__ double u128_to_double(u128 x) {
  unsigned long long lo = (unsigned long long)x, hi = (unsigned long long)(x >> 64);
  double d = (double)(uint32_t)(hi >> 32) * 0x1p96;
  d = d + (double)(uint32_t)hi * 0x1p64;
  d = d + (double)(uint32_t)(lo >> 32) * 0x1p32;
  d = d + (double)(uint32_t)lo;
  return d;
}
__device__ __forceinline__ float apply_penalty(float z, uint32_t c, float rep, float pres, float freq) {
  z = (z > 0.0f) ? (z / rep) : (z * rep);
  float fc = freq * (float)c;
  z = z - fc;
  z = z - pres;
  return z;
}
__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

struct RowParams {
  float T, tp, rep, pres, freq, u;
  int k;
  bool greedy, topk_on, topp_on, pen_on;
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
  return p;
}

// ---------------------------------------------------------------- block utils

template <int THREADS>
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v, unsigned long long* s) {
  for (int o = 32; o > 0; o >>= 1) {
    unsigned long long w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) s[wv] = v;
  __syncthreads();
  unsigned long long r = s[0];
  for (int i = 1; i < THREADS / 64; ++i) r = s[i] > r ? s[i] : r;
  __syncthreads();
  return r;
}

struct Acc {  // (count, 128-bit mass)
  unsigned long long lo, hi;
  unsigned int c;
};
__device__ __forceinline__ Acc acc_add(Acc a, Acc b) {
  Acc r;
  r.lo = a.lo + b.lo;
  r.hi = a.hi + b.hi + (r.lo < a.lo ? 1ull : 0ull);
  r.c = a.c + b.c;
  return r;
}
__device__ __forceinline__ u128 acc_mass(const Acc& a) { return ((u128)a.hi << 64) | a.lo; }
__device__ __forceinline__ Acc acc_of(u128 m, unsigned int c) {
  Acc r;
  r.lo = (unsigned long long)m;
  r.hi = (unsigned long long)(m >> 64);
  r.c = c;
  return r;
}

// Exclusive prefix over threads in threadIdx order; returns the exclusive value,
// writes the total to *total.  s must hold 3 * THREADS/64 + 3 u64.
template <int THREADS>
__device__ Acc block_excl_scan(Acc v, unsigned long long* s, Acc* total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  constexpr int NW = THREADS / 64;
  Acc inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    Acc t;
    t.lo = __shfl_up(inc.lo, o, 64);
    t.hi = __shfl_up(inc.hi, o, 64);
    t.c = __shfl_up(inc.c, o, 64);
    if (lane >= o) inc = acc_add(inc, t);
  }
  __syncthreads();
  if (lane == 63) {
    s[3 * wv] = inc.lo;
    s[3 * wv + 1] = inc.hi;
    s[3 * wv + 2] = inc.c;
  }
  __syncthreads();
  Acc base = {0, 0, 0}, tot = {0, 0, 0};
  for (int i = 0; i < NW; ++i) {
    Acc wt = {s[3 * i], s[3 * i + 1], (unsigned int)s[3 * i + 2]};
    if (i < wv) base = acc_add(base, wt);
    tot = acc_add(tot, wt);
  }
  __syncthreads();
  *total = tot;
  Acc excl = acc_add(base, inc);
  // excl = base + inc - v
  Acc r;
  r.lo = excl.lo - v.lo;
  r.hi = excl.hi - v.hi - (excl.lo < v.lo ? 1ull : 0ull);
  r.c = excl.c - v.c;
  return r;
}

// Bitonic sort of n (power of two) u64 values in LDS, descending.
template <int THREADS>
__device__ void bitonic_desc(unsigned long long* s, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += THREADS) {
        int ixj = i ^ j;
        if (ixj > i) {
          unsigned long long a = s[i], b = s[ixj];
          bool desc = (i & k) == 0;
          if (desc ? (a < b) : (a > b)) {
            s[i] = b;
            s[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}
template <int THREADS>
__device__ void bitonic_asc(unsigned long long* s, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += THREADS) {
        int ixj = i ^ j;
        if (ixj > i) {
          unsigned long long a = s[i], b = s[ixj];
          bool asc = (i & k) == 0;
          if (asc ? (a > b) : (a < b)) {
            s[i] = b;
            s[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ int pow2_ceil(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

template <typename T>
__device__ __forceinline__ T ld_acquire(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Row penalty tables in the workspace: count of token i (0 if not in history).
__device__ __forceinline__ uint32_t hist_count(const Args& a, int row, int i) {
  const int w = i >> 5, b = i & 31;
  const uint32_t bits = a.pbits[(size_t)row * a.nwords + w];
  if (!((bits >> b) & 1u)) return 0u;
  const int chunk = i / a.CH;
  const uint32_t slot = a.pwpre[(size_t)row * a.nwords + w] + __popc(bits & ((1u << b) - 1u));
  return a.pcnt[((size_t)row * a.G + chunk) * a.seg_cap + slot];
}

template <int DT>
__device__ __forceinline__ float load_logit(const Args& a, int row, int i) {
  if (DT == QS_DTYPE_F32) {
    return ((const float*)a.logits)[(size_t)row * a.row_stride + i];
  } else {
    return bf16_to_f32(((const uint16_t*)a.logits)[(size_t)row * a.row_stride + i]);
  }
}

// q = (penalised logit) / T for a sampling row (one IEEE fp32 division).
template <int DT>
__device__ __forceinline__ float load_z(const Args& a, const RowParams& p, int row, int i) {
  float z = load_logit<DT>(a, row, i);
  if (p.pen_on) {
    uint32_t c = hist_count(a, row, i);
    if (c) z = apply_penalty(z, c, p.rep, p.pres, p.freq);
  }
  return z / p.T;
}

// Clear a row's state (the caller is the last reader of it in this call).
__device__ __forceinline__ void clear_row(RowState* r) {
  unsigned int* w = (unsigned int*)r;
  for (int i = threadIdx.x; i < (int)(sizeof(RowState) / 4); i += blockDim.x) w[i] = 0u;
}

// Find, over nb bins given as a descending sequence (bin nb-1 first), the bin
// where the running sum of `by_count ? count : mass` passes target.  Threads
// own contiguous runs of bins.  Writes bin index, and count/mass above it.
template <int THREADS>
__device__ void find_bin(const unsigned int* cnt, const unsigned long long* mlo, const unsigned long long* mhi,
                         int nb, bool by_count, u128 target, unsigned long long* scan_s, int* out_bin,
                         Acc* out_above) {
  const int per = (nb + THREADS - 1) / THREADS;
  const int t = threadIdx.x;
  Acc loc = {0, 0, 0};
  for (int q = 0; q < per; ++q) {
    int b = nb - 1 - (t * per + q);
    if (b < 0) break;
    u128 m = mlo ? (((u128)mhi[b] << 32) + (u128)mlo[b]) : 0;
    loc = acc_add(loc, acc_of(m, cnt[b]));
  }
  Acc tot;
  Acc ex = block_excl_scan<THREADS>(loc, scan_s, &tot);
  u128 lo = by_count ? (u128)ex.c : acc_mass(ex);
  u128 sz = by_count ? (u128)loc.c : acc_mass(loc);
  if (target >= lo && target < lo + sz) {
    Acc run = ex;
    for (int q = 0; q < per; ++q) {
      int b = nb - 1 - (t * per + q);
      if (b < 0) break;
      u128 m = mlo ? (((u128)mhi[b] << 32) + (u128)mlo[b]) : 0;
      Acc nxt = acc_add(run, acc_of(m, cnt[b]));
      u128 hiv = by_count ? (u128)nxt.c : acc_mass(nxt);
      if (target < hiv) {
        *out_bin = b;
        *out_above = run;
        break;
      }
      run = nxt;
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- main kernel

struct MainShared {
  unsigned long long red[16];
  unsigned long long scan[64];
  int bin;
  Acc above;
  unsigned int counter;
  unsigned int flag;
};

template <int DT, int EPT, bool VEC>
__global__ __launch_bounds__(kMainThreads) void k_main(Args a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
  __shared__ MainShared sh;
  const int row = blockIdx.y, chunk = blockIdx.x, tid = threadIdx.x;
  const int start = chunk * a.CH;
  const int end = min(a.V, start + a.CH);
  const RowParams p = row_params(a, row);
  RowState* rs = a.rs + row;
  constexpr int VW = (DT == QS_DTYPE_F32) ? 4 : 8;
  constexpr int NV = EPT / VW;

  // ---- history penalties: bitmap + slot counts for this chunk (LDS)
  unsigned int* bits = (unsigned int*)lds;                 // CH/32
  unsigned int* wpre = bits + (a.CH >> 5);                 // CH/32
  unsigned int* cnts = wpre + (a.CH >> 5);                 // seg_cap
  const int nw = a.CH >> 5;
  if (p.pen_on) {
    for (int i = tid; i < nw; i += kMainThreads) bits[i] = 0u;
    for (int i = tid; i < a.seg_cap; i += kMainThreads) cnts[i] = 0u;
    __syncthreads();
    const int* h = a.hist + (size_t)row * a.H;
    for (int i = tid; i < a.H; i += kMainThreads) {
      int id = h[i];
      if (id >= start && id < end) atomicOr(&bits[(id - start) >> 5], 1u << ((id - start) & 31));
    }
    __syncthreads();
    {
      // exclusive prefix of popcounts over the chunk's words
      const int per = (nw + kMainThreads - 1) / kMainThreads;
      unsigned int loc = 0;
      for (int q = 0; q < per; ++q) {
        int w = tid * per + q;
        if (w < nw) loc += __popc(bits[w]);
      }
      Acc tot;
      Acc ex = block_excl_scan<kMainThreads>(Acc{0, 0, loc}, sh.scan, &tot);
      unsigned int run = ex.c;
      for (int q = 0; q < per; ++q) {
        int w = tid * per + q;
        if (w < nw) {
          wpre[w] = run;
          run += __popc(bits[w]);
        }
      }
    }
    __syncthreads();
    for (int i = tid; i < a.H; i += kMainThreads) {
      int id = h[i];
      if (id >= start && id < end) {
        int l = id - start;
        unsigned int bw = bits[l >> 5];
        unsigned int slot = wpre[l >> 5] + __popc(bw & ((1u << (l & 31)) - 1u));
        atomicAdd(&cnts[slot], 1u);
      }
    }
    __syncthreads();
    // publish the tables for later kernels
    const int wbase = start >> 5;
    for (int i = tid; i < nw && wbase + i < a.nwords; i += kMainThreads) {
      a.pbits[(size_t)row * a.nwords + wbase + i] = bits[i];
      a.pwpre[(size_t)row * a.nwords + wbase + i] = wpre[i];
    }
    unsigned int* gc = a.pcnt + ((size_t)row * a.G + chunk) * a.seg_cap;
    for (int i = tid; i < a.seg_cap; i += kMainThreads) gc[i] = cnts[i];
  }

  // ---- load the chunk into registers
  float z[EPT];
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int e0 = start + (v * kMainThreads + tid) * VW;
    if (VEC && e0 + VW <= end) {
      if (DT == QS_DTYPE_F32) {
        const float4 q = *(const float4*)((const float*)a.logits + (size_t)row * a.row_stride + e0);
        z[v * VW + 0] = q.x;
        z[v * VW + 1] = q.y;
        z[v * VW + 2] = q.z;
        z[v * VW + 3] = q.w;
      } else {
        const uint4 q = *(const uint4*)((const uint16_t*)a.logits + (size_t)row * a.row_stride + e0);
        const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
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
        const int l = e0 + j - start;
        if (e0 + j < end) {
          const unsigned int bw = bits[l >> 5];
          if ((bw >> (l & 31)) & 1u) {
            const unsigned int c = cnts[wpre[l >> 5] + __popc(bw & ((1u << (l & 31)) - 1u))];
            z[v * VW + j] = apply_penalty(z[v * VW + j], c, p.rep, p.pres, p.freq);
          }
        }
      }
    }
    if (!p.greedy) {
#pragma unroll
      for (int j = 0; j < VW; ++j) z[v * VW + j] = z[v * VW + j] / p.T;
    }
  }

  // ---- row maximum (greedy: NaN is maximum; sampling: NaN is minimum)
  {
    unsigned long long best = 0ull;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const int e = start + (v * kMainThreads + tid) * VW + j;
        if (e < end) {
          const uint32_t k = p.greedy ? gkey(z[v * VW + j]) : skey(z[v * VW + j]);
          const unsigned long long pk = ((unsigned long long)k << 32) | (0xffffffffu - (uint32_t)e);
          best = pk > best ? pk : best;
        }
      }
    }
    best = block_max_u64<kMainThreads>(best, sh.red);
    if (tid == 0) atomicMax(&rs->maxpack, best);
  }

  // ---- top-k rows: local candidates
  const bool fast_topk = p.topk_on && p.k <= QS_TOPK_FAST_MAX;
  if (fast_topk) {
    const int nvalid = end - start;
    const int per_chunk = 2 * ((p.k + a.G - 1) / a.G) + 8;
    const int kc = min(p.k, per_chunk);
    unsigned int tau = 0u;
    unsigned int* hist = (unsigned int*)lds + 2 * nw + a.seg_cap;  // after penalty tables
    if (kc < nvalid) {
      unsigned int prefix = 0u, mask = 0u;
      unsigned int remaining = (unsigned int)kc;  // rank target counted from the top (1-based)
      const int shifts[3] = {21, 10, 0};
      const int nbits[3] = {11, 11, 10};
      for (int lv = 0; lv < 3; ++lv) {
        const int nb = 1 << nbits[lv];
        const unsigned int dmask = (unsigned int)nb - 1u;
        for (int i = tid; i < nb; i += kMainThreads) hist[i] = 0u;
        __syncthreads();
#pragma unroll
        for (int v = 0; v < NV; ++v) {
#pragma unroll
          for (int j = 0; j < VW; ++j) {
            const int e = start + (v * kMainThreads + tid) * VW + j;
            if (e < end) {
              const uint32_t k = skey(z[v * VW + j]);
              if ((k & mask) == prefix) atomicAdd(&hist[(k >> shifts[lv]) & dmask], 1u);
            }
          }
        }
        __syncthreads();
        find_bin<kMainThreads>(hist, nullptr, nullptr, nb, true, (u128)(remaining - 1u), sh.scan, &sh.bin,
                               &sh.above);
        const int d = sh.bin;
        remaining -= sh.above.c;
        prefix |= (unsigned int)d << shifts[lv];
        mask |= dmask << shifts[lv];
        __syncthreads();
      }
      tau = prefix;
    } else if (tid == 0) {
      atomicAdd(&rs->all_emitted, 1u);
    }
    // emit elements with key >= tau (local reservation, one global atomic)
    if (tid == 0) sh.counter = 0u;
    __syncthreads();
    unsigned int mine = 0;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const int e = start + (v * kMainThreads + tid) * VW + j;
        if (e < end && skey(z[v * VW + j]) >= tau) ++mine;
      }
    }
    const unsigned int my_off = atomicAdd(&sh.counter, mine);
    __syncthreads();
    if (tid == 0) {
      sh.flag = atomicAdd(&rs->cand_count, sh.counter);
      atomicMax(&rs->tau_max, tau);
    }
    __syncthreads();
    unsigned int pos = sh.flag + my_off;
    unsigned long long* cd = a.cand + (size_t)row * kCap;
#pragma unroll
    for (int v = 0; v < NV; ++v) {
#pragma unroll
      for (int j = 0; j < VW; ++j) {
        const int e = start + (v * kMainThreads + tid) * VW + j;
        if (e < end) {
          const uint32_t k = skey(z[v * VW + j]);
          if (k >= tau) {
            if (pos < (unsigned int)kCap)
              cd[pos] = ((unsigned long long)k << 32) | (0xffffffffu - (uint32_t)e);
            ++pos;
          }
        }
      }
    }
  }

  // ---- arrival; the last workgroup of the row finishes it
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned int prev = __hip_atomic_fetch_add(&rs->arrive_main, 1u, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
    sh.flag = (prev == (unsigned int)a.G - 1u) ? 1u : 0u;
  }
  __syncthreads();
  if (!sh.flag) return;
  __threadfence();

  const unsigned long long mp = ld_acquire(&rs->maxpack);
  if (p.greedy) {
    if (tid == 0) {
      const long long id = (long long)(0xffffffffu - (uint32_t)mp);
      a.out_ids[row] = id;
      rs->chosen = id;
      rs->greedy = 1u;
      rs->status = kDone;
    }
    __syncthreads();
    if (a.last_kernel == 1) clear_row(rs);
    return;
  }
  const int N = octave_of(z_of_key((uint32_t)(mp >> 32)), kLog2e);
  if (tid == 0) rs->n_max = N;
  if (!fast_topk) {
    if (tid == 0) rs->status = kNeedsResolve;
    return;
  }

  // merge candidates (keys >= tau_max are complete)
  const unsigned int total = ld_acquire(&rs->cand_count);
  const unsigned int tau = ld_acquire(&rs->tau_max);
  const unsigned int allem = ld_acquire(&rs->all_emitted);
  unsigned long long* s = (unsigned long long*)lds;  // reuses the chunk tables
  if (total > (unsigned int)kCap) {
    if (tid == 0) rs->status = kNeedsResolve;
    return;
  }
  if (tid == 0) sh.counter = 0u;
  __syncthreads();
  const unsigned long long* cd = a.cand + (size_t)row * kCap;
  for (unsigned int i = tid; i < total; i += kMainThreads) {
    const unsigned long long c = cd[i];
    if ((uint32_t)(c >> 32) >= tau) {
      const unsigned int slot = atomicAdd(&sh.counter, 1u);
      if (slot < (unsigned int)kMergeCap) s[slot] = c;
    }
  }
  __syncthreads();
  const int m = (int)sh.counter;
  const bool complete = ((m >= p.k) || (allem == (unsigned int)a.G)) && m <= kMergeCap;
  if (!complete) {
    if (tid == 0) rs->status = kNeedsResolve;
    return;
  }
  const int P = pow2_ceil(m);
  for (int i = m + tid; i < P; i += kMainThreads) s[i] = 0ull;
  __syncthreads();
  bitonic_desc<kMainThreads>(s, P);
  // top-k set = sorted prefix with key >= kappa_k
  int kend = m;
  if (p.k <= m) {
    const uint32_t kk = (uint32_t)(s[p.k - 1] >> 32);
    if (tid == 0) sh.counter = (unsigned int)m;
    __syncthreads();
    for (int i = tid; i < m; i += kMainThreads)
      if ((uint32_t)(s[i] >> 32) < kk) atomicMin(&sh.counter, (unsigned int)i);
    __syncthreads();
    kend = (int)sh.counter;
  }
  const double cT = kLog2e;
  // each thread owns a contiguous run of sorted positions
  const int per = (kend + kMainThreads - 1) / kMainThreads;
  Acc loc = {0, 0, 0};
  for (int q = 0; q < per; ++q) {
    const int i = tid * per + q;
    if (i < kend) {
      const unsigned long long w = weight_of(z_of_key((uint32_t)(s[i] >> 32)), cT, N);
      loc = acc_add(loc, acc_of((u128)w, w ? 1u : 0u));
    }
  }
  Acc tot;
  Acc ex = block_excl_scan<kMainThreads>(loc, sh.scan, &tot);
  int pend = kend;
  if (p.topp_on) {
    const u128 Tp = mul_frac(acc_mass(tot), p.tp);
    // pend = number of positions (< kend) with exclusive mass <= Tp
    if (tid == 0) sh.counter = (unsigned int)kend;
    __syncthreads();
    u128 run = acc_mass(ex);
    for (int q = 0; q < per; ++q) {
      const int i = tid * per + q;
      if (i < kend) {
        if (run > Tp) {
          atomicMin(&sh.counter, (unsigned int)i);
          break;
        }
        run += (u128)weight_of(z_of_key((uint32_t)(s[i] >> 32)), cT, N);
      }
    }
    __syncthreads();
    pend = (int)sh.counter;
  }
  // W and the kept description
  Acc loc2 = {0, 0, 0};
  for (int q = 0; q < per; ++q) {
    const int i = tid * per + q;
    if (i < pend) {
      const unsigned long long w = weight_of(z_of_key((uint32_t)(s[i] >> 32)), cT, N);
      loc2 = acc_add(loc2, acc_of((u128)w, w ? 1u : 0u));
    }
  }
  Acc W;
  (void)block_excl_scan<kMainThreads>(loc2, sh.scan, &W);
  const unsigned long long last = s[pend - 1];
  __syncthreads();
  // re-sort the kept prefix by id ascending: (id << 32) | sorted position
  unsigned long long* s2 = s + P;  // second buffer
  const int P2 = pow2_ceil(pend);
  for (int i = tid; i < P2; i += kMainThreads) {
    if (i < pend) {
      const uint32_t id = 0xffffffffu - (uint32_t)s[i];
      s2[i] = ((unsigned long long)id << 32) | (unsigned int)i;
    } else {
      s2[i] = ~0ull;
    }
  }
  __syncthreads();
  bitonic_asc<kMainThreads>(s2, P2);
  const u128 t = mul_frac(acc_mass(W), p.u);
  const int per2 = (pend + kMainThreads - 1) / kMainThreads;
  Acc l3 = {0, 0, 0};
  for (int q = 0; q < per2; ++q) {
    const int i = tid * per2 + q;
    if (i < pend) {
      const int sp = (int)(unsigned int)s2[i];
      l3 = acc_add(l3, acc_of((u128)weight_of(z_of_key((uint32_t)(s[sp] >> 32)), cT, N), 0));
    }
  }
  Acc tot3;
  Acc ex3 = block_excl_scan<kMainThreads>(l3, sh.scan, &tot3);
  if (tid == 0) sh.flag = 0xffffffffu;
  __syncthreads();
  {
    u128 run = acc_mass(ex3);
    for (int q = 0; q < per2; ++q) {
      const int i = tid * per2 + q;
      if (i < pend) {
        const int sp = (int)(unsigned int)s2[i];
        run += (u128)weight_of(z_of_key((uint32_t)(s[sp] >> 32)), cT, N);
        if (run > t) {
          atomicMin(&sh.flag, (unsigned int)(s2[i] >> 32));
          break;
        }
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    const long long id = (long long)sh.flag;
    a.out_ids[row] = id;
    rs->chosen = id;
    rs->kappa_p = (uint32_t)(last >> 32);
    rs->id_p = 0xffffffffu - (uint32_t)last;
    rs->w_lo = W.lo;
    rs->w_hi = W.hi;
    rs->status = kDone;
  }
  __syncthreads();
  if (a.last_kernel == 1) clear_row(rs);
}

// ---------------------------------------------------------------- resolver

struct ResolveShared {
  unsigned int cnt[2048];
  unsigned long long mlo[2048];
  unsigned long long mhi[2048];
  unsigned long long scan[64];
  int bin;
  Acc above;
  unsigned int flag;
  unsigned long long result;
};

struct Found {
  uint32_t key;
  Acc above;  // elements above key (count, mass)
  Acc tie;    // elements at key
};

// Radix select over the row in (key desc) order among elements with key >= key_lo.
// by_count: rank target (0-based); else mass target.
template <int DT>
__device__ Found radix_find(const Args& a, const RowParams& p, int row, int N, double cT, uint32_t key_lo,
                            bool by_count, u128 target, ResolveShared& sh) {
  const int shifts[3] = {21, 10, 0};
  const int nbits[3] = {11, 11, 10};
  unsigned int prefix = 0u, mask = 0u;
  Acc above = {0, 0, 0}, tie = {0, 0, 0};
  for (int lv = 0; lv < 3; ++lv) {
    const int nb = 1 << nbits[lv];
    const unsigned int dmask = (unsigned int)nb - 1u;
    for (int i = threadIdx.x; i < nb; i += kResolveThreads) {
      sh.cnt[i] = 0u;
      sh.mlo[i] = 0ull;
      sh.mhi[i] = 0ull;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < a.V; i += kResolveThreads) {
      const float z = load_z<DT>(a, p, row, i);
      const uint32_t k = skey(z);
      if (k < key_lo || (k & mask) != prefix) continue;
      const unsigned int d = (k >> shifts[lv]) & dmask;
      atomicAdd(&sh.cnt[d], 1u);
      const unsigned long long w = weight_of(z, cT, N);
      if (w) {
        atomicAdd(&sh.mlo[d], w & 0xffffffffull);
        atomicAdd(&sh.mhi[d], w >> 32);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) sh.bin = -1;
    __syncthreads();
    find_bin<kResolveThreads>(sh.cnt, sh.mlo, sh.mhi, nb, by_count, target, sh.scan, &sh.bin, &sh.above);
    const int d = sh.bin;
    if (d < 0) {  // target beyond the total: cannot happen for valid callers
      Found f;
      f.key = 0;
      f.above = above;
      f.tie = tie;
      return f;
    }
    above = acc_add(above, sh.above);
    target -= by_count ? (u128)sh.above.c : acc_mass(sh.above);
    prefix |= (unsigned int)d << shifts[lv];
    mask |= dmask << shifts[lv];
    tie = acc_of(((u128)sh.mhi[d] << 32) + (u128)sh.mlo[d], sh.cnt[d]);
    __syncthreads();
  }
  Found f;
  f.key = prefix;
  f.above = above;
  f.tie = tie;
  return f;
}

// Totals over elements with key >= key_lo: (count, mass).
template <int DT>
__device__ Acc row_total(const Args& a, const RowParams& p, int row, int N, double cT, uint32_t key_lo,
                         ResolveShared& sh) {
  Acc loc = {0, 0, 0};
  for (int i = threadIdx.x; i < a.V; i += kResolveThreads) {
    const float z = load_z<DT>(a, p, row, i);
    if (skey(z) < key_lo) continue;
    loc = acc_add(loc, acc_of((u128)weight_of(z, cT, N), 1u));
  }
  Acc tot;
  (void)block_excl_scan<kResolveThreads>(loc, sh.scan, &tot);
  return tot;
}

template <int DT>
__global__ __launch_bounds__(kResolveThreads) void k_resolve(Args a) {
  __shared__ ResolveShared sh;
  const int row = blockIdx.x;
  RowState* rs = a.rs + row;
  const unsigned int st = ld_acquire(&rs->status);
  if (st != kNeedsResolve) {
    __syncthreads();
    if (a.last_kernel == 2) clear_row(rs);
    return;
  }
  const RowParams p = row_params(a, row);
  const int N = rs->n_max;
  const double cT = kLog2e;
  // top-k: rank k-1 over all elements
  uint32_t kappa_k = 0u;
  Acc Sk;
  if (p.topk_on) {
    Found f = radix_find<DT>(a, p, row, N, cT, 0u, true, (u128)(p.k - 1), sh);
    kappa_k = f.key;
    Sk = acc_add(f.above, f.tie);
  } else {
    Sk = row_total<DT>(a, p, row, N, cT, 0u, sh);
  }
  uint32_t kappa_p = kappa_k, id_p = 0xffffffffu;
  Acc W = Sk;
  if (p.topp_on) {
    const u128 S = acc_mass(Sk);
    const u128 Tp = mul_frac(S, p.tp);
    if (Tp < S) {
      Found f = radix_find<DT>(a, p, row, N, cT, kappa_k, false, Tp, sh);
      kappa_p = f.key;
      const u128 A = acc_mass(f.above);
      const unsigned long long wk = weight_of(z_of_key(f.key), cT, N);
      // tie members j with A + j*wk <= Tp are kept (0-based j, ascending id)
      unsigned long long j = div_small(Tp - A, wk);
      if (j + 1 >= f.tie.c) {
        id_p = 0xffffffffu;
        W = acc_add(f.above, f.tie);
      } else {
        W = acc_add(f.above, acc_of((u128)wk * (u128)(j + 1), (unsigned int)(j + 1)));
        // id of the j-th (0-based) tie member in ascending id
        const int L = (a.V + kResolveThreads - 1) / kResolveThreads;
        const int i0 = threadIdx.x * L, i1 = min(a.V, i0 + L);
        unsigned int c = 0;
        for (int i = i0; i < i1; ++i)
          if (skey(load_z<DT>(a, p, row, i)) == kappa_p) ++c;
        if (threadIdx.x == 0) sh.flag = 0xffffffffu;
        Acc tot;
        Acc ex = block_excl_scan<kResolveThreads>(Acc{0, 0, c}, sh.scan, &tot);
        if (j >= ex.c && j < ex.c + c) {
          unsigned int r = ex.c;
          for (int i = i0; i < i1; ++i) {
            if (skey(load_z<DT>(a, p, row, i)) == kappa_p) {
              if (r == j) {
                sh.flag = (unsigned int)i;
                break;
              }
              ++r;
            }
          }
        }
        __syncthreads();
        id_p = sh.flag;
        __syncthreads();
      }
    }
  }
  // draw in ascending id over kept tokens
  const u128 t = mul_frac(acc_mass(W), p.u);
  const int L = (a.V + kResolveThreads - 1) / kResolveThreads;
  const int i0 = threadIdx.x * L, i1 = min(a.V, i0 + L);
  Acc loc = {0, 0, 0};
  for (int i = i0; i < i1; ++i) {
    const float z = load_z<DT>(a, p, row, i);
    const uint32_t k = skey(z);
    if (k > kappa_p || (k == kappa_p && (uint32_t)i <= id_p))
      loc = acc_add(loc, acc_of((u128)weight_of(z, cT, N), 0));
  }
  Acc tot;
  Acc ex = block_excl_scan<kResolveThreads>(loc, sh.scan, &tot);
  if (threadIdx.x == 0) sh.flag = 0xffffffffu;
  __syncthreads();
  {
    const u128 lo = acc_mass(ex);
    if (t >= lo && t < lo + acc_mass(loc)) {
      u128 run = lo;
      for (int i = i0; i < i1; ++i) {
        const float z = load_z<DT>(a, p, row, i);
        const uint32_t k = skey(z);
        if (k > kappa_p || (k == kappa_p && (uint32_t)i <= id_p)) {
          run += (u128)weight_of(z, cT, N);
          if (run > t) {
            sh.flag = (unsigned int)i;
            break;
          }
        }
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const long long id = (long long)sh.flag;
    a.out_ids[row] = id;
    rs->chosen = id;
    rs->kappa_p = kappa_p;
    rs->id_p = id_p;
    rs->w_lo = W.lo;
    rs->w_hi = W.hi;
    rs->status = kDone;
  }
  __syncthreads();
  if (a.last_kernel == 2) clear_row(rs);
}

// ---------------------------------------------------------------- probabilities

template <int DT>
__global__ __launch_bounds__(kMainThreads) void k_probs(Args a) {
  __shared__ unsigned long long red[16];
  __shared__ unsigned int last;
  const int row = blockIdx.y, chunk = blockIdx.x;
  const int start = chunk * a.CH, end = min(a.V, start + a.CH);
  RowState* rs = a.rs + row;
  const RowParams p = row_params(a, row);
  const long long chosen = rs->chosen;
  unsigned int kept = 0;
  if (rs->greedy) {
    for (int i = start + threadIdx.x; i < end; i += kMainThreads) {
      a.out_probs[(size_t)row * a.V + i] = (i == chosen) ? 1.0f : 0.0f;
      kept += (i == chosen);
    }
  } else {
    const int N = rs->n_max;
    const double cT = kLog2e;
    const u128 W = ((u128)rs->w_hi << 64) | rs->w_lo;
    const double Wd = u128_to_double(W);
    const uint32_t kp = rs->kappa_p, idp = rs->id_p;
    for (int i = start + threadIdx.x; i < end; i += kMainThreads) {
      const float z = load_z<DT>(a, p, row, i);
      const uint32_t k = skey(z);
      float pr = 0.0f;
      if (k > kp || (k == kp && (uint32_t)i <= idp)) {
        const unsigned long long w = weight_of(z, cT, N);
        pr = (float)((double)w / Wd);
        kept += (w != 0ull);
      }
      a.out_probs[(size_t)row * a.V + i] = pr;
    }
  }
  (void)red;
  for (int o = 32; o > 0; o >>= 1) kept += __shfl_xor(kept, o, 64);
  if ((threadIdx.x & 63) == 0) atomicAdd(&rs->kept_count, kept);
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned int prev = __hip_atomic_fetch_add(&rs->arrive_probs, 1u, __ATOMIC_ACQ_REL,
                                                     __HIP_MEMORY_SCOPE_AGENT);
    last = (prev == (unsigned int)a.G - 1u) ? 1u : 0u;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (threadIdx.x == 0 && a.out_kept) a.out_kept[row] = (int)ld_acquire(&rs->kept_count);
  __syncthreads();
  if (a.last_kernel == 3) clear_row(rs);
}

__global__ void k_zero(unsigned int* p, size_t n) {
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
  int CH, G, nwords, seg_cap;
  size_t off_rs, off_cand, off_bits, off_wpre, off_cnt, total;
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

Layout layout_for(int B, int V, int H) {
  Layout L;
  const int big = (int)(((long long)B * ((V + 16383) / 16384)) >= 512);
  L.CH = big ? 16384 : 4096;
  L.G = (V + L.CH - 1) / L.CH;
  L.nwords = (V + 31) / 32;
  L.seg_cap = H > 0 ? (H < L.CH ? H : L.CH) : 0;
  size_t o = 0;
  L.off_rs = o;
  o = align_up(o + (size_t)B * sizeof(RowState), 256);
  L.off_cand = o;
  o = align_up(o + (size_t)B * kCap * 8, 256);
  L.off_bits = o;
  o = align_up(o + (H > 0 ? (size_t)B * L.nwords * 4 : 0), 256);
  L.off_wpre = o;
  o = align_up(o + (H > 0 ? (size_t)B * L.nwords * 4 : 0), 256);
  L.off_cnt = o;
  o = align_up(o + (H > 0 ? (size_t)B * L.G * L.seg_cap * 4 : 0), 256);
  L.total = o;
  return L;
}

template <int DT, int EPT, bool VEC>
hipError_t launch_main(const Args& a, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((k_main<DT, EPT, VEC>), dim3(a.G, a.B), dim3(kMainThreads), lds, st, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_main_dt(const Args& a, bool vec, size_t lds, hipStream_t st) {
  if (a.CH == 16384) return vec ? launch_main<DT, 64, true>(a, lds, st) : launch_main<DT, 64, false>(a, lds, st);
  return vec ? launch_main<DT, 16, true>(a, lds, st) : launch_main<DT, 16, false>(a, lds, st);
}

int run(const void* logits, int64_t row_stride, int dtype, int B, int V, const float* temperature,
        const float* top_p, const int32_t* top_k, const float* rep, const float* pres, const float* freq,
        const int32_t* hist, int H, const float* uniforms, uint32_t flags, int64_t* out_ids, float* out_probs,
        int32_t* out_kept, void* ws, size_t ws_bytes, hipStream_t stream) {
  g_err[0] = 0;
  if (dtype != QS_DTYPE_F32 && dtype != QS_DTYPE_BF16) return fail("qs_sample: unknown logits dtype%s");
  if (B < 0 || V <= 0 || V >= (1 << 28)) return fail("qs_sample: bad shape (B >= 0, 0 < V < 2^28)%s");
  if (B == 0) return 0;
  if (row_stride < V) return fail("qs_sample: row_stride < V%s");
  if (!logits || !out_ids || !ws) return fail("qs_sample: null logits, out_ids or workspace%s");
  if (!(flags & QS_FLAG_ALL_GREEDY) && !temperature) return fail("qs_sample: temperature required%s");
  if (H < 0 || (H > 0 && !hist)) return fail("qs_sample: bad history arguments%s");
  if (out_kept && !out_probs) return fail("qs_sample: out_kept requires out_probs%s");
  const int Heff = hist ? H : 0;
  const Layout L = layout_for(B, V, Heff);
  if (ws_bytes < L.total) return fail("qs_sample: workspace too small (see qs_workspace_bytes)%s");
  if (((uintptr_t)ws) % 256) return fail("qs_sample: workspace must be 256-byte aligned%s");
  const bool all_greedy = (flags & QS_FLAG_ALL_GREEDY) != 0;
  if (!all_greedy && !uniforms) return fail("qs_sample: uniforms required unless all rows are greedy%s");

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
  a.nwords = L.nwords;
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
  a.rs = (RowState*)(base + L.off_rs);
  a.cand = (unsigned long long*)(base + L.off_cand);
  a.pbits = (unsigned int*)(base + L.off_bits);
  a.pwpre = (unsigned int*)(base + L.off_wpre);
  a.pcnt = (unsigned int*)(base + L.off_cnt);
  a.last_kernel = out_probs ? 3 : (all_greedy ? 1 : 2);

  const int esz = dtype == QS_DTYPE_F32 ? 4 : 2;
  const bool vec = (((uintptr_t)logits) % 16 == 0) && ((row_stride * esz) % 16 == 0);
  const size_t pen_lds = (size_t)(2 * (L.CH / 32) + L.seg_cap) * 4;
  const size_t main_lds_a = pen_lds + 2048 * 4;
  const size_t main_lds_b = (size_t)kMergeCap * 8 * 2;
  const size_t main_lds = main_lds_a > main_lds_b ? main_lds_a : main_lds_b;
  if (main_lds > 160 * 1024 - sizeof(MainShared)) return fail("qs_sample: history too long for LDS tables%s");

  hipError_t e = dtype == QS_DTYPE_F32 ? launch_main_dt<QS_DTYPE_F32>(a, vec, main_lds, stream)
                                       : launch_main_dt<QS_DTYPE_BF16>(a, vec, main_lds, stream);
  if (e != hipSuccess) return fail("qs_sample: main kernel launch failed: %s", hipGetErrorString(e));
  if (!all_greedy) {
    if (dtype == QS_DTYPE_F32)
      hipLaunchKernelGGL(k_resolve<QS_DTYPE_F32>, dim3(B), dim3(kResolveThreads), 0, stream, a);
    else
      hipLaunchKernelGGL(k_resolve<QS_DTYPE_BF16>, dim3(B), dim3(kResolveThreads), 0, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return fail("qs_sample: resolve kernel launch failed: %s", hipGetErrorString(e));
  }
  if (out_probs) {
    if (dtype == QS_DTYPE_F32)
      hipLaunchKernelGGL(k_probs<QS_DTYPE_F32>, dim3(a.G, B), dim3(kMainThreads), 0, stream, a);
    else
      hipLaunchKernelGGL(k_probs<QS_DTYPE_BF16>, dim3(a.G, B), dim3(kMainThreads), 0, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return fail("qs_sample: probs kernel launch failed: %s", hipGetErrorString(e));
  }
  return 0;
}

}  // namespace

extern "C" {

int qs_version(void) { return 100; }

const char* qs_last_error(void) { return g_err; }

size_t qs_workspace_bytes(int B, int V, int logits_dtype, int H) {
  (void)logits_dtype;
  if (B <= 0 || V <= 0) return 256;
  return layout_for(B, V, H > 0 ? H : 0).total;
}

int qs_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream) {
  g_err[0] = 0;
  if (!workspace) return fail("qs_workspace_init: null workspace%s");
  const size_t n = workspace_bytes / 4;
  hipLaunchKernelGGL(k_zero, dim3(1024), dim3(256), 0, stream, (unsigned int*)workspace, n);
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
