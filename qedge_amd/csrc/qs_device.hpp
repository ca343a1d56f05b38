// Device helpers of the sampler: memory model, wave64/workgroup collectives
// and the arithmetic of the sampling contract (stated in include/qsampler.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qs {

typedef unsigned long long u64;
typedef uint32_t u32;
typedef unsigned __int128 u128;

constexpr int kThreads = 512;  // every kernel: 8 waves of 64
constexpr int kWaves = kThreads / 64;

// ---------------------------------------------------------------- memory model
//
// Data that one workgroup writes and another reads in the same launch go
// through device-coherent accesses: relaxed agent-scope atomic stores and
// loads (global_store/global_load with sc1 on gfx950: the store is written
// through to the device-coherent level, the load is served from it).  A
// writer waits for its own stores to complete (s_waitcnt vmcnt(0)), then the
// workgroup barrier, then one thread updates a counter with a relaxed
// agent-scope atomic; a reader that has seen the counter issues its loads
// after that.  No release/acquire fences: at agent scope they write back or
// invalidate the whole L2 of an XCD.

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
// Every access to device memory goes through these, with the pointer cast to
// the global address space: generic (flat) accesses would also count against
// the LDS wait counter, so each workgroup barrier would wait for them.
// (The host compilation pass parses these device functions too; it keeps
// generic pointers.)
#if defined(__HIP_DEVICE_COMPILE__)
template <typename T>
using gptr = __attribute__((address_space(1))) T*;
#else
template <typename T>
using gptr = T*;
#endif
template <typename T>
__device__ __forceinline__ gptr<T> gp(T* p) {
  return (gptr<T>)p;
}
template <typename T>
__device__ __forceinline__ T gld(const T* p) {
  return *gp(p);
}
template <typename T>
__device__ __forceinline__ void gst(T* p, T v) {
  *gp(p) = v;
}
// A value the same for the whole launch (row parameters, the dispatch order),
// read through the scalar data cache: a scalar load, counted apart from the
// vector loads of the logits, so that waiting for it does not wait for them.
// Read-only data only: nothing the launch writes.
#if defined(__HIP_DEVICE_COMPILE__)
template <typename T>
__device__ __forceinline__ T sld(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}
#else
template <typename T>
__device__ __forceinline__ T sld(const T* p) {
  return *p;
}
#endif
template <typename T>
__device__ __forceinline__ T ldc(const T* p) {
  return __hip_atomic_load(gp(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void stc(T* p, T v) {
  __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T addc(T* p, T v) {
  return __hip_atomic_fetch_add(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void orc(u32* p, u32 v) {
  __hip_atomic_fetch_or(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- wave64 collectives (DPP)

__device__ __forceinline__ u32 lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

template <int CTRL, int ROWMASK>
__device__ __forceinline__ u32 dpp_mov(u32 v) {
  return (u32)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xF, false);
}
template <int CTRL, int ROWMASK>
__device__ __forceinline__ u64 dpp_mov64(u64 v) {
  return ((u64)dpp_mov<CTRL, ROWMASK>((u32)(v >> 32)) << 32) | dpp_mov<CTRL, ROWMASK>((u32)v);
}
// Inclusive scan (add) over the lanes of the wave.
__device__ __forceinline__ u32 wave_incl_scan(u32 v) {
  v += dpp_mov<0x111, 0xF>(v);  // row_shr:1
  v += dpp_mov<0x112, 0xF>(v);  // row_shr:2
  v += dpp_mov<0x114, 0xF>(v);  // row_shr:4
  v += dpp_mov<0x118, 0xF>(v);  // row_shr:8
  v += dpp_mov<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  v += dpp_mov<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}
__device__ __forceinline__ u64 wave_incl_scan64(u64 v) {
  v += dpp_mov64<0x111, 0xF>(v);
  v += dpp_mov64<0x112, 0xF>(v);
  v += dpp_mov64<0x114, 0xF>(v);
  v += dpp_mov64<0x118, 0xF>(v);
  v += dpp_mov64<0x142, 0xA>(v);
  v += dpp_mov64<0x143, 0xC>(v);
  return v;
}
__device__ __forceinline__ u32 readlane(u32 v, int l) { return (u32)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ u64 readlane64(u64 v, int l) {
  return ((u64)readlane((u32)(v >> 32), l) << 32) | readlane((u32)v, l);
}
__device__ __forceinline__ u32 wave_sum(u32 v) { return readlane(wave_incl_scan(v), 63); }
__device__ __forceinline__ u64 wave_sum64(u64 v) { return readlane64(wave_incl_scan64(v), 63); }
// Maximum over the wave, returned to every lane.
__device__ __forceinline__ u32 wave_max(u32 v) {
  v = max(v, dpp_mov<0xB1, 0xF>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_mov<0x4E, 0xF>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_mov<0x141, 0xF>(v));  // row_half_mirror
  v = max(v, dpp_mov<0x140, 0xF>(v));  // row_mirror
  v = max(v, dpp_mov<0x142, 0xA>(v));  // row_bcast:15
  v = max(v, dpp_mov<0x143, 0xC>(v));  // row_bcast:31
  return readlane(v, 63);
}
// Minimum: the maximum of the complements.
__device__ __forceinline__ u32 wave_min(u32 v) { return ~wave_max(~v); }
template <int CTRL, int ROWMASK>
__device__ __forceinline__ u64 max64_step(u64 v) {
  const u64 t = dpp_mov64<CTRL, ROWMASK>(v);
  return t > v ? t : v;
}
__device__ __forceinline__ u64 wave_max64(u64 v) {
  v = max64_step<0xB1, 0xF>(v);
  v = max64_step<0x4E, 0xF>(v);
  v = max64_step<0x141, 0xF>(v);
  v = max64_step<0x140, 0xF>(v);
  v = max64_step<0x142, 0xA>(v);
  v = max64_step<0x143, 0xC>(v);
  return readlane64(v, 63);
}
__device__ __forceinline__ u32 popc64(u64 m) { return (u32)__popcll(m); }
// Rank of this lane among the lanes whose bit is set in m (lanes below it).
__device__ __forceinline__ u32 lanes_below(u64 m) {
  return __builtin_amdgcn_mbcnt_hi((u32)(m >> 32), __builtin_amdgcn_mbcnt_lo((u32)m, 0u));
}

// ---------------------------------------------------------------- workgroup collectives

struct Scratch {
  u32 v[kWaves][8];
  u64 w[kWaves][4];
  u32 r[16];
  u64 r64[16];
};

__device__ __forceinline__ u32 block_max(u32 v, Scratch& s) {
  v = wave_max(v);
  if (lane_id() == 0) s.v[wave_id()][0] = v;
  lds_sync();
  u32 r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r = max(r, s.v[i][0]);
  lds_sync();
  return r;
}
__device__ __forceinline__ u64 block_max64(u64 v, Scratch& s) {
  v = wave_max64(v);
  if (lane_id() == 0) s.w[wave_id()][0] = v;
  lds_sync();
  u64 r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r = s.w[i][0] > r ? s.w[i][0] : r;
  lds_sync();
  return r;
}
__device__ __forceinline__ u32 block_sum(u32 v, Scratch& s) {
  v = wave_sum(v);
  if (lane_id() == 0) s.v[wave_id()][1] = v;
  lds_sync();
  u32 r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r += s.v[i][1];
  lds_sync();
  return r;
}
__device__ __forceinline__ u64 block_sum64(u64 v, Scratch& s) {
  v = wave_sum64(v);
  if (lane_id() == 0) s.w[wave_id()][1] = v;
  lds_sync();
  u64 r = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) r += s.w[i][1];
  lds_sync();
  return r;
}
// Exclusive scans in thread order; total in *total.
__device__ __forceinline__ u32 block_excl(u32 v, Scratch& s, u32* total) {
  const u32 inc = wave_incl_scan(v);
  if (lane_id() == 63) s.v[wave_id()][2] = inc;
  lds_sync();
  u32 base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    base += (i < wave_id()) ? s.v[i][2] : 0u;
    tot += s.v[i][2];
  }
  lds_sync();
  *total = tot;
  return base + inc - v;
}
__device__ __forceinline__ u64 block_excl64(u64 v, Scratch& s, u64* total) {
  const u64 inc = wave_incl_scan64(v);
  if (lane_id() == 63) s.w[wave_id()][2] = inc;
  lds_sync();
  u64 base = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    base += (i < wave_id()) ? s.w[i][2] : 0ull;
    tot += s.w[i][2];
  }
  lds_sync();
  *total = tot;
  return base + inc - v;
}
// Both scans with one pair of barriers.
__device__ __forceinline__ void block_excl2(u32& c, u64& m, Scratch& s, u32* ctot, u64* mtot) {
  const u32 ci = wave_incl_scan(c);
  const u64 mi = wave_incl_scan64(m);
  if (lane_id() == 63) {
    s.v[wave_id()][3] = ci;
    s.w[wave_id()][3] = mi;
  }
  lds_sync();
  u32 cb = 0, ct = 0;
  u64 mb = 0, mt = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const bool lo = i < wave_id();
    cb += lo ? s.v[i][3] : 0u;
    ct += s.v[i][3];
    mb += lo ? s.w[i][3] : 0ull;
    mt += s.w[i][3];
  }
  lds_sync();
  *ctot = ct;
  *mtot = mt;
  c = cb + ci - c;
  m = mb + mi - m;
}

// ---------------------------------------------------------------- contract arithmetic

// Sampling key: orderable bits, NaN lowest (0), -0 == +0.
__device__ __forceinline__ u32 skey(float z) {
  // z + 0 turns -0 into +0 (round to nearest) and keeps every other value,
  // denormals included; then the sign-magnitude bits become an unsigned order
  const u32 u = __float_as_uint(z + 0.0f);
  const u32 k = u ^ ((u32)((int)u >> 31) | 0x80000000u);
  return (z != z) ? 0u : k;
}
// Greedy key: NaN highest.
__device__ __forceinline__ u32 gkey(float z) { return (z != z) ? 0xffffffffu : skey(z); }
__device__ __forceinline__ float f_of_key(u32 k) {
  const u32 u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}
__device__ __forceinline__ float bf16_to_f32(u32 h) { return __uint_as_float(h << 16); }

// ---------------------------------------------------------------- 16-bit keys of bf16 logits, two per register
//
// For streaming passes over bf16 logits without penalties (z is the logit
// itself): the h key of a bf16 bit pattern x is (x ^ (sign ? 0xffff : 0x8000))
// + 0x7f mod 2^16, computed for both halves of a register with packed 16-bit
// operations.  It orders like the values, with the NaNs wrapped below -inf:
// NaNs in [0, 0xfd], -inf 0xfe, finite values and +inf in [0xff, 0xffff]; -0
// (0x807e) sits one below +0 (0x807f), so code that needs them equal compares
// through key_of_h, which maps both to the key of +0 only after skey().
typedef unsigned short us2 __attribute__((ext_vector_type(2)));
typedef short ss2 __attribute__((ext_vector_type(2)));
constexpr u32 kHNegInf = 0xfeu;  // h key of -inf; every h key below it is a NaN
__host__ __device__ __forceinline__ u32 hkey2(u32 x) {
  const u32 s = __builtin_bit_cast(u32, __builtin_bit_cast(ss2, x) >> (ss2)15);
  return __builtin_bit_cast(u32, __builtin_bit_cast(us2, x ^ (s | 0x80008000u)) + (us2)0x7f);
}
// The sampling key (skey without the -0 fold: -0 gives 0x7fffffff) of the value
// with h key h; 0 for NaN.
__host__ __device__ __forceinline__ u32 key_of_h(u32 h) {
  if (h < kHNegInf) return 0u;
  const u32 k = (h - 0x7fu) & 0xffffu;
  return k >= 0x8000u ? (k << 16) : ((k << 16) | 0xffffu);
}
__device__ __forceinline__ u32 pk_max_u16(u32 a, u32 b) {
  return __builtin_bit_cast(u32, __builtin_elementwise_max(__builtin_bit_cast(us2, a), __builtin_bit_cast(us2, b)));
}
__device__ __forceinline__ u32 pk_min_u16(u32 a, u32 b) {
  return __builtin_bit_cast(u32, __builtin_elementwise_min(__builtin_bit_cast(us2, a), __builtin_bit_cast(us2, b)));
}
__device__ __forceinline__ u32 pk_add_u16(u32 a, u32 b) {
  return __builtin_bit_cast(u32, __builtin_bit_cast(us2, a) + __builtin_bit_cast(us2, b));
}
// max(a - b, 0) per half.  Written as the instruction itself: in source form
// the compiler turns min(sub_sat(a, b), 1) into compares and selects per half.
__device__ __forceinline__ u32 pk_sub_sat_u16(u32 a, u32 b) {
  u32 r;
  asm("v_pk_sub_u16 %0, %1, %2 clamp" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// Per half: 1 when h >= t + 1, else 0 (t1 holds t in both halves).
__device__ __forceinline__ u32 pk_above(u32 h, u32 t1) { return pk_min_u16(pk_sub_sat_u16(h, t1), 0x00010001u); }

// z / b for a row-constant b with r = 1 / b (correctly rounded): Markstein's
// correction of q0 = z * r by the exact residual fma(-q0, b, z).  It equals the
// correctly rounded z / b whenever div_fast_ok holds (|z| and |q0| in
// [2^-100, 2^100)); tests/test_fastdiv.py checks this on the host.
__device__ __forceinline__ float div_fast(float z, float b, float r) {
  const float q0 = z * r;
  const float e = __builtin_fmaf(-q0, b, z);
  return __builtin_fmaf(e, r, q0);
}
__device__ __forceinline__ bool div_fast_ok(float z, float r) {
  const u32 aq = __float_as_uint(z * r) & 0x7fffffffu, az = __float_as_uint(z) & 0x7fffffffu;
  return (aq - 0x0d800000u) < (0x71800000u - 0x0d800000u) && (az - 0x0d800000u) < (0x71800000u - 0x0d800000u);
}
// The contract's q = z / T (one IEEE division).
__device__ __forceinline__ float qdiv(float z, float T, float rT, bool t_one) {
  if (t_one) return z;
  return div_fast_ok(z, rT) ? div_fast(z, T, rT) : z / T;
}
// One IEEE step each (rrep = 1 / rep, for the exact fast division).
__device__ __forceinline__ float apply_penalty(float z, u32 c, float rep, float rrep, float pres, float freq) {
  z = (z > 0.0f) ? (div_fast_ok(z, rrep) ? div_fast(z, rep, rrep) : z / rep) : (z * rep);
  const float fc = freq * (float)c;
  z = z - fc;
  z = z - pres;
  return z;
}
// 2^f on [0, 1]: degree-6 fp32 Horner with FMA (coefficients from oracle/fit_exp2.py).
__device__ __forceinline__ float exp2_poly(float f) {
  float p = 0x1.c5417ap-13f;
  p = __builtin_fmaf(p, f, 0x1.46d64cp-10f);
  p = __builtin_fmaf(p, f, 0x1.3d0b92p-7f);
  p = __builtin_fmaf(p, f, 0x1.c68912p-5f);
  p = __builtin_fmaf(p, f, 0x1.ebfd58p-3f);
  p = __builtin_fmaf(p, f, 0x1.62e42cp-1f);
  p = __builtin_fmaf(p, f, 1.0f);
  return p;
}
constexpr float kL2E = 0x1.715476p+0f;  // fp32(log2 e)
// The contract weight of a token with q (key k) given the row maximum qs (key
// ks), SH = 40 - ceil(log2 V), packed in 32 bits as ((s + 64) << 24) | M with
// w = M << s (s >= 0) or M >> -s; 0 when the weight is 0.  Branch-free.
__device__ __forceinline__ u32 wpack_of(float q, u32 k, float qs, u32 ks, int SH) {
  // Dead tokens are computed through and masked at the end: NaN q has key 0, and
  // with q* finite (or d = 0) every other y is a number or -inf, so s > -24
  // (which implies y >= -64 for SH <= 40) decides; floor(y) is clamped before
  // its conversion so that the conversion stays in range.
  const float d = (k == ks) ? 0.0f : q - qs;
  const float y = d * kL2E;
  const float fl = __builtin_floorf(y);
  const float f = y - fl;
  float p = exp2_poly(f);
  p = __builtin_amdgcn_fmed3f(p, 1.0f, __uint_as_float(0x3fffffffu));
  const u32 m = 0x800000u | (__float_as_uint(p) & 0x7fffffu);
  const int s = (int)fmaxf(fl, -128.0f) + SH;
  const bool live = k != 0u && s > -24;
  return live ? ((u32)(s + 64) << 24) | m : 0u;
}
__device__ __forceinline__ u64 wunpack(u32 wp) {
  // wp == 0 has m == 0; a live weight has -23 <= s <= 39, so m << s < 2^63
  const u64 m = wp & 0xffffffu;
  const int s = (int)(wp >> 24) - 64;
  return (m << (s > 0 ? s : 0)) >> (s < 0 ? min(-s, 63) : 0);
}
// The same weight as wunpack(wpack_of(q, skey(q), qs, skey(qs), SH)) for a
// finite row maximum qs, from d = q - qs and without the key: d is 0 at the
// maximum (also for -0 against +0), NaN for a NaN q and -inf for q = -inf.
// flmin = -(SH + 40) clamps the shift to s >= -40, where the weights below 1
// (s <= -24, which takes in the NaN and -inf tokens) come out of the right
// shift as 0 since m < 2^24; every weight of 1 or more has its s unchanged.
__device__ __forceinline__ u64 weight_finite(float d, float flmin, int SH) {
  const float y = d * kL2E;
  const float fl = __builtin_floorf(y);
  const float f = y - fl;
  float p = exp2_poly(f);
  p = __builtin_amdgcn_fmed3f(p, 1.0f, __uint_as_float(0x3fffffffu));
  const u64 m = 0x800000u | (__float_as_uint(p) & 0x7fffffu);
  const int s = (int)fmaxf(fl, flmin) + SH;
  return (m << max(s, 0)) >> max(-s, 0);
}
__device__ __forceinline__ u64 weight_of(float q, u32 k, float qs, u32 ks, int SH) {
  return wunpack(wpack_of(q, k, qs, ks, SH));
}
// floor(x * f) for f in [0, 1] given as fp32, x < 2^64.
__device__ __forceinline__ u64 mul_frac(u64 x, float f) {
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
  return (u64)(((u128)x * (u128)m) >> shift);
}
// ceil(f * 2^e) for f in [0, 1] as fp32, e >= 0.
__device__ __forceinline__ u64 ceil_scaled(float f, int e) {
  if (!(f > 0.0f)) return 0;
  const u32 b = __float_as_uint(f);
  const u32 ex = (b >> 23) & 0xffu;
  u64 m = b & 0x7fffffu;
  int sh;
  if (ex == 0) {
    sh = 149;
  } else {
    m |= 0x800000u;
    sh = 150 - (int)ex;
  }
  sh -= e;
  if (sh <= 0) return m << (-sh);
  if (sh >= 64) return 1;
  return (m >> sh) + ((m & ((1ull << sh) - 1ull)) != 0ull);
}
// The least packed weight (as wpack_of makes them) whose weight is >= thr, so
// that w >= thr can be tested on packed weights: packed weights are ordered as
// their weights.  0 for thr == 0; 0xffffffff when no weight reaches thr.
__device__ __forceinline__ u32 packed_threshold(u64 thr) {
  if (thr == 0ull) return 0u;
  for (int s = -23; s < 64; ++s) {
    const u32 top = (u32)(s + 64) << 24;
    if (wunpack(top | 0xffffffu) < thr) continue;
    u32 lo = 0x800000u, hi = 0xffffffu;  // the least mantissa M with unpack >= thr
    while (lo < hi) {
      const u32 mid = (lo + hi) >> 1;
      if (wunpack(top | mid) >= thr)
        hi = mid;
      else
        lo = mid + 1u;
    }
    return top | lo;
  }
  return 0xffffffffu;
}
// Values equal in every lane, moved to scalar registers.
__device__ __forceinline__ u32 uni(u32 v) { return (u32)__builtin_amdgcn_readfirstlane((int)v); }
__device__ __forceinline__ u64 uni64(u64 v) { return ((u64)uni((u32)(v >> 32)) << 32) | uni((u32)v); }
__device__ __forceinline__ int bitlen(u32 x) { return x ? 32 - __clz((int)x) : 0; }

}  // namespace qs
