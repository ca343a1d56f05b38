// One workgroup per row, for large batches: the workgroup streams its row in
// passes with the next chunk's loads in flight while it works on the current
// one, and needs no other workgroup.  Same contract and results as k_sample.
//
//   pass 1  key range of q (and the greedy id)
//   top-k   the k-th largest key: passes histogramming the keys (256 bins)
//           until the bin holds one key
//   pass 2  weights: S, the per-segment masses, the first mass histogram
//   rounds  while the bin holding the top-p boundary is too large: one more
//           pass histograms the bin's tokens by key (256 bins, counts and mass)
//   pass 3  the bracket's tokens listed (key, id) in LDS, the mass above it per
//           segment (a segment is one wave's share of one chunk: kWaveSpan ids)
//   final   the exact boundary among the listed tokens, the segment holding the
//           draw, and the token inside it from one wave's re-read of the segment.
#pragma once

#include "qs_kernels.hpp"

namespace qs {

constexpr int kSoloList = 2048;   // bracket tokens listed in LDS
constexpr int kSoloSegs = 1024;   // segments per row (G * kWaves)
constexpr int kSoloRounds = 6;    // bracket rounds: the first in x = q* - q, then in key space
constexpr int kSoloHist = 4096;   // history ids copied to LDS (the rest are read from memory)
constexpr int kSoloCBuf = 128;    // pass 3: tokens at or below the bracket per wave and chunk, compacted

struct SoloFin {
  u64 ent[kSoloList];  // listed tokens (key << 32 | id), in no particular order
  u32 lk[kDirect];     // a select bin's keys for the direct resolution
  u64 lw[kDirect];
};
struct SoloSel {
  u32 hc[2 * kNB];  // two buffers
  u64 hm[2 * kNB];
};
struct SoloLds {
  union {
    SoloFin fin;
  } u;
  u32 pen[kCH / 2];      // the chunk's history counts
  int hist[kSoloHist];   // the row's history ids
  SoloSel sel;           // select histogram of the final selection
  u64 mh[kNB];           // bracket histogram: mass per bin
  u32 hc[kNB];           // and tokens per bin (key-space rounds)
  u64 seg[kSoloSegs];    // per segment: total mass, then the mass above the bracket, then kept mass
  u32 segt[kSoloSegs];   // per segment: tokens at the boundary key (a bracket of one key)
  u64 cbuf[kWaves][kSoloCBuf];  // pass 3: each wave's tokens at or below the bracket, compacted
  u32 nlist;
  Scratch s;
};

__device__ __forceinline__ u32* pen_table(SoloLds& L) { return L.pen; }
__device__ __forceinline__ const u32* pen_table(const SoloLds& L) { return L.pen; }
__device__ __forceinline__ int hist_id(const RowP& p, const SoloLds& L, int i) {
  return i < kSoloHist ? L.hist[i] : gld(p.hist + i);
}

// Segment of a token id: one wave's share (kWaveSpan ids) of a chunk.
__device__ __forceinline__ int solo_seg_of(int id) { return id / kWaveSpan; }
// seg_find over segment s (its J vector spans in id order): the id where the
// running total of val passes t, or -1.
template <int DT, typename VF>
__device__ __forceinline__ long long solo_seg_find(const Args& a, const RowP& p, int row, const SoloLds& L, int s,
                                                   u64 t, VF&& val) {
  constexpr int J = Chunk<DT>::J;
  for (int j = 0; j < J; ++j) {
    u64 tot;
    const long long id = seg_find<DT>(a, p, row, L, s * J + j, t, val, &tot);
    if (id >= 0) return id;
    t -= tot;  // the span's total is at most t
  }
  return -1;
}

// Loads of chunk c for the streaming passes with 16-byte vectors (Args::vec_ok
// and V >= VL): one vector load each, always issued, so that the number of
// loads in flight does not depend on the data and the next chunk's loads stay
// in flight while this one is worked on.  A vector that is not wholly below V
// reads the row's first vector instead; chunk_tail completes the chunk holding
// V before use.
template <int DT>
__device__ __forceinline__ void load_chunk_vec(const Args& a, int row, int c, Chunk<DT>& ch) {
  constexpr int VL = Chunk<DT>::VL;
  ch.base = c * kCH + wave_id() * kWaveSpan + lane_id() * VL;
  ch.nval = a.V - ch.base;
  const char* rp = (const char*)a.logits + (size_t)row * (size_t)a.row_stride * (16 / VL);
#pragma unroll
  for (int j = 0; j < Chunk<DT>::J; ++j) {
    const int i0 = ch.base + j * 64 * VL;
    const int at = i0 + VL <= a.V ? i0 : 0;
    ch.v[j] = gld((const uint4*)(rp + (size_t)at * (16 / VL)));
  }
}
// The vector holding id V - 1 when V is not a multiple of VL: its ids below V,
// NaN past them (NaN padding everywhere when V is a multiple of VL).
template <int DT>
__device__ __forceinline__ uint4 row_tail_vec(const Args& a, int row) {
  constexpr int VL = Chunk<DT>::VL;
  const int i0 = a.V / VL * VL;
  const u32 pad = DT == QS_DTYPE_F32 ? 0x7fc00000u : 0x7fc07fc0u;
  u32 x[4] = {pad, pad, pad, pad};
  const size_t rowoff = (size_t)row * (size_t)a.row_stride;
  if (DT == QS_DTYPE_F32) {
    const float* q = (const float*)a.logits + rowoff;
    for (int e = 0; e < 4; ++e)
      if (i0 + e < a.V) x[e] = __float_as_uint(gld(q + i0 + e));
  } else {
    const uint16_t* q = (const uint16_t*)a.logits + rowoff;
    for (int e = 0; e < 8; ++e)
      if (i0 + e < a.V) x[e >> 1] = (x[e >> 1] & ~(0xffffu << ((e & 1) * 16))) | ((u32)gld(q + i0 + e) << ((e & 1) * 16));
  }
  return make_uint4(uni(x[0]), uni(x[1]), uni(x[2]), uni(x[3]));  // the same in every lane
}
// The chunk holding V: the vector across V from tv, NaN past it.
template <int DT>
__device__ __forceinline__ void chunk_tail(const Args& a, Chunk<DT>& ch, const uint4& tv) {
  constexpr int VL = Chunk<DT>::VL;
  const u32 pad = DT == QS_DTYPE_F32 ? 0x7fc00000u : 0x7fc07fc0u;
#pragma unroll
  for (int j = 0; j < Chunk<DT>::J; ++j) {
    const int i0 = ch.base + j * 64 * VL;
    if (i0 + VL > a.V) ch.v[j] = i0 < a.V ? tv : make_uint4(pad, pad, pad, pad);
  }
}

// f(ch, c) over the row's chunks, with chunk c + 1's loads in flight during
// chunk c and the history table built per chunk.  VEC: the loads of
// load_chunk_vec (the chunk past the last re-reads the last chunk, which is
// never worked on), tv the row's tail vector.
template <int DT, bool VEC, typename F>
__device__ __forceinline__ void solo_pass(const Args& a, const RowP& p, int row, SoloLds& L, const uint4& tv, F&& f) {
  Chunk<DT> b0, b1;
  if constexpr (VEC) {
    const int last = a.G - 1;
    const bool tail = a.V % kCH != 0;  // the last chunk holds V
    load_chunk_vec<DT>(a, row, 0, b0);
    for (int c = 0; c < a.G; c += 2) {
      load_chunk_vec<DT>(a, row, min(c + 1, last), b1);
      if (p.pen) pen_build(p, c, L);
      if (tail && c == last) chunk_tail<DT>(a, b0, tv);
      f(b0, c);
      if (p.pen) lds_sync();
      if (c + 1 >= a.G) break;
      load_chunk_vec<DT>(a, row, min(c + 2, last), b0);
      if (p.pen) pen_build(p, c + 1, L);
      if (tail && c + 1 == last) chunk_tail<DT>(a, b1, tv);
      f(b1, c + 1);
      if (p.pen) lds_sync();
    }
  } else {
    load_chunk<DT>(a, row, 0, b0);
    for (int c = 0; c < a.G; c += 2) {
      if (c + 1 < a.G) load_chunk<DT>(a, row, c + 1, b1);
      if (p.pen) pen_build(p, c, L);
      f(b0, c);
      if (p.pen) lds_sync();
      if (c + 1 >= a.G) break;
      if (c + 2 < a.G) load_chunk<DT>(a, row, c + 2, b0);
      if (p.pen) pen_build(p, c + 1, L);
      f(b1, c + 1);
      if (p.pen) lds_sync();
    }
  }
}

// The bracket: the tokens with key in [lo, hi].  After the first round it is
// mass bin b0's exact key range (mass_bin falls as the key grows); each
// key-space round narrows it to one of its 256 key bins.
struct Bracket {
  MassBins mb0;
  u32 b0, lo, hi;
};
// Key-space bin of round r >= 1 for a key of bin b0 (range [lo, hi], width 2^sh per bin).
__device__ __forceinline__ u32 key_bin(u32 k, u32 lo, u32 hi, int sh) {
  return k > hi ? 0u : (k < lo ? (u32)kNB - 1u : (hi - k) >> sh);
}
// 0: above the bracket, 1: in it, 2: below it (the bracket is the key range [lo, hi]).
__device__ __forceinline__ int bracket_side(const Bracket& br, u32 k) {
  return k > br.hi ? 0 : (k < br.lo ? 2 : 1);
}

#ifdef QS_TRACE
#define QS_TRS(i)                                                                  \
  do {                                                                             \
    if (a.trace && threadIdx.x == 0) a.trace[(size_t)row * a.G * 32 + (i)] = wall_clock64(); \
  } while (0)
#else
#define QS_TRS(i) \
  do {            \
  } while (0)
#endif

// VEC: the logits in 16-byte vectors (Args::vec_ok) and V >= VL.
template <int DT, bool VEC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_solo(Args a) {
  __shared__ SoloLds L;
  constexpr int J = Chunk<DT>::J, VL = Chunk<DT>::VL;
  const int row = (int)uni(a.order ? (u32)gld(a.order + blockIdx.x) : blockIdx.x);
  if ((unsigned)row >= (unsigned)a.B) return;
  const RowP p = row_params(a, row);
  const uint4 tv = VEC ? row_tail_vec<DT>(a, row) : make_uint4(0u, 0u, 0u, 0u);
  const int SH = a.SH;
  const u64 thr = ceil_scaled(p.mp, 23 + SH);
  const u32 pthr = uni(packed_threshold(thr));
  if (p.pen) {
    for (int i = threadIdx.x; i < min(p.hlen, kSoloHist); i += kThreads) L.hist[i] = gld(p.hist + i);
    lds_sync();
  }
  QS_TRS(0);
  // ---- pass 1: key range of q, or the greedy id
  if (p.kind == kKindGreedy) {
    u64 best = 0;
    solo_pass<DT, VEC>(a, p, row, L, tv, [&](const Chunk<DT>& ch, int c) {
      with_pen(p.pen, [&](auto pen) {
        constexpr bool PEN = decltype(pen)::value;
        u32 pw[kEPT / 2] = {};
        if constexpr (PEN) chunk_counts(L, ch, c, pw);
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int e = 0; e < VL; ++e) {
            const float z = elem_zt<PEN>(ch, p, pw, j, e);
            const u64 pk = ((u64)(ch.valid(j, e) ? gkey(z) : 0u) << 32) | (0xffffffffu - (u32)ch.id(j, e));
            best = pk > best ? pk : best;
          }
      });
    });
    best = block_max64(best, L.s);
    const u32 id = 0xffffffffu - (u32)best;
    write_result(a, row, p, (long long)id, 0, 0, kPathGreedy, 0u, 0u, 0u, id, 1u);
    return;
  }
  u32 kmax = 0, kmin = 0xffffffffu, nnan = 0;
  u64 gbest = 0;
  if (!p.pen) {
    // z is the logit: q* and q_min are the quotients of its maximum and minimum
    // (z / T is monotone), which NaN-ignoring max / min find; NaN past V
    float zmx = -__builtin_inff(), zmn = __builtin_inff();
    solo_pass<DT, VEC>(a, p, row, L, tv, [&](const Chunk<DT>& ch, int c) {
      (void)c;
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int e = 0; e < VL; ++e) {
          const float z = ch.raw(j, e);
          zmx = fmaxf(zmx, z);
          zmn = fminf(zmn, z);
          nnan += z == z ? 1u : 0u;
        }
    });
    u32 kx = skey(zmx), kn = ~skey(zmn);
    block_max2(kx, kn, L.s);
    nnan = block_sum(nnan, L.s);
    if (nnan) {
      kmax = skey(qdiv(f_of_key(kx), p));
      kmin = skey(qdiv(f_of_key(~kn), p));
    }
    gbest = 0xffffffffu;  // every z NaN: the first id
  } else {
    solo_pass<DT, VEC>(a, p, row, L, tv, [&](const Chunk<DT>& ch, int c) {
      with_pen(p.pen, [&](auto pen) {
        constexpr bool PEN = decltype(pen)::value;
        u32 pw[kEPT / 2] = {};
        if constexpr (PEN) chunk_counts(L, ch, c, pw);
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
          for (int e = 0; e < VL; ++e) {
            const float z = elem_zt<PEN>(ch, p, pw, j, e);
            const u32 k = skey(qdiv(z, p));  // 0 past V (NaN padding)
            kmax = max(kmax, k);
            kmin = k ? min(kmin, k) : kmin;
            nnan += k ? 1u : 0u;
            const u64 pk = ((u64)(ch.valid(j, e) ? gkey(z) : 0u) << 32) | (0xffffffffu - (u32)ch.id(j, e));
            gbest = pk > gbest ? pk : gbest;
          }
      });
    });
    u32 nk = ~kmin;
    block_max2(kmax, nk, L.s);
    kmin = ~nk;
    gbest = block_max64(gbest, L.s);
    nnan = block_sum(nnan, L.s);  // tokens whose q is not NaN
  }
  // the row's figures are the same in every lane: scalar registers
  kmax = uni(kmax);
  kmin = uni(kmin);
  nnan = uni(nnan);
  gbest = uni64(gbest);
  if (kmax == 0u) {  // every q is NaN: no weights, the greedy id (as the exact path)
    write_result(a, row, p, (long long)(0xffffffffu - (u32)gbest), 0, thr, kPathSolo, 0u, 0u, 0u, 0u, 0u);
    return;
  }
  const float qs = f_of_key(kmax);
  QS_TRS(1);
  // ---- top-k: the k-th largest key (ties kept), by key histograms
  u32 kk = 1u;
  if ((p.kind == kKindTopK || p.kind == kKindSingle) && nnan > (u32)p.k) {
    u32 lo = kmin, hi = kmax;
    u64 target = (u64)p.k;
    for (int r = 0; r < 5; ++r) {
      for (int b = threadIdx.x; b < kNB; b += kThreads) L.hc[b] = 0u;
      lds_sync();
      const int bl = bitlen(hi - lo);
      const int sh = bl > 8 ? bl - 8 : 0;
      solo_pass<DT, VEC>(a, p, row, L, tv, [&](const Chunk<DT>& ch, int c) {
        with_pen(p.pen, [&](auto pen) {
          constexpr bool PEN = decltype(pen)::value;
          u32 pw[kEPT / 2] = {};
          if constexpr (PEN) chunk_counts(L, ch, c, pw);
#pragma unroll
          for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < VL; ++e) {
              const u32 k = skey(qdiv(elem_zt<PEN>(ch, p, pw, j, e), p));
              if (k >= lo && k <= hi && k) atomicAdd(&L.hc[(hi - k) >> sh], 1u);
            }
        });
      });
      lds_sync();
      const int b = threadIdx.x;
      const u32 bc = b < kNB ? L.hc[b] : 0u;
      u32 tot;
      const u32 ex = block_excl(bc, L.s, &tot);
      if (threadIdx.x == 0) L.s.r[12] = 0xffffffffu;
      lds_sync();
      if (b < kNB && (u64)ex < target && target <= (u64)ex + bc) {
        L.s.r[12] = (u32)b;
        L.s.r[13] = ex;
      }
      lds_sync();
      const u32 bsel = uni(L.s.r[12]), exs = uni(L.s.r[13]);
      lds_sync();
      if (bsel == 0xffffffffu) break;  // cannot happen: nnan > k tokens lie in [kmin, kmax]
      target -= exs;
      const u32 nhi = hi - (bsel << sh);
      const u32 span = (1u << sh) - 1u;
      lo = (nhi - lo) > span ? nhi - span : lo;
      hi = nhi;
      if (sh == 0) {
        kk = hi;
        break;
      }
    }
  }
  auto wpk = [&](float q, u32 k) -> u32 {
    const u32 x = (k >= kk && k) ? wpack_of(q, k, qs, kmax, SH) : 0u;
    return x >= pthr ? x : 0u;
  };
  const int nseg = a.G * kWaves;
  QS_TRS(2);
  // ---- pass 2: weights, S, per-segment masses, the first bracket histogram
  Bracket br;
  br.mb0 = mass_bins_first(qs - f_of_key(kmin));
  br.lo = 0u;
  br.hi = 0xffffffffu;
  br.b0 = 0u;
  for (int b = threadIdx.x; b < kNB; b += kThreads) L.mh[b] = 0ull;
  lds_sync();
  u64 S = 0;
  u32 nz = 0;
  // With a finite maximum (every row with a finite q) the weights come from
  // d = q - qs without keys; mode 1 also drops the division (T = 1) and the
  // top-k and min-p tests (none set).  Mode 0 is the keyed form for a row
  // whose maximum is +inf or -inf.
  const int wmode = !(qs - qs == 0.0f) ? 0 : ((p.t_one && kk == 1u && thr == 0ull) ? 1 : 2);
  const float flmin = -(float)(SH + 40);
  const float qk = kk > 1u ? f_of_key(kk) : -__builtin_inff();  // q >= qk: key >= kk
  solo_pass<DT, VEC>(a, p, row, L, tv, [&](const Chunk<DT>& ch, int c) {
    with_pen(p.pen, [&](auto pen) {
      constexpr bool PEN = decltype(pen)::value;
      u32 pw[kEPT / 2] = {};
      if constexpr (PEN) chunk_counts(L, ch, c, pw);
      auto body = [&](auto mode) {
        constexpr int M = decltype(mode)::value;
        u64 sj = 0;  // the segment's mass
#pragma unroll
        for (int j = 0; j < J; ++j) {
#pragma unroll
          for (int e = 0; e < VL; ++e) {
            const float z = elem_zt<PEN>(ch, p, pw, j, e);
            u64 w;
            if constexpr (M == 0) {
              const float q = qdiv(z, p);
              const u32 k = skey(q);
              w = wunpack(wpk(q, k));
              if (p.topp && w) atomicAdd(&L.mh[mass_bin(q, k, qs, kmax, br.mb0)], w);
            } else {
              const float q = M == 1 ? z : qdiv(z, p);
              const float d = q - qs;
              w = weight_finite(d, flmin, SH);
              if constexpr (M == 2) w = (q >= qk && w >= thr) ? w : 0ull;
              if (p.topp && w) atomicAdd(&L.mh[mass_bin_first(d, br.mb0)], w);
            }
            sj += w;
            nz += w ? 1u : 0u;
          }
        }
        const u64 sw = wave_sum64(sj);
        if (lane_id() == 0) L.seg[c * kWaves + wave_id()] = sw;
        S += lane_id() == 0 ? sw : 0ull;
      };
      if (wmode == 1)
        body(ITag<1>{});
      else if (wmode == 2)
        body(ITag<2>{});
      else
        body(ITag<0>{});
    });
  });
  block_sum2(S, nz, L.s);
  S = uni64(S);
  nz = uni(nz);
  u64 W = S, A = 0, wt = 0;
  u32 klo = kk, idlo = (u32)a.V, kept = nz;  // without top-p: K, the tokens with key >= kk
  bool single = false;  // the bracket holds one key (too many tokens to list)
  u32 jties = 0u;
  if (p.topp) {
    QS_TRS(3);
    // ---- the bracket rounds
    const u64 Tp = mul_frac(S, p.tp);
    bool listed = false;
    u32 rlo = 0u, rhi = 0u;  // key range binned by the next key-space round
    for (int r = 0; r < kSoloRounds && !listed; ++r) {
      if (r > 0) {
        for (int b = threadIdx.x; b < kNB; b += kThreads) {
          L.mh[b] = 0ull;
          L.hc[b] = 0u;
        }
        lds_sync();
        const u32 lo = rlo, hi = rhi;
        const int bl = bitlen(hi - lo);
        const int sh = bl > 8 ? bl - 8 : 0;
        solo_pass<DT, VEC>(a, p, row, L, tv, [&](const Chunk<DT>& ch, int c) {
          with_pen(p.pen, [&](auto pen) {
            constexpr bool PEN = decltype(pen)::value;
            u32 pw[kEPT / 2] = {};
            if constexpr (PEN) chunk_counts(L, ch, c, pw);
#pragma unroll
            for (int j = 0; j < J; ++j)
#pragma unroll
              for (int e = 0; e < VL; ++e) {
                const float q = qdiv(elem_zt<PEN>(ch, p, pw, j, e), p);
                const u32 k = skey(q);
                if (k && k >= br.lo && k <= br.hi) {
                  const u64 w = wunpack(wpk(q, k));
                  if (w) {
                    const u32 b = key_bin(k, lo, hi, sh);
                    atomicAdd(&L.mh[b], w);
                    atomicAdd(&L.hc[b], 1u);
                  }
                }
              }
          });
        });
        lds_sync();
      }
      // the crossing bin
      const int b = threadIdx.x;
      const u64 bm = b < kNB ? L.mh[b] : 0ull;
      const u32 bc = (b < kNB && r > 0) ? L.hc[b] : 0u;
      u64 tot;
      const u64 ex = block_excl64(bm, L.s, &tot);
      const u64 target = Tp - A;
      if (threadIdx.x == 0) L.s.r[12] = 0xffffffffu;
      lds_sync();
      if (b < kNB && ex <= target && target < ex + bm) {
        L.s.r[12] = (u32)b;
        L.s.r64[12] = ex;
        u32 fits;
        if (r == 0) {
          const float wl = bin_least_weight(br.mb0, b, SH);
          fits = (float)bm <= wl * (float)kSoloList ? 1u : 0u;
        } else {
          fits = bc <= (u32)kSoloList ? 1u : 0u;
        }
        L.s.r[13] = fits;
        L.s.r[14] = bc;
      }
      lds_sync();
      const u32 bsel = uni(L.s.r[12]), fits = uni(L.s.r[13]), bcount = uni(L.s.r[14]);
      const u64 exs = uni64(L.s.r64[12]);
      lds_sync();
      if (bsel == 0xffffffffu) {  // cannot happen with exact sums: every row resolves below
        write_result(a, row, p, -1ll, 0, thr, kPathSolo, kStList, kmax, 0u, 0u, 0u);
        return;
      }
      A += exs;
      if (r == 0) {
        br.b0 = bsel;
        // the bin's exact key range: mass_bin falls as the key grows
        auto bin = [&](u32 k) { return mass_bin(f_of_key(k), k, qs, kmax, br.mb0); };
        u32 lo = kmin, hi = kmax;  // the largest key whose bin is >= bsel
        while (lo < hi) {
          const u32 mid = lo + (hi - lo + 1u) / 2u;
          if (bin(mid) >= bsel) lo = mid; else hi = mid - 1u;
        }
        br.hi = lo;
        lo = kmin;
        hi = kmax;  // the least key whose bin is <= bsel
        while (lo < hi) {
          const u32 mid = lo + (hi - lo) / 2u;
          if (bin(mid) <= bsel) hi = mid; else lo = mid + 1u;
        }
        br.lo = lo;
        rhi = br.hi;
        rlo = min(br.lo, rhi);
      } else {
        const int bl = bitlen(rhi - rlo);
        const int sh = bl > 8 ? bl - 8 : 0;
        const u32 nhi = rhi - (bsel << sh);
        const u32 span = (1u << sh) - 1u;
        const u32 nlo = (nhi - rlo) > span ? nhi - span : rlo;
        // the first and last bins also hold the bin-b0 keys past the binned range
        if (bsel != 0u) br.hi = min(br.hi, nhi);
        if (bsel != (u32)kNB - 1u) br.lo = max(br.lo, nlo);
        rhi = min(br.hi, kmax);
        rlo = min(max(br.lo, kmin), rhi);
        if (max(br.lo, kmin) == min(br.hi, kmax) && !fits) {
          single = true;  // one key, too many tokens to list
          jties = bcount;
          break;
        }
      }
      listed = fits != 0u;
    }
    if (!listed && !single) {  // a bracket still too wide after every round: cannot happen for 32-bit keys
      write_result(a, row, p, -1ll, 0, thr, kPathSolo, kStList, kmax, 0u, 0u, 0u);
      return;
    }
    QS_TRS(4);
    // ---- pass 3: the bracket's tokens listed, the mass above it per segment
    if (threadIdx.x == 0) L.nlist = 0u;
    for (int i = threadIdx.x; i < nseg; i += kThreads) L.segt[i] = 0u;
    lds_sync();
    // Each segment's mass above the bracket, and the bracket's tokens listed.
    // Each wave weighs one side per chunk: the tokens at or below the bracket
    // (their mass off the segment's total) or those above it and in it (the
    // mass above directly), the side that was the smaller in its previous
    // chunk, starting with the tokens at or below.  The weighed tokens
    // are compacted through LDS so that the lanes take them in turn, unless
    // there are more than kSoloCBuf of them, when the wave takes its elements
    // in place.
    u32 nab = 0;      // tokens at or below the bracket (not NaN)
    bool up = false;  // the wave weighs the tokens above the bracket
    // key <= br.hi as q <= qhi and key >= br.lo as q >= qlo (NaN fails every
    // test); no token has the key 0x7fffffff (skey folds -0 into +0), whose q
    // would be -0 and admit +0, and every key up to that of -inf (0x007fffff)
    // admits all but NaN
    const float qhi = f_of_key(br.hi == 0x7fffffffu ? 0x7ffffffeu : br.hi);
    const float qlo = br.lo <= 0x007fffffu ? -__builtin_inff() : f_of_key(br.lo);
    solo_pass<DT, VEC>(a, p, row, L, tv, [&](const Chunk<DT>& ch, int c) {
      with_pen(p.pen, [&](auto pen) {
        constexpr bool PEN = decltype(pen)::value;
        constexpr int E = kEPT;
        u32 pw[kEPT / 2] = {};
        if constexpr (PEN) chunk_counts(L, ch, c, pw);
        float qv[E];
        u32 set = 0;  // bit i: element i above or in the bracket (up), else at or below it
        if (up) {
          u32 nv = 0;  // not NaN
#pragma unroll
          for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < VL; ++e) {
              const int i = j * VL + e;
              qv[i] = qdiv(elem_zt<PEN>(ch, p, pw, j, e), p);
              set |= qv[i] >= qlo ? 1u << i : 0u;
              nv += qv[i] == qv[i] ? 1u : 0u;
            }
          nab += nv - (u32)__popc(set);  // below (the bracket's tokens are counted as taken)
        } else {
#pragma unroll
          for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < VL; ++e) {
              const int i = j * VL + e;
              qv[i] = qdiv(elem_zt<PEN>(ch, p, pw, j, e), p);
              set |= qv[i] <= qhi ? 1u << i : 0u;
            }
          nab += (u32)__popc(set);
        }
        const u32 cnt = (u32)__popc(set);
        const u32 incl = wave_incl_scan(cnt);
        const u32 total = readlane(incl, 63);
        const int sg = c * kWaves + wave_id();
        // one weighed token: its weight to (above) or off (at or below) its
        // segment's mass, and a bracket token listed (or counted, for a bracket
        // of one key); add(w) and tie() take the segment's share
        auto take = [&](float q, int j, int e, u32 lane, auto&& add, auto&& tie) {
          const u32 k = skey(q);
          const int side = bracket_side(br, k);
          const u64 w = wunpack(wpk(q, k));
          if (up ? side == 0 : true) add(w);
          if (up && side == 1) ++nab;
          if (side == 1 && w) {
            if (single) {
              tie();
            } else {
              const u32 slot = atomicAdd(&L.nlist, 1u);
              const int id = c * kCH + wave_id() * kWaveSpan + (int)lane * VL + j * 64 * VL + e;
              if (slot < (u32)kSoloList) L.u.fin.ent[slot] = ((u64)k << 32) | (u32)id;
            }
          }
        };
        if (total <= (u32)kSoloCBuf) {
          // lanes take tokens of any of the wave's elements: LDS atomics
          if (up && lane_id() == 0) L.seg[sg] = 0ull;
          u64* cb = L.cbuf[wave_id()];
          u32 pos = incl - cnt;
#pragma unroll
          for (int i = 0; i < E; ++i)
            if ((set >> i) & 1u) cb[pos++] = ((u64)__float_as_uint(qv[i]) << 32) | (lane_id() << 4) | (u32)i;
          // the wave's own LDS writes: complete before its lanes read each other's
          __builtin_amdgcn_s_waitcnt(0xC07F);
          auto add = [&](u64 w) {
            if (w) atomicAdd(&L.seg[sg], up ? w : (u64)0 - w);
          };
          auto tie = [&]() { atomicAdd(&L.segt[sg], 1u); };
          for (u32 x = lane_id(); x < total; x += 64) {
            const u64 en = cb[x];
            const u32 i = (u32)en & 15u;
            take(__uint_as_float((u32)(en >> 32)), (int)(i / VL), (int)(i % VL), ((u32)en >> 4) & 63u, add, tie);
          }
          __builtin_amdgcn_s_waitcnt(0xC07F);  // read before the next chunk writes the buffer again
        } else {
          // in place: the segment's share summed in registers
          auto tie = [&]() { atomicAdd(&L.segt[sg], 1u); };
          u64 sj = 0;
          auto add = [&](u64 w) { sj += w; };
#pragma unroll
          for (int j = 0; j < J; ++j)
#pragma unroll
            for (int e = 0; e < VL; ++e)
              if ((set >> (j * VL + e)) & 1u) take(qv[j * VL + e], j, e, lane_id(), add, tie);
          const u64 sw = wave_sum64(sj);
          if (lane_id() == 0) L.seg[sg] = up ? sw : L.seg[sg] - sw;
        }
        // the next chunk weighs the other side when this one took more than half
        if (total > 32u * (u32)E) up = !up;
      });
    });
    const u32 na = nnan - block_sum(nab, L.s);  // tokens above the bracket
    if (!single) {
      const u32 n = uni(L.nlist);
      if (n > (u32)kSoloList || n == 0u) {  // the bound was exceeded: cannot happen
        write_result(a, row, p, -1ll, 0, thr, kPathSolo, kStOverflow, kmax, 0u, 0u, 0u);
        return;
      }
      Held h;
      hold_entries(L, n, h);
      u32 wq[kFPer];
#pragma unroll
      for (int i = 0; i < kFPer; ++i) {
        const u32 k = (u32)(h.e[i] >> 32);
        wq[i] = ((u32)i < h.per && k) ? wpk(f_of_key(k), k) : 0u;
      }
      const SelRes q = held_select<true>(a, L, h, wq, max(max(br.lo, kmin), 1u), min(br.hi, kmax), Tp - A);
      if (!q.ok) {
        write_result(a, row, p, -1ll, 0, thr, kPathSolo, kStList, kmax, 0u, 0u, 0u);
        return;
      }
      klo = q.kappa;
      wt = wunpack(wpk(f_of_key(klo), klo));
      const u64 jj = div_small(Tp - A - q.mass_above, wt) + 1ull;
      jties = (u32)(jj < (u64)q.cnt_at ? jj : (u64)q.cnt_at);
      W = A + q.mass_above + (u64)jties * wt;
      kept = na + q.cnt_above + jties;
      idlo = (u32)a.V;
      if (jties < q.cnt_at) {
        // the jties-th tie in id order: the jties-th largest of ~id among the ties
        Held t;
        t.per = h.per;
#pragma unroll
        for (int i = 0; i < kFPer; ++i) {
          const u32 k = (u32)(h.e[i] >> 32), id = (u32)h.e[i];
          t.e[i] = (wq[i] && k == klo) ? (((u64)(~id) << 32) | id) : 0ull;
        }
        const SelRes r = held_select<false>(a, L, t, wq, ~(u32)(a.V - 1), 0xffffffffu, (u64)jties);
        if (!r.ok) {
          write_result(a, row, p, -1ll, 0, thr, kPathSolo, kStList, kmax, 0u, 0u, 0u);
          return;
        }
        idlo = ~r.kappa;
      }
      // kept mass per segment: above the bracket, plus the listed tokens kept
#pragma unroll
      for (int i = 0; i < kFPer; ++i) {
        if ((u32)i < h.per && wq[i]) {
          const u32 k = (u32)(h.e[i] >> 32), id = (u32)h.e[i];
          if (k > klo || (k == klo && id <= idlo)) atomicAdd(&L.seg[solo_seg_of((int)id)], wunpack(wq[i]));
        }
      }
      lds_sync();
    } else {
      // a bracket of one key: every token in it weighs wt; the first jties in id order are kept
      klo = min(br.hi, kmax);
      wt = wunpack(wpk(f_of_key(klo), klo));
      const u32 cnt_at = jties;
      const u64 jj = div_small(Tp - A, wt) + 1ull;
      jties = (u32)(jj < (u64)cnt_at ? jj : (u64)cnt_at);
      W = A + (u64)jties * wt;
      kept = na + jties;
      idlo = (u32)a.V;
      if (jties < cnt_at) {
        // the segment holding the jties-th tie, then its id from one wave's re-read
        u32 c0 = threadIdx.x * 2 < (u32)nseg ? L.segt[threadIdx.x * 2] : 0u;
        u32 c1 = threadIdx.x * 2 + 1 < (u32)nseg ? L.segt[threadIdx.x * 2 + 1] : 0u;
        u32 ctot;
        const u32 cx = block_excl(c0 + c1, L.s, &ctot);
        if (threadIdx.x == 0) L.s.r[12] = 0xffffffffu;
        lds_sync();
        const u32 jt = jties - 1u;  // ties before the wanted one
        if (cx <= jt && jt < cx + c0) {
          L.s.r[12] = threadIdx.x * 2;
          L.s.r[13] = jt - cx;
        } else if (cx + c0 <= jt && jt < cx + c0 + c1) {
          L.s.r[12] = threadIdx.x * 2 + 1;
          L.s.r[13] = jt - cx - c0;
        }
        lds_sync();
        const u32 sg = uni(L.s.r[12]), within = uni(L.s.r[13]);
        lds_sync();
        if (sg == 0xffffffffu) {
          write_result(a, row, p, -1ll, 0, thr, kPathSolo, kStList, kmax, 0u, 0u, 0u);
          return;
        }
        if (p.pen) pen_build(p, (int)sg / kWaves, L);
        if (threadIdx.x < 64) {
          const long long id = solo_seg_find<DT>(a, p, row, L, (int)sg, (u64)within, [&](float z, int) -> u64 {
            const float q = qdiv(z, p);
            const u32 k = skey(q);
            return (k == klo && wpk(q, k)) ? 1ull : 0ull;
          });
          if (threadIdx.x == 0) L.s.r[15] = (u32)id;
        }
        lds_sync();
        idlo = L.s.r[15];
        lds_sync();
      }
      // kept mass per segment: above, plus the ties up to the jties-th
      // ties before segment s in id order (exclusive), capped at jties
      {
        const u32 s0 = threadIdx.x * 2, s1 = s0 + 1;
        u32 c0 = s0 < (u32)nseg ? L.segt[s0] : 0u;
        u32 c1 = s1 < (u32)nseg ? L.segt[s1] : 0u;
        u32 ctot;
        const u32 cx = block_excl(c0 + c1, L.s, &ctot);
        const u32 k0 = min(c0, jties > cx ? jties - cx : 0u);
        const u32 cx1 = cx + c0;
        const u32 k1 = min(c1, jties > cx1 ? jties - cx1 : 0u);
        if (s0 < (u32)nseg) L.seg[s0] += (u64)k0 * wt;
        if (s1 < (u32)nseg) L.seg[s1] += (u64)k1 * wt;
      }
      lds_sync();
    }
  }
  QS_TRS(5);
  // ---- the draw: the segment holding t, then the token inside it
  const u64 t = mul_frac(W, p.u);
  {
    const u32 s0 = threadIdx.x * 2, s1 = s0 + 1;
    const u64 m0 = s0 < (u32)nseg ? L.seg[s0] : 0ull, m1 = s1 < (u32)nseg ? L.seg[s1] : 0ull;
    u64 mt;
    const u64 mx = block_excl64(m0 + m1, L.s, &mt);
    if (threadIdx.x == 0) L.s.r[12] = 0xffffffffu;
    lds_sync();
    if (mx <= t && t < mx + m0) {
      L.s.r[12] = s0;
      L.s.r64[12] = t - mx;
    } else if (mx + m0 <= t && t < mx + m0 + m1) {
      L.s.r[12] = s1;
      L.s.r64[12] = t - mx - m0;
    }
    lds_sync();
  }
  const u32 sg = uni(L.s.r[12]);
  const u64 tin = uni64(L.s.r64[12]);
  lds_sync();
  if (sg == 0xffffffffu) {
    write_result(a, row, p, -1ll, 0, thr, kPathSolo, kStIncomplete, kmax, 0u, 0u, 0u);
    return;
  }
  if (p.pen) pen_build(p, (int)sg / kWaves, L);
  if (threadIdx.x < 64) {
    const bool topp = p.topp;
    const long long id = solo_seg_find<DT>(a, p, row, L, (int)sg, tin, [&](float z, int i) -> u64 {
      const float q = qdiv(z, p);
      const u32 k = skey(q);
      const u64 w = wunpack(wpk(q, k));
      if (!topp) return w;
      return (k > klo || (k == klo && (u32)i <= idlo)) ? w : 0ull;
    });
    if (threadIdx.x == 0) L.s.r[15] = (u32)(id < 0 ? 0xffffffffu : (u32)id);
  }
  lds_sync();
  const u32 pick = L.s.r[15];
  write_result(a, row, p, pick == 0xffffffffu ? -1ll : (long long)pick, W, thr, kPathSolo,
               pick == 0xffffffffu ? kStIncomplete : 0u, kmax, klo, idlo, kept);
  QS_TRS(6);
}

}  // namespace qs
