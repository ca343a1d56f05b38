// Kernels of the sampler (one launch per call).  Included by qsampler.hip.
//
// Grid (G, B): workgroup (c, s) streams chunk c (kCH logits) of row
// order[s] (s itself without an order) into registers once, applies the
// history penalties from an LDS count table, and plays its row's role:
//   greedy  local argmax, published to the chunk's slot;
//   top-k   the chunk's tokens at or above a threshold taken from its
//           per-thread maxima, written in id order to the chunk's region;
//   mass    (top-k off) keys of q in registers; one row barrier exchanges the
//           chunk maxima (the row maximum q* anchors the weights); with top-p
//           each workgroup publishes a 256-bin mass histogram and the last one
//           to arrive (the reducer) picks the bin that holds the top-p
//           boundary; then every workgroup publishes its mass above that bin
//           and lists its tokens inside it.
// Every workgroup then counts its arrival; the last workgroup of a row
// resolves the row (top-k, min_p, top-p and the draw) from what the others
// published, writes the id and returns the row's counters to zero.  Rows the
// fast paths cannot serve exactly (top-k above kTopkMax, a region or list
// overflow, an incomplete candidate set, a barrier time-out) are resolved by
// that last workgroup alone with exact passes over the row.
#pragma once
#include "qs_device.hpp"
#include "qsampler.h"

namespace qs {

constexpr int kCH = 8192;                  // logits per chunk (one workgroup)
constexpr int kEPT = kCH / kThreads;       // logits per thread
constexpr int kWaveSpan = kCH / kWaves;    // contiguous ids per wave
constexpr int kMaxG = 256;                 // chunks per row
constexpr int kRegionTotal = 8192;         // top-k candidate entries per row (G * R)
constexpr int kTopkMax = QS_TOPK_FAST_MAX; // top-k served from candidates
constexpr int kFCap = 4096;                // gathered entries per row
constexpr int kFPer = kFCap / kThreads;    // of them per finishing thread
constexpr int kDirect = kThreads / 8;      // a selection bin this small is resolved by direct ranking
constexpr int kNB = 256;                   // mass histogram bins (one per thread)
constexpr int kRounds = 3;                 // bracket rounds before the exact path
constexpr int kLC = 256;                   // bracket entries per chunk
constexpr int kNBS = 1024;                 // select histogram bins
constexpr int kRegionCap = 1024;           // candidate entries of one chunk at most

enum : u32 { kStOverflow = 1u, kStIncomplete = 2u, kStTimeout = 4u, kStList = 8u };
constexpr u32 kWhyLargeK = 16u;          // top-k above kTopkMax
constexpr u32 kNotLast = 0xffffffffu;    // not the row's last workgroup
enum : u32 { kKindGreedy = 0, kKindTopK = 1, kKindMass = 2, kKindSingle = 3 };
// How the last call resolved a row (RowRes::path).
enum : u32 { kPathGreedy = 1, kPathTopK = 2, kPathMassTopP = 3, kPathMassAll = 4, kPathSingle = 5, kPathSolo = 6 };

// Per-row counters, each on its own 128-byte line.  Zero between calls.
struct __attribute__((aligned(128))) RowSync {
  u32 arrive;  u32 p0[31];
  u32 status;  u32 p1[31];
  u32 barA;    u32 p2[31];
  u32 barB;    u32 p3[31];
  u32 dec;     u32 p4[31];
};
// Per-row result of the last call (read by k_probs and by the tests).
struct __attribute__((aligned(128))) RowRes {
  long long id;
  u64 W, thr;       // kept mass, min_p threshold on weights
  u64 Tp, S, Ahi;   // mass rows with top-p: floor(top_p * S), S, mass above the boundary bin
  u32 kind, path, why;
  u32 kstar;        // key of q*
  u32 klo, idlo;    // kept iff key > klo || (key == klo && id <= idlo), and weight > 0
  u32 kept;
  u32 pad[13];
};
static_assert(sizeof(RowRes) == 128, "row result is 128 bytes");
// Per-(row, chunk) published values.
struct __attribute__((aligned(32))) Slot {
  u64 a;  // greedy: (gkey << 32 | ~id); top-k: (below << 32 | n); mass: (kmax << 32 | kmin)
  u64 b;  // mass: S_c (total weight), then mass above the boundary bin
  u64 c;  // mass: count of nonzero weights; then (n listed << 32 | count above)
  u64 d;
};

struct Args {
  const void* logits;
  long long row_stride;
  int B, V, G, R, SH, H;
  int vec_ok;
  float kmu;  // kCH / V: the share of a row's top k that a chunk holds on average
  u32 flags, spin_limit;
  const float* temperature;
  const float* top_p;
  const int* top_k;
  const float* min_p;
  const float* rep;
  const float* pres;
  const float* freq;
  const int* hist;       // [B, H]
  const int* hist_len;   // [B] or null: row r uses hist[r, 0:hist_len[r]]
  const float* uniforms;
  const int* order;      // [B] or null
  long long* out_ids;
  float* out_probs;
  int* out_kept;
  RowSync* sync;
  RowRes* res;
  Slot* slots;  // [B, kMaxG]
  u64* data;    // [B, data_per_row]
  long long data_per_row;  // u64 entries
  u64* trace;   // trace builds only: [B, G, 32] phase time stamps
};

#ifdef QS_TRACE
#define QS_TR(i)                                                                             \
  do {                                                                                       \
    if (a.trace && threadIdx.x == 0) a.trace[((size_t)row * a.G + c) * 32 + (i)] = wall_clock64(); \
  } while (0)
// the same from code that has the arguments but not the row (slot of dispatch position blockIdx.y)
#define QS_TRA(i)                                                                                     \
  do {                                                                                                \
    if (a.trace && threadIdx.x == 0) {                                                                \
      a.trace[((size_t)blockIdx.y * a.G + blockIdx.x) * 32 + (i)] = wall_clock64();                  \
    }                                                                                                 \
  } while (0)
#else
#define QS_TR(i) \
  do {           \
  } while (0)
#define QS_TRA(i) \
  do {            \
  } while (0)
#endif

struct RowP {
  float T, rT, tp, mp, rep, rrep, pres, freq, u;
  int k, kind, hlen;
  u32 dspan;  // qdiv's range of |z| bits for the fast division (0: none)
  bool t_one, topp, pen;
  const int* hist;
};

// Row parameters, moved to scalar registers: every branch on them is uniform.
__device__ __forceinline__ float unif(float v) { return __uint_as_float(uni(__float_as_uint(v))); }
__device__ __forceinline__ RowP row_params(const Args& a, int row) {
  RowP p;
  row = (int)uni((u32)row);
  p.T = a.temperature ? unif(sld(a.temperature + row)) : 0.0f;
  const bool greedy = (a.flags & QS_FLAG_ALL_GREEDY) || (p.T <= 1e-5f);
  p.k = a.top_k ? (int)uni((u32)sld(a.top_k + row)) : 0;
  const bool topk_on = p.k > 0 && p.k < a.V;
  p.tp = ((a.flags & QS_FLAG_USE_TOP_P) && a.top_p) ? unif(sld(a.top_p + row)) : 1.0f;
  // the flags from the bit patterns, by scalar integer compares (a float compare
  // runs on the vector unit and leaves a 64-bit lane mask in scalar registers)
  const u32 tpb = __float_as_uint(p.tp);
  p.topp = (int)tpb < 0x3f800000 && (tpb & 0x7fffffffu) <= 0x7f800000u;  // tp < 1 (not NaN)
  p.mp = a.min_p ? unif(sld(a.min_p + row)) : 0.0f;
  p.rep = a.rep ? unif(sld(a.rep + row)) : 1.0f;
  p.rrep = 1.0f / p.rep;
  p.pres = a.pres ? unif(sld(a.pres + row)) : 0.0f;
  p.freq = a.freq ? unif(sld(a.freq + row)) : 0.0f;
  p.hlen = a.hist ? (a.hist_len ? (int)uni((u32)sld(a.hist_len + row)) : a.H) : 0;
  if (p.hlen > a.H) p.hlen = a.H;
  if (p.hlen < 0) p.hlen = 0;
  p.hist = a.hist ? a.hist + (size_t)row * a.H : nullptr;
  p.pen = p.hist != nullptr && p.hlen > 0 &&
          (__float_as_uint(p.rep) != 0x3f800000u || (__float_as_uint(p.pres) & 0x7fffffffu) != 0u ||
           (__float_as_uint(p.freq) & 0x7fffffffu) != 0u);  // rep != 1, pres != 0 or freq != 0
  p.u = a.uniforms ? unif(sld(a.uniforms + row)) : 0.0f;
  if (!(p.u >= 0.0f)) p.u = 0.0f;
  if (p.u >= 1.0f) p.u = __uint_as_float(0x3f7fffffu);
  p.kind = greedy ? kKindGreedy : (topk_on ? (p.k <= kTopkMax ? kKindTopK : kKindSingle) : kKindMass);
  p.t_one = __float_as_uint(p.T) == 0x3f800000u;  // T == 1
  p.rT = 1.0f / p.T;
  // T in [2^-16, 2^16]: |z| in [2^-80, 2^80) keeps |z * rT| in [2^-100, 2^100)
  p.dspan = __float_as_uint(p.T) - 0x37800000u <= 0x10000000u ? 0x50000000u : 0u;
  return p;
}

// The contract's q = z / T (one IEEE division) of the row: z itself for T = 1,
// else the fast division (div_fast) where div_fast_ok holds by the ranges of z
// and T alone, the division otherwise.
__device__ __forceinline__ float qdiv(float z, const RowP& p) {
  if (p.t_one) return z;
  return (__float_as_uint(z) & 0x7fffffffu) - 0x17800000u < p.dspan ? div_fast(z, p.T, p.rT) : z / p.T;
}

// ---------------------------------------------------------------- LDS

struct SelLds {
  u32 hc[kNBS];
  u64 hm[kNBS];
};
struct FinLds {
  u64 ent[kFCap];           // gathered entries (key << 32 | id), in id order
  u32 lk[kDirect];          // a bin's keys for the direct resolution
  u64 lw[kDirect];          // and their weights
};
constexpr int kSegPre = 1024;  // segment masses a mass row's finisher loads with its lists
struct Lds {
  union {
    u32 pen[kCH / 2];       // history counts of the chunk, two 16-bit counts per word
    u32 kq[kCH];            // top-k-off rows: keys of q, element i of thread t at i * kThreads + t
    FinLds fin;             // the finishing workgroup's candidates
  } u;
  SelLds sel;               // select histogram (beside the table: the exact pass needs both)
  u64 mh[kNB];              // mass histogram of the chunk
  u64 segm[kSegPre];        // finisher: every chunk's segment masses (when they fit)
  u64 cmass[kMaxG];         // finisher: per-chunk masses
  u32 cties[kMaxG];         // finisher: per-chunk tie counts
  u32 coff[kMaxG + 1];      // finisher: gathered offsets per chunk
  Scratch s;
};

// ---------------------------------------------------------------- chunk in registers

template <int DT>
struct Chunk {
  static constexpr int VL = DT == QS_DTYPE_F32 ? 4 : 8;  // logits per 16-byte vector
  static constexpr int J = kEPT / VL;                    // vectors per thread
  uint4 v[J];
  int nval;  // valid logits of this thread's span: element (j, e) is valid iff j*64*VL + e < nval
  int base;  // id of element (0, 0)
  __device__ __forceinline__ int id(int j, int e) const { return base + j * 64 * VL + e; }
  __device__ __forceinline__ bool valid(int j, int e) const { return j * 64 * VL + e < nval; }
  __device__ __forceinline__ float raw(int j, int e) const {
    const uint4 q = v[j];
    if (DT == QS_DTYPE_F32) {
      const u32 w = e == 0 ? q.x : e == 1 ? q.y : e == 2 ? q.z : q.w;
      return __uint_as_float(w);
    }
    const u32 w = (e >> 1) == 0 ? q.x : (e >> 1) == 1 ? q.y : (e >> 1) == 2 ? q.z : q.w;
    return bf16_to_f32((e & 1) ? (w >> 16) : (w & 0xffffu));
  }
};

// Issue the loads of chunk c of a row (no wait).
template <int DT>
__device__ __forceinline__ void load_chunk(const Args& a, int row, int c, Chunk<DT>& ch) {
  constexpr int VL = Chunk<DT>::VL;
  const int l = lane_id(), w = wave_id();
  ch.base = c * kCH + w * kWaveSpan + l * VL;
  ch.nval = a.V - ch.base;
  const size_t rowoff = (size_t)row * (size_t)a.row_stride;
#pragma unroll
  for (int j = 0; j < Chunk<DT>::J; ++j) {
    const int i0 = ch.base + j * 64 * VL;
    if (a.vec_ok && i0 + VL <= a.V) {
      if (DT == QS_DTYPE_F32)
        ch.v[j] = gld((const uint4*)((const float*)a.logits + rowoff + i0));
      else
        ch.v[j] = gld((const uint4*)((const uint16_t*)a.logits + rowoff + i0));
    } else {
      // past V: NaN, whose key of q is 0 (no weight, never a candidate)
      const u32 pad = DT == QS_DTYPE_F32 ? 0x7fc00000u : 0x7fc07fc0u;
      u32 x[4] = {pad, pad, pad, pad};
      if (DT == QS_DTYPE_F32) {
        const float* p = (const float*)a.logits + rowoff;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (i0 + e < a.V) x[e] = __float_as_uint(gld(p + i0 + e));
      } else {
        const uint16_t* p = (const uint16_t*)a.logits + rowoff;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (i0 + e < a.V)
            x[e >> 1] = (x[e >> 1] & ~(0xffffu << ((e & 1) * 16))) | ((u32)gld(p + i0 + e) << ((e & 1) * 16));
      }
      ch.v[j] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  }
}

// The chunk's history-count table (two 16-bit counts per word) of an LDS layout.
__device__ __forceinline__ u32* pen_table(Lds& L) { return L.u.pen; }
__device__ __forceinline__ const u32* pen_table(const Lds& L) { return L.u.pen; }
// The i-th history id of the row (overloads may keep a copy in LDS).
__device__ __forceinline__ int hist_id(const RowP& p, const Lds&, int i) { return gld(p.hist + i); }

// History counts of the ids in [c*kCH, (c+1)*kCH) into the LDS table.
template <typename LT>
__device__ __forceinline__ void pen_build(const RowP& p, int c, LT& L) {
  u32* t = pen_table(L);
  uint4* t4 = (uint4*)t;
  for (int i = threadIdx.x; i < kCH / 8; i += kThreads) t4[i] = make_uint4(0u, 0u, 0u, 0u);
  lds_sync();
  const int lo = c * kCH;
  for (int i = threadIdx.x; i < p.hlen; i += kThreads) {
    const int d = hist_id(p, L, i) - lo;
    if ((unsigned)d < (unsigned)kCH) atomicAdd(&t[d >> 1], (d & 1) ? 0x10000u : 1u);
  }
  lds_sync();
}
// The same with the first kHistPre * kThreads history ids already loaded (pre[i]
// is id threadIdx.x + i * kThreads, loaded beside the chunk so that the table
// costs no further round trip).
constexpr int kHistPre = 8;
__device__ __forceinline__ void pen_build_pre(const RowP& p, int c, Lds& L, const int (&pre)[kHistPre]) {
  u32* t = pen_table(L);
  uint4* t4 = (uint4*)t;
  for (int i = threadIdx.x; i < kCH / 8; i += kThreads) t4[i] = make_uint4(0u, 0u, 0u, 0u);
  lds_sync();
  const int lo = c * kCH;
#pragma unroll
  for (int k = 0; k < kHistPre; ++k) {
    const int i = (int)threadIdx.x + k * kThreads;
    const int d = pre[k] - lo;
    if (i < p.hlen && (unsigned)d < (unsigned)kCH) atomicAdd(&t[d >> 1], (d & 1) ? 0x10000u : 1u);
  }
  for (int i = threadIdx.x + kHistPre * kThreads; i < p.hlen; i += kThreads) {
    const int d = gld(p.hist + i) - lo;
    if ((unsigned)d < (unsigned)kCH) atomicAdd(&t[d >> 1], (d & 1) ? 0x10000u : 1u);
  }
  lds_sync();
}
// Count of element (j, e) of the thread from the table.
template <int DT, typename LT>
__device__ __forceinline__ u32 pen_count(const LT& L, const Chunk<DT>& ch, int c, int j, int e) {
  const int li = ch.base - c * kCH + j * 64 * Chunk<DT>::VL + e;
  return (pen_table(L)[li >> 1] >> ((li & 1) * 16)) & 0xffffu;
}
// z of element (j, e): the logit with the penalties applied.
template <int DT, typename LT>
__device__ __forceinline__ float elem_z(const Chunk<DT>& ch, const RowP& p, const LT& L, int c, int j, int e) {
  float z = ch.raw(j, e);
  if (p.pen) {
    const u32 n = pen_count(L, ch, c, j, e);
    if (n) z = apply_penalty(z, n, p.rep, p.rrep, p.pres, p.freq);
  }
  return z;
}
// The history counts of the thread's elements, two per word as in the table
// (element j*VL + e in word (j*VL + e) / 2): one vector LDS read per vector.
template <int DT, typename LT>
__device__ __forceinline__ void chunk_counts(const LT& L, const Chunk<DT>& ch, int c, u32 (&pw)[kEPT / 2]) {
  constexpr int VL = Chunk<DT>::VL;
#pragma unroll
  for (int j = 0; j < Chunk<DT>::J; ++j) {
    const int li = ch.base - c * kCH + j * 64 * VL;  // a multiple of VL
    if (VL == 8) {
      const uint4 w = *(const uint4*)&pen_table(L)[li >> 1];
      pw[j * 4 + 0] = w.x;
      pw[j * 4 + 1] = w.y;
      pw[j * 4 + 2] = w.z;
      pw[j * 4 + 3] = w.w;
    } else {
      const uint2 w = *(const uint2*)&pen_table(L)[li >> 1];
      pw[j * 2 + 0] = w.x;
      pw[j * 2 + 1] = w.y;
    }
  }
}
// z of element (j, e) with the counts from chunk_counts.
template <int DT>
__device__ __forceinline__ float elem_zc(const Chunk<DT>& ch, const RowP& p, const u32 (&pw)[kEPT / 2], int j, int e) {
  float z = ch.raw(j, e);
  if (p.pen) {
    const int i = j * Chunk<DT>::VL + e;
    const u32 n = (pw[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
    if (n) z = apply_penalty(z, n, p.rep, p.rrep, p.pres, p.freq);
  }
  return z;
}
// The row's penalty flag as a compile-time constant: f(Tag<p.pen>()), so that
// the per-element loops test it once.
template <bool B>
struct Tag {
  static constexpr bool value = B;
};
template <typename F>
__device__ __forceinline__ void with_pen(bool pen, F&& f) {
  if (pen)
    f(Tag<true>{});
  else
    f(Tag<false>{});
}
template <int M>
struct ITag {
  static constexpr int value = M;
};
// elem_zc with the penalty flag known at compile time.
template <bool PEN, int DT>
__device__ __forceinline__ float elem_zt(const Chunk<DT>& ch, const RowP& p, const u32 (&pw)[kEPT / 2], int j, int e) {
  float z = ch.raw(j, e);
  if constexpr (PEN) {
    const int i = j * Chunk<DT>::VL + e;
    const u32 n = (pw[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
    if (n) z = apply_penalty(z, n, p.rep, p.rrep, p.pres, p.freq);
  }
  return z;
}
// Keys of q = z / T for every element (0 for NaN and invalid elements).
template <int DT, typename LT>
__device__ __forceinline__ void chunk_qkeys(const Chunk<DT>& ch, const RowP& p, const LT& L, int c, u32 (&kq)[kEPT]) {
  with_pen(p.pen, [&](auto pen) {
    constexpr bool PEN = decltype(pen)::value;
    u32 pw[kEPT / 2] = {};
    if constexpr (PEN) chunk_counts(L, ch, c, pw);
#pragma unroll
    for (int j = 0; j < Chunk<DT>::J; ++j)
#pragma unroll
      for (int e = 0; e < Chunk<DT>::VL; ++e) {
        const float q = qdiv(elem_zt<PEN>(ch, p, pw, j, e), p);
        kq[j * Chunk<DT>::VL + e] = skey(q);  // 0 past V (NaN padding)
      }
  });
}

// ---------------------------------------------------------------- row synchronisation

// Count this workgroup in *ctr after its stores completed; returns the count
// before it (to every thread).
__device__ __forceinline__ u32 arrive(u32* ctr, Scratch& s) {
  wait_mem();
  lds_sync();
  if (threadIdx.x == 0) s.r[0] = addc(ctr, 1u);
  lds_sync();
  return s.r[0];
}
// The same counting n (the chunks this workgroup served).
__device__ __forceinline__ u32 arrive_n(u32* ctr, u32 n, Scratch& s) {
  wait_mem();
  lds_sync();
  if (threadIdx.x == 0) s.r[0] = addc(ctr, n);
  lds_sync();
  return s.r[0];
}
// Thread 0 waits until *ctr >= target (or the row failed / the limit passed).
// Returns true when the target was reached, to every thread.
__device__ __forceinline__ bool wait_count(const Args& a, int row, const u32* ctr, u32 target, Scratch& s) {
  if (threadIdx.x == 0) {
    bool ok = false;
    if (a.spin_limit == 0u) orc(&a.sync[row].status, kStTimeout);  // the test hook: give up at once
    for (u32 it = 0; a.spin_limit != 0u; ++it) {
      const u32 v = ldc(ctr), st = ldc(&a.sync[row].status);
      if (v >= target) {
        ok = true;
        break;
      }
      if (st != 0u) break;
      if (it >= a.spin_limit) {
        orc(&a.sync[row].status, kStTimeout);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
    s.r[1] = ok ? 1u : 0u;
  }
  lds_sync();
  return s.r[1] != 0u;
}
__device__ __forceinline__ void fail_row(const Args& a, int row, u32 why) {
  if (threadIdx.x == 0) orc(&a.sync[row].status, why);
}
// The last workgroup of a row returns the row's counters to zero.
__device__ __forceinline__ void reset_row(const Args& a, int row) {
  if (threadIdx.x == 0) {
    RowSync* y = &a.sync[row];
    stc(&y->arrive, 0u);
    stc(&y->status, 0u);
    stc(&y->barA, 0u);
    stc(&y->barB, 0u);
    stc(&y->dec, 0u);
  }
}
__device__ __forceinline__ u64* row_data(const Args& a, int row) { return a.data + (size_t)row * a.data_per_row; }
__device__ __forceinline__ Slot* row_slots(const Args& a, int row) { return a.slots + (size_t)row * kMaxG; }

__device__ __forceinline__ void write_result(const Args& a, int row, const RowP& p, long long id, u64 W, u64 thr,
                                             u32 path, u32 why, u32 kstar, u32 klo, u32 idlo, u32 kept) {
  if (threadIdx.x == 0) {
    gst(a.out_ids + row, id);
    if (a.out_kept) gst(a.out_kept + row, (int)kept);
    RowRes* r = &a.res[row];
    gst(&r->id, id);
    gst(&r->W, W);
    gst(&r->thr, thr);
    gst(&r->kind, (u32)p.kind);
    gst(&r->path, path);
    gst(&r->why, why);
    gst(&r->kstar, kstar);
    gst(&r->klo, klo);
    gst(&r->idlo, idlo);
    gst(&r->kept, kept);
  }
}

// ---------------------------------------------------------------- selection over a set of (key, weight)
//
// Finds, among items with key in a range, the key kappa at which a running
// total (counts, or weights) taken in key-descending order crosses a target:
// total(key > kappa) <= target < total(key >= kappa) for weights, and
// count(key > kappa) < target <= count(key >= kappa) for counts.  Each round
// histograms the range into kNBS bins of 2^s keys (s chosen so the range
// fits), finds the crossing bin and narrows to it; the last round has bins of
// one key.  Items are fed by the caller through add(); rounds() drives it.
struct Sel {
  u32 hi, lo;   // current key range [lo, hi]
  int s;        // bin width 2^s
  bool by_mass;
  u64 target;   // remaining target inside the range
  u64 above_m;  // weight above the range (accumulated)
  u32 above_c;  // count above the range
  u32 found;    // 1 when kappa is found
  u32 kappa, kcount;  // result and its multiplicity
  u64 kmass;          // weight of the items at kappa
};
__device__ __forceinline__ void sel_init(Sel& q, u32 lo, u32 hi, bool by_mass, u64 target) {
  q.lo = lo;
  q.hi = hi;
  const u32 width = hi - lo;  // + 1 keys
  const int bits = bitlen(width);
  q.s = bits > 10 ? bits - 10 : 0;
  q.by_mass = by_mass;
  q.target = target;
  q.above_m = 0;
  q.above_c = 0;
  q.found = 0;
  q.kappa = 0;
  q.kcount = 0;
  q.kmass = 0;
}
__device__ __forceinline__ void sel_clear(Lds& L) {
  for (int i = threadIdx.x; i < kNBS; i += kThreads) {
    L.sel.hc[i] = 0u;
    L.sel.hm[i] = 0ull;
  }
}
__device__ __forceinline__ void sel_add(const Sel& q, Lds& L, u32 key, u64 w) {
  if (key >= q.lo && key <= q.hi) {
    const u32 b = (q.hi - key) >> q.s;
    atomicAdd(&L.sel.hc[b], 1u);
    if (w) atomicAdd(&L.sel.hm[b], w);
  }
}
// After the items of a round were added (and lds_sync'd): find the crossing
// bin, narrow the range.  Returns true when kappa is found.
__device__ __forceinline__ bool sel_step(Sel& q, Lds& L) {
  constexpr int P = kNBS / kThreads;
  const int b0 = threadIdx.x * P;
  u32 c = 0;
  u64 m = 0;
  u32 hc[P];
  u64 hm[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    hc[i] = L.sel.hc[b0 + i];
    hm[i] = L.sel.hm[b0 + i];
    c += hc[i];
    m += hm[i];
  }
  u32 ctot;
  u64 mtot;
  block_excl2(c, m, L.s, &ctot, &mtot);
  // crossing bin: the first (in key-descending order) whose inclusive total passes the target
  if (threadIdx.x == 0) L.s.r[4] = 0xffffffffu;
  lds_sync();
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const bool hit = q.by_mass ? (m <= q.target && q.target < m + hm[i]) : (c < q.target && q.target <= c + hc[i]);
    if (hit) {
      L.s.r[4] = (u32)(b0 + i);
      L.s.r64[4] = m;
      L.s.r[5] = c;
      L.s.r[6] = hc[i];
      L.s.r64[5] = hm[i];
    }
    c += hc[i];
    m += hm[i];
  }
  lds_sync();
  const u32 b = L.s.r[4];
  if (b == 0xffffffffu) {  // no crossing: the target is beyond the range's total
    q.found = 2;
    lds_sync();
    return true;
  }
  const u64 mb = L.s.r64[4], hmb = L.s.r64[5];
  const u32 cb = L.s.r[5], hcb = L.s.r[6];
  lds_sync();
  q.above_m += mb;
  q.above_c += cb;
  if (q.by_mass)
    q.target -= mb;
  else
    q.target -= cb;
  const u32 nhi = q.hi - (b << q.s);
  const u32 span = (1u << q.s) - 1u;
  const u32 nlo = (nhi - q.lo) > span ? nhi - span : q.lo;
  if (q.s == 0) {
    q.found = 1;
    q.kappa = nhi;
    q.kcount = hcb;
    q.kmass = hmb;
    return true;
  }
  q.hi = nhi;
  q.lo = nlo;
  q.s = q.s > 10 ? q.s - 10 : 0;
  return false;
}

// ---------------------------------------------------------------- id-order walk of a chunk in registers
//
// For the chunk held as Chunk<DT> by the workgroup, kw(i) gives element i's
// kept weight (0 if not kept outright) and whether it is a tie at the
// boundary key.  With ties counting wt each up to jties of them, finds the
// element at which the inclusive id-order total crosses t and returns its id
// (or -1).  Id order is (wave, j, lane, e).
struct KW {
  u64 w;
  bool tie;
};
template <int DT, typename F>
__device__ __forceinline__ int chunk_locate(const Chunk<DT>& ch, F&& kw, u64 wt, u32 jties, u64 t, Lds& L) {
  constexpr int VL = Chunk<DT>::VL, J = Chunk<DT>::J;
  u64 ex_m[J];
  u32 ex_t[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    u64 m = 0;
    u32 tc = 0;
#pragma unroll
    for (int e = 0; e < VL; ++e) {
      const KW x = kw(j * VL + e);
      m += x.w;
      tc += x.tie ? 1u : 0u;
    }
    const u64 im = wave_incl_scan64(m);
    const u32 it = wave_incl_scan(tc);
    ex_m[j] = im - m;
    ex_t[j] = it - tc;
    if (lane_id() == 63) {
      L.cmass[wave_id() * J + j] = im;
      L.cties[wave_id() * J + j] = it;
    }
  }
  if (threadIdx.x == 0) L.s.r[8] = 0xffffffffu;
  lds_sync();
  u64 off_m = 0;
  u32 off_t = 0;
  for (int q = 0; q < wave_id() * J; ++q) {
    off_m += L.cmass[q];
    off_t += L.cties[q];
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    u64 mb = off_m + ex_m[j];
    u32 tb = off_t + ex_t[j];
#pragma unroll
    for (int e = 0; e < VL; ++e) {
      const KW x = kw(j * VL + e);
      const u64 before = mb + (u64)min(tb, jties) * wt;
      mb += x.w;
      tb += x.tie ? 1u : 0u;
      const u64 after = mb + (u64)min(tb, jties) * wt;
      if (before <= t && t < after) L.s.r[8] = (u32)ch.id(j, e);
    }
    off_m += L.cmass[wave_id() * J + j];
    off_t += L.cties[wave_id() * J + j];
  }
  lds_sync();
  const u32 r = L.s.r[8];
  lds_sync();
  return r == 0xffffffffu ? -1 : (int)r;
}

// ---------------------------------------------------------------- exact single-workgroup resolution
//
// Passes over the whole row from global memory, one 16-byte vector per thread
// at a time: q* and the key range; the top-k boundary (count select, one pass
// per round); the mass S of K; the top-p boundary (mass select); the draw and
// the last kept tie.  Serves every row the fast paths leave (top-k above
// kTopkMax, overflows, time-outs, rows without weights).

// Calls f(z, id) for element s of chunk c of this thread, id = c * kCH + s *
// kThreads + t (when below V): one logit per thread and step, so that the
// steps of a chunk run in id order and the exact path stays small.
constexpr int kElemSteps = kCH / kThreads;
template <int DT, typename F>
__device__ __forceinline__ void chunk_elem(const Args& a, const RowP& p, int row, int c, int s, const Lds& L, F&& f) {
  const int id = c * kCH + s * kThreads + (int)threadIdx.x;
  if (id >= a.V) return;
  const size_t rowoff = (size_t)row * (size_t)a.row_stride;
  float z = DT == QS_DTYPE_F32 ? gld((const float*)a.logits + rowoff + id)
                               : bf16_to_f32((u32)gld((const uint16_t*)a.logits + rowoff + id));
  if (p.pen) {
    const int li = id - c * kCH;
    const u32 n = (L.u.pen[li >> 1] >> ((li & 1) * 16)) & 0xffffu;
    if (n) z = apply_penalty(z, n, p.rep, p.rrep, p.pres, p.freq);
  }
  f(z, id);
}

// f(z, id) over the whole row (chunk by chunk, penalty table per chunk).
template <int DT, typename F>
__device__ __forceinline__ void row_pass(const Args& a, const RowP& p, int row, Lds& L, F&& f) {
#pragma unroll 1
  for (int c = 0; c < a.G; ++c) {
    if (p.pen) pen_build(p, c, L);
#pragma unroll 1
    for (int s = 0; s < kElemSteps; ++s) chunk_elem<DT>(a, p, row, c, s, L, f);
    if (p.pen) lds_sync();
  }
}

// The launch's Args read afresh from the kernel-argument segment (the kernel's
// only explicit argument, at offset 0).  Code that is rarely taken reads its
// arguments through this, so that their loads are not merged with those of the
// streaming paths and the merged values do not stay in scalar registers across
// the whole kernel.
__device__ __forceinline__ const Args& kernel_args() {
  return *(const Args*)__builtin_amdgcn_kernarg_segment_ptr();
}

template <int DT>
__device__ __forceinline__ void resolve_single(const Args& a, int row, u32 why, Lds& L) {
  const RowP p = row_params(a, row);
  const int SH = a.SH;
  const u64 thr = ceil_scaled(p.mp, 23 + SH);
  // pass 1: key range of q over non-NaN tokens, and the greedy id for rows without weights
  u32 kmax = 0, kmin = 0xffffffffu;
  u64 gbest = 0;
  row_pass<DT>(a, p, row, L, [&](float z, int id) {
    const u32 k = skey(qdiv(z, p));
    kmax = max(kmax, k);
    if (k) kmin = min(kmin, k);
    const u64 pk = ((u64)gkey(z) << 32) | (0xffffffffu - (u32)id);
    gbest = pk > gbest ? pk : gbest;
  });
  kmax = block_max(kmax, L.s);
  kmin = ~block_max(~kmin, L.s);
  gbest = block_max64(gbest, L.s);
  if (kmax == 0u) {  // every q is NaN: the greedy id
    write_result(a, row, p, (long long)(0xffffffffu - (u32)gbest), 0, thr, kPathSingle, why, 0u, 0u, 0u, 0u);
    return;
  }
  const float qs = f_of_key(kmax);
  auto key_w = [&](float z, u32& k) -> u64 {
    const float q = qdiv(z, p);
    k = skey(q);
    const u64 w = weight_of(q, k, qs, kmax, SH);
    return w >= thr ? w : 0ull;
  };
  // top-k boundary: the k-th largest key (ties kept); 1 when K is every non-NaN token
  u32 kk = 1u;
  if (p.k > 0 && p.k < a.V) {
    Sel q;
    sel_init(q, kmin, kmax, false, (u64)p.k);
    for (;;) {
      sel_clear(L);
      lds_sync();
      row_pass<DT>(a, p, row, L, [&](float z, int) { sel_add(q, L, skey(qdiv(z, p)), 0); });
      lds_sync();
      if (sel_step(q, L)) break;
    }
    if (q.found == 1) kk = q.kappa;
  }
  // S over K and the count of nonzero weights
  u64 S = 0;
  u32 nz = 0;
  row_pass<DT>(a, p, row, L, [&](float z, int) {
    u32 k;
    const u64 w = key_w(z, k);
    if (k >= kk) {
      S += w;
      nz += w ? 1u : 0u;
    }
  });
  S = block_sum64(S, L.s);
  nz = block_sum(nz, L.s);
  // top-p boundary: kept iff key > klo, or key == klo among the first jties ties
  u32 klo = kk, jties = 0xffffffffu, kept = nz;
  u64 W = S, wt = 0;
  if (p.topp) {
    const u64 Tp = mul_frac(S, p.tp);
    Sel q;
    sel_init(q, kk, kmax, true, Tp);
    for (;;) {
      sel_clear(L);
      lds_sync();
      row_pass<DT>(a, p, row, L, [&](float z, int) {
        u32 k;
        const u64 w = key_w(z, k);
        if (w && k >= kk) sel_add(q, L, k, w);
      });
      lds_sync();
      if (sel_step(q, L)) break;
    }
    if (q.found == 1) {
      klo = q.kappa;
      wt = q.kmass / q.kcount;
      const u64 A = q.above_m;
      const u64 jj = (Tp - A) / wt + 1ull;
      jties = (u32)(jj < (u64)q.kcount ? jj : (u64)q.kcount);
      W = A + (u64)jties * wt;
      kept = q.above_c + jties;
    }
  }
  const bool ties_on = jties != 0xffffffffu;
  // the draw, chunk by chunk in id order; the id of the last kept tie
  const u64 t = mul_frac(W, p.u);
  u64 acc = 0;         // kept mass of the chunks before, ties included
  u64 acc_above = 0;   // the same without the ties (they count through ties_before)
  u32 ties_before = 0;
  int pick = -1, idlo = -1;
#pragma unroll 1
  for (int c = 0; c < a.G && (pick < 0 || (ties_on && idlo < 0)); ++c) {
    if (p.pen) pen_build(p, c, L);
    // kept mass and ties of the chunk
    u64 cm = 0;
    u32 ct = 0;
#pragma unroll 1
    for (int m = 0; m < kElemSteps; ++m)
      chunk_elem<DT>(a, p, row, c, m, L, [&](float z, int) {
        u32 k;
        const u64 w = key_w(z, k);
        if (k >= kk && (ties_on ? k > klo : k >= klo)) cm += w;
        if (ties_on && w && k == klo) ++ct;
      });
    cm = block_sum64(cm, L.s);
    ct = block_sum(ct, L.s);
    const u32 jl = ties_on ? (jties > ties_before ? jties - ties_before : 0u) : 0u;
    const u64 kc = cm + (u64)min(ct, jl) * wt;
    const bool has_pick = pick < 0 && t < acc + kc;
    const bool has_tie = ties_on && idlo < 0 && jties > ties_before && jties <= ties_before + ct;
    if (has_pick || has_tie) {
      // id-order walk of the chunk: step m of every thread, then m + 1
      u64 run_m = acc_above;
      u32 run_t = ties_before;
#pragma unroll 1
      for (int m = 0; m < kElemSteps; ++m) {
        u64 vm = 0;
        u32 vt = 0;
        chunk_elem<DT>(a, p, row, c, m, L, [&](float z, int) {
          u32 k;
          const u64 w = key_w(z, k);
          if (k >= kk && (ties_on ? k > klo : k >= klo)) vm += w;
          if (ties_on && w && k == klo) ++vt;
        });
        u32 ttot;
        u64 mtot;
        u32 tex = vt;
        u64 mex = vm;
        block_excl2(tex, mex, L.s, &ttot, &mtot);
        if (threadIdx.x == 0) {
          L.s.r[8] = 0xffffffffu;
          L.s.r[9] = 0xffffffffu;
        }
        lds_sync();
        u64 mb = run_m + mex;
        u32 tb = run_t + tex;
        chunk_elem<DT>(a, p, row, c, m, L, [&](float z, int id) {
          u32 k;
          const u64 w = key_w(z, k);
          const bool above = k >= kk && (ties_on ? k > klo : k >= klo);
          const bool tie = ties_on && w && k == klo;
          const u64 before = mb + (u64)min(tb, ties_on ? jties : 0u) * wt;
          mb += above ? w : 0ull;
          tb += tie ? 1u : 0u;
          const u64 after = mb + (u64)min(tb, ties_on ? jties : 0u) * wt;
          if (before <= t && t < after) L.s.r[8] = (u32)id;
          if (tie && tb == jties) L.s.r[9] = (u32)id;
        });
        lds_sync();
        if (pick < 0 && L.s.r[8] != 0xffffffffu) pick = (int)L.s.r[8];
        if (ties_on && idlo < 0 && L.s.r[9] != 0xffffffffu) idlo = (int)L.s.r[9];
        lds_sync();
        run_m += mtot;
        run_t += ttot;
      }
    }
    if (p.pen) lds_sync();
    acc += kc;
    acc_above += cm;
    ties_before += ct;
  }
  const u32 idlo_u = ties_on ? (u32)idlo : (u32)a.V;
  write_result(a, row, p, pick, W, thr, kPathSingle, why, kmax, klo, idlo_u, kept);
}

// ---------------------------------------------------------------- finishers

// Greedy: the largest (gkey, -id) over the chunks' slots.
__device__ __forceinline__ void finish_greedy(const Args& a, const RowP& p, int row, Lds& L) {
  const Slot* sl = row_slots(a, row);
  u64 best = 0;
  for (int c = threadIdx.x; c < a.G; c += kThreads) {
    const u64 v = ldc(&sl[c].a);
    best = v > best ? v : best;
  }
  best = block_max64(best, L.s);
  const u32 id = 0xffffffffu - (u32)best;
  write_result(a, row, p, (long long)id, 0, 0, kPathGreedy, 0u, 0u, 0u, id, 1u);
}

// ---------------------------------------------------------------- gathering candidates
//
// Entries of per-chunk lists (chunk c: cnt_of(c, mx) entries at base + c*stride,
// in id order) go to L.u.fin.ent in chunk order, so the result is in id order.
// The first P entries of every list (P a power of two) are loaded together with
// the counts (one round trip); longer lists load the rest afterwards.
// cnt_of(c, mx) returns 0xffffffff for a list that overflowed, and may set three
// values mx[] whose workgroup maxima are returned in mx (threads past the lists
// hold zeros).  Returns the total, or 0xffffffff when a list overflowed or the
// total exceeds kFCap.  Needs G <= kThreads.
struct NoXf {
  __device__ __forceinline__ u64 operator()(u64 e) const { return e; }
};
template <typename CF, typename XF = NoXf>
__device__ __forceinline__ u32 gather_lds(const Args& a, const u64* base, int stride, CF&& cnt_of, Lds& L,
                                          u32 (&mx)[3], XF xf = XF()) {
  constexpr int M = kFCap / kThreads;
  const int G = a.G;
  const int lp = 31 - __clz(min(stride, kFCap / G));
  const int P = 1 << lp;
  mx[0] = mx[1] = mx[2] = 0u;
  const u32 raw = (int)threadIdx.x < G ? cnt_of((int)threadIdx.x, mx) : 0u;
  u64 spec[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int f = (int)threadIdx.x + m * kThreads;
    const int c = f >> lp, i = f & (P - 1);
    spec[m] = c < G ? ldc(base + (size_t)c * stride + i) : 0ull;
  }
  const u32 nc = raw == 0xffffffffu ? (u32)kFCap + 1u : min(raw, (u32)kFCap + 1u);
  // offsets (bit 24 counts the lists longer than P; the counts sum to less than
  // 2^24) and the maxima, with one pair of barriers
  const u32 v = nc | (nc > (u32)P ? 1u << 24 : 0u);
  const u32 inc = wave_incl_scan(v);
  const u32 m0 = wave_max(mx[0]), m1 = wave_max(mx[1]), m2 = wave_max(mx[2]);
  if (lane_id() == 63) {
    L.s.v[wave_id()][2] = inc;
    L.s.v[wave_id()][5] = m0;
    L.s.v[wave_id()][6] = m1;
    L.s.v[wave_id()][7] = m2;
  }
  lds_sync();
  u32 base_w = 0, total = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const u32 x = L.s.v[i][2];
    base_w += i < wave_id() ? x : 0u;
    total += x;
    mx[0] = max(mx[0], L.s.v[i][5]);
    mx[1] = max(mx[1], L.s.v[i][6]);
    mx[2] = max(mx[2], L.s.v[i][7]);
  }
  const u32 off = (base_w + inc - v) & 0xffffffu;
  const bool any_long = (total >> 24) != 0u;
  total &= 0xffffffu;
  if ((int)threadIdx.x < G) {
    L.coff[threadIdx.x] = off;
    L.cties[threadIdx.x] = nc;
  }
  lds_sync();
  if (total > (u32)kFCap) return 0xffffffffu;
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int f = (int)threadIdx.x + m * kThreads;
    const int c = f >> lp, i = f & (P - 1);
    if (c < G && (u32)i < L.cties[c]) L.u.fin.ent[L.coff[c] + i] = xf(spec[m]);
  }
  if (any_long) {
    for (int c = 0; c < G; ++c) {  // lists longer than P
      const u32 n_c = L.cties[c];
      for (u32 i = (u32)P + threadIdx.x; i < n_c; i += kThreads)
        L.u.fin.ent[L.coff[c] + i] = xf(ldc(base + (size_t)c * stride + i));
    }
  }
  lds_sync();
  return total;
}

// ---------------------------------------------------------------- selection over the gathered entries

// The gathered entries spread over the workgroup: thread t holds entries
// [t*per, t*per + per) of L.u.fin.ent, per = ceil(n / kThreads) (<= kFPer),
// so the thread order is the id order.  Missing entries are 0 (key 0).
struct Held {
  u64 e[kFPer];
  u32 per;  // uniform
};
template <typename LT>
__device__ __forceinline__ void hold_entries(const LT& L, u32 n, Held& h) {
  h.per = uni((n + kThreads - 1) / kThreads);
  const u32 i0 = threadIdx.x * h.per;
#pragma unroll
  for (int i = 0; i < kFPer; ++i) {
    h.e[i] = 0ull;
    if ((u32)i < h.per) h.e[i] = i0 + i < n ? L.u.fin.ent[i0 + i] : 0ull;
  }
}

// floor(x / d) for a quotient below 2^20 (a float estimate, corrected).
__device__ __forceinline__ u64 div_small(u64 x, u64 d) {
  u64 q = (u64)fmaxf(0.0f, __builtin_floorf((float)x / (float)d));
#pragma unroll
  for (int i = 0; i < 2; ++i) q = q * d > x ? q - 1 : q;
#pragma unroll
  for (int i = 0; i < 2; ++i) q = (q + 1) * d <= x ? q + 1 : q;
  return q;
}

// Among the held entries whose key lies in [lo, hi] (by mass: whose packed
// weight wq is nonzero) finds the key kappa at which the running total in
// key-descending order crosses target:
//   by count: count(key > kappa) < target <= count(key >= kappa)
//   by mass:  mass(key > kappa) <= target < mass(key >= kappa).
// Each round histograms the range into 256 bins of 2^s keys (one wave scans
// them) and narrows to the crossing bin; a bin of at most kDirect entries is
// resolved by ranking its entries directly; a bin of one key ends it.
struct SelRes {
  u32 kappa, cnt_above, cnt_at;
  u64 mass_above, mass_at;
  bool ok;
  u32 total_cnt;   // the first round's totals over the range
  u64 total_mass;
  int clean;       // the histogram buffer (0 or 1) left cleared
};
// With frac >= 0 (by mass) the target is floor(frac * total), the total being
// the range's mass, found in the first round; the totals are returned.  The
// histogram has two buffers: a round clears the next one's.  Without TAIL
// the select returns with no closing barrier: the caller must not write the
// scratch fields the result is read from (r[4..10], r64[4..7]) before its next
// barrier.  With clean0 >= 0 the histogram buffer clean0 is known to be cleared
// (a previous select's result) and the select starts on it without clearing.
template <bool BY_MASS, bool TAIL = true, typename LT>
__device__ __forceinline__ SelRes held_select(const Args& a, LT& L, const Held& h, const u32 (&wq)[kFPer], u32 lo,
                                              u32 hi, u64 target, float frac = -1.0f, int clean0 = -1) {
  (void)a;
  SelRes r;
  r.kappa = r.cnt_above = r.cnt_at = 0u;
  r.mass_above = r.mass_at = 0ull;
  r.ok = false;
  r.total_cnt = 0u;
  r.total_mass = 0ull;
  const int p0 = clean0 >= 0 ? clean0 : 0;
  if (clean0 < 0) {
    for (int b = threadIdx.x; b < kNB; b += kThreads) {
      L.sel.hc[b] = 0u;
      L.sel.hm[b] = 0ull;
    }
    lds_sync();
  }
  r.clean = p0;
  for (int round = 0; round < 6; ++round) {
    const int bl = bitlen(hi - lo);
    const int sh = bl > 8 ? bl - 8 : 0;
    const int cur = ((round + p0) & 1) * kNB, nxt = kNB - cur;
    r.clean = ((round + p0) & 1) ^ 1;  // nxt, cleared below
    if (round < 4) QS_TRA(15 + 3 * round);
#pragma unroll
    for (int i = 0; i < kFPer; ++i) {
      if ((u32)i < h.per) {
        const u32 key = (u32)(h.e[i] >> 32);
        if (key >= lo && key <= hi && (!BY_MASS || wq[i] != 0u)) {
          const u32 b = (hi - key) >> sh;
          atomicAdd(&L.sel.hc[cur + b], 1u);
          if (BY_MASS) atomicAdd(&L.sel.hm[cur + b], wunpack(wq[i]));
        }
      }
    }
    for (int b = threadIdx.x; b < kNB; b += kThreads) {
      L.sel.hc[nxt + b] = 0u;
      L.sel.hm[nxt + b] = 0ull;
    }
    lds_sync();
    if (round < 4) QS_TRA(16 + 3 * round);
    if (threadIdx.x < 64) {
      const int l = (int)lane_id();
      u32 c4[4], cs = 0;
      u64 m4[4], ms = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c4[j] = L.sel.hc[cur + 4 * l + j];
        m4[j] = BY_MASS ? L.sel.hm[cur + 4 * l + j] : 0ull;
        cs += c4[j];
        ms += m4[j];
      }
      const u32 ci = wave_incl_scan(cs);
      const u64 mi = BY_MASS ? wave_incl_scan64(ms) : 0ull;
      u32 cb = ci - cs;
      u64 mb = mi - ms;
      if (round == 0 && frac >= 0.0f) {
        const u64 tm = readlane64(mi, 63);
        target = mul_frac(tm, frac);
        if (l == 0) {
          L.s.r64[10] = tm;
          L.s.r[13] = readlane(ci, 63);
        }
      }
      if (l == 0) {
        L.s.r[4] = 0xffffffffu;
        L.s.r[7] = 0u;  // for a direct resolution
        L.s.r[8] = 0xffffffffu;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool hit = BY_MASS ? (mb <= target && target < mb + m4[j]) : (cb < target && target <= cb + c4[j]);
        if (hit) {
          L.s.r[4] = (u32)(4 * l + j);
          L.s.r[5] = cb;
          L.s.r[6] = c4[j];
          L.s.r64[4] = mb;
          L.s.r64[5] = m4[j];
        }
        cb += c4[j];
        mb += m4[j];
      }
    }
    lds_sync();
    if (round < 4) QS_TRA(17 + 3 * round);
    if (round == 0 && frac >= 0.0f) {
      r.total_mass = uni64(L.s.r64[10]);
      r.total_cnt = uni(L.s.r[13]);
      target = mul_frac(r.total_mass, frac);
    }
    const u32 b = uni(L.s.r[4]);
    const u32 cb = uni(L.s.r[5]), cnt_b = uni(L.s.r[6]);
    const u64 mb = uni64(L.s.r64[4]), mass_b = uni64(L.s.r64[5]);
    if (b == 0xffffffffu) {  // the target lies beyond the range's total
      lds_sync();
      return r;
    }
    r.cnt_above += cb;
    r.mass_above += mb;
    target -= BY_MASS ? mb : (u64)cb;
    const u32 nhi = hi - (b << sh);
    const u32 span = (1u << sh) - 1u;
    const u32 nlo = (nhi - lo) > span ? nhi - span : lo;
    if (sh == 0) {
      r.kappa = nhi;
      r.cnt_at = cnt_b;
      r.mass_at = mass_b;
      r.ok = true;
      if (TAIL) lds_sync();
      return r;
    }
    hi = nhi;
    lo = nlo;
    if (cnt_b <= (u32)kDirect) {
      // the bin's entries, ranked directly: entry x by the 8 threads 8x..8x+7
#pragma unroll
      for (int i = 0; i < kFPer; ++i) {
        if ((u32)i < h.per) {
          const u32 key = (u32)(h.e[i] >> 32);
          if (key >= lo && key <= hi && (!BY_MASS || wq[i] != 0u)) {
            const u32 slot = atomicAdd(&L.s.r[7], 1u);
            L.u.fin.lk[slot] = key;
            L.u.fin.lw[slot] = BY_MASS ? wunpack(wq[i]) : 0ull;
          }
        }
      }
      lds_sync();
      if (round < 4) QS_TRA(27);
      const u32 m = uni(L.s.r[7]);
      const u32 xi = threadIdx.x >> 3, part = threadIdx.x & 7u;
      const u32 x = xi < m ? L.u.fin.lk[xi] : 0u;
      u32 gc = 0, ec = 0;
      u64 gm = 0, em = 0;
      for (u32 j = part; j < m; j += 8) {
        const u32 y = L.u.fin.lk[j];
        const u64 wy = BY_MASS ? L.u.fin.lw[j] : 0ull;
        gc += y > x ? 1u : 0u;
        ec += y == x ? 1u : 0u;
        gm += y > x ? wy : 0ull;
        em += y == x ? wy : 0ull;
      }
#pragma unroll
      for (int sh8 = 1; sh8 < 8; sh8 <<= 1) {
        gc += __shfl_xor(gc, sh8);
        ec += __shfl_xor(ec, sh8);
        if (BY_MASS) {
          gm += (u64)__shfl_xor((unsigned long long)gm, sh8);
          em += (u64)__shfl_xor((unsigned long long)em, sh8);
        }
      }
      if (xi < m && part == 0u) {
        const bool hit = BY_MASS ? (gm <= target && target < gm + em) : (gc < target && target <= gc + ec);
        if (hit) {
          L.s.r[8] = x;
          L.s.r[9] = gc;
          L.s.r[10] = ec;
          L.s.r64[6] = gm;
          L.s.r64[7] = em;
        }
      }
      lds_sync();
      if (round < 4) QS_TRA(28);
      const u32 kx = uni(L.s.r[8]);
      r.kappa = kx;
      r.cnt_above += uni(L.s.r[9]);
      r.cnt_at = uni(L.s.r[10]);
      r.mass_above += uni64(L.s.r64[6]);
      r.mass_at = uni64(L.s.r64[7]);
      r.ok = kx != 0xffffffffu;
      if (TAIL) lds_sync();
      return r;
    }
  }
  return r;
}

// Maxima of two values and the sum of a third over the workgroup, with one
// pair of barriers.
__device__ __forceinline__ void block_max2_sum(u32& x, u32& y, u32& z, Scratch& s) {
  x = wave_max(x);
  y = wave_max(y);
  z = wave_sum(z);
  if (lane_id() == 0) {
    s.v[wave_id()][5] = x;
    s.v[wave_id()][6] = y;
    s.v[wave_id()][7] = z;
  }
  lds_sync();
  x = y = z = 0u;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    x = max(x, s.v[i][5]);
    y = max(y, s.v[i][6]);
    z += s.v[i][7];
  }
  lds_sync();
}
// Maxima of two values over the workgroup with one pair of barriers.
__device__ __forceinline__ void block_max2(u32& x, u32& y, Scratch& s) {
  x = wave_max(x);
  y = wave_max(y);
  if (lane_id() == 0) {
    s.v[wave_id()][5] = x;
    s.v[wave_id()][6] = y;
  }
  lds_sync();
  x = y = 0u;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    x = max(x, s.v[i][5]);
    y = max(y, s.v[i][6]);
  }
  lds_sync();
}
// Sums of a u64 and a u32 over the workgroup with one pair of barriers.
__device__ __forceinline__ void block_sum2(u64& m, u32& c, Scratch& s) {
  u32 ct;
  u64 mt;
  block_excl2(c, m, s, &ct, &mt);
  c = ct;
  m = mt;
}

// Finish a top-k row whose K (the nk <= 64 held tokens with key >= kk) fits one
// wave: K is compacted in id order, one wave ranks it in (key desc, id asc)
// order and moves it there (lane permutes), the top-p rule is applied token by
// token on the exclusive prefix masses (the same set as by kappa_p and its
// ties), and the draw is a prefix over K back in id order.  No barrier after
// the compaction.
template <typename WPK>
__device__ __forceinline__ bool finish_small_k(const Args& a, const RowP& p, int row, Lds& L, const Held& h, u32 kk,
                                               u32 nk, u32 kmax, u64 thr, WPK&& wpk) {
  nk = uni(nk);
  u32 cnt = 0;
#pragma unroll
  for (int i = 0; i < kFPer; ++i)
    if ((u32)i < h.per && (u32)(h.e[i] >> 32) >= kk) ++cnt;
  u32 tot;
  u32 pos = block_excl(cnt, L.s, &tot);
  u64* kl = L.sel.hm;  // free once the selects are done
#pragma unroll
  for (int i = 0; i < kFPer; ++i)
    if ((u32)i < h.per && (u32)(h.e[i] >> 32) >= kk) kl[pos++] = h.e[i];
  lds_sync();
  if (tot != nk) return false;  // K is not what the select counted: cannot happen
  if (threadIdx.x < 64) {
    const u32 l = lane_id();
    const bool have = l < nk;
    const u64 e = have ? kl[l] : 0ull;
    const u32 key = (u32)(e >> 32), id = (u32)e;
    const u32 x = have ? wpk(key) : 0u;
    const u64 w = wunpack(x);
    // rank in (key desc, id asc); lanes without a token take the ranks past nk
    u32 rank = have ? 0u : l;
    for (u32 j = 0; j < nk; ++j) {
      const u32 kj = readlane(key, (int)j), ij = readlane(id, (int)j);
      rank += (have && (kj > key || (kj == key && ij < id))) ? 1u : 0u;
    }
    // lane r gets the token of rank r
    auto push = [&](u32 v) { return (u32)__builtin_amdgcn_ds_permute((int)(rank << 2), (int)v); };
    const u32 rkey = push(key), rid = push(id), rlo = push((u32)w), rhi = push((u32)(w >> 32));
    const u64 rw = ((u64)rhi << 32) | rlo;
    const u64 rin = wave_incl_scan64(rw);
    const u64 S = readlane64(rin, 63);
    u64 W = S;
    u32 klo = kk, idlo = (u32)a.V;
    bool rkept = l < nk;
    if (p.topp) {
      const u64 Tp = mul_frac(S, p.tp);
      rkept = l < nk && rin - rw <= Tp;  // exclusive prefix within floor(top_p * S)
      const u64 kb = __ballot(rkept);
      const int last = 63 - __clzll((long long)kb);  // kept tokens are a prefix of the ranks
      klo = readlane(rkey, last);
      idlo = readlane(rid, last);
      W = readlane64(rin, last);
    }
    const u32 kept = popc64(__ballot(rkept && rw != 0ull));
    // back to id order: lane l reads its token's rank's verdict
    const bool kp = __builtin_amdgcn_ds_bpermute((int)(rank << 2), rkept ? 1 : 0) != 0 && have;
    const u64 kw = kp ? w : 0ull;
    const u64 inc = wave_incl_scan64(kw);
    const u64 t = mul_frac(W, p.u);
    const u64 pb = __ballot(kw != 0ull && inc - kw <= t && t < inc);
    const int src = pb ? __ffsll((long long)pb) - 1 : -1;
    const long long pick = src >= 0 ? (long long)readlane(id, src) : -1ll;
    if (l == 0) {
      L.s.r[11] = pick >= 0 ? 1u : 0u;
      if (pick >= 0) write_result(a, row, p, pick, W, thr, kPathTopK, 0u, kmax, klo, idlo, kept);
    }
  }
  lds_sync();
  const bool ok = L.s.r[11] != 0u;
  lds_sync();
  return ok;
}

// ---------------------------------------------------------------- wave sorting networks

// The value of lane l ^ J, by DPP moves within rows of 16 lanes and the
// permlane swaps across them (no LDS traffic).
template <int J>
__device__ __forceinline__ u32 xlane(u32 v) {
  const u32 l = lane_id();
  if constexpr (J == 1) {
    return (u32)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xf, 0xf, true);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (J == 2) {
    return (u32)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xf, 0xf, true);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (J == 4) {
    const u32 up = (u32)__builtin_amdgcn_mov_dpp((int)v, 0x104, 0xf, 0xf, true);  // row_shl 4: lane l + 4
    const u32 dn = (u32)__builtin_amdgcn_mov_dpp((int)v, 0x114, 0xf, 0xf, true);  // row_shr 4: lane l - 4
    return (l & 4u) ? dn : up;
  } else if constexpr (J == 8) {
    return (u32)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, true);  // row_ror 8
  } else if constexpr (J == 16) {
    const auto s = __builtin_amdgcn_permlane16_swap(v, v, false, false);  // rows (0,0,2,2) and (1,1,3,3)
    return (l & 16u) ? (u32)s[0] : (u32)s[1];
  } else {
    static_assert(J == 32, "lane distances 1 .. 32");
    const auto s = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // halves (lo, lo) and (hi, hi)
    return (l & 32u) ? (u32)s[0] : (u32)s[1];
  }
}
// Compare-exchange with lane l ^ J: the lane keeps the larger of the pair iff
// (it is the lower lane) == desc.
template <int J>
__device__ __forceinline__ u64 cmpx(u64 v, bool desc) {
  const u64 o = ((u64)xlane<J>((u32)(v >> 32)) << 32) | xlane<J>((u32)v);
  const bool big = ((lane_id() & (u32)J) == 0u) == desc;
  return big ? (o > v ? o : v) : (o < v ? o : v);
}
// One value per lane, sorted over the wave (bitonic network): descending or ascending.
template <bool DESC>
__device__ __forceinline__ u64 wave_sort(u64 v) {
  const u32 l = lane_id();
  auto d = [&](u32 k) { return ((l & k) == 0u) == DESC; };  // the block of size k runs descending
  v = cmpx<1>(v, d(2));
  v = cmpx<2>(v, d(4));
  v = cmpx<1>(v, d(4));
  v = cmpx<4>(v, d(8));
  v = cmpx<2>(v, d(8));
  v = cmpx<1>(v, d(8));
  v = cmpx<8>(v, d(16));
  v = cmpx<4>(v, d(16));
  v = cmpx<2>(v, d(16));
  v = cmpx<1>(v, d(16));
  v = cmpx<16>(v, d(32));
  v = cmpx<8>(v, d(32));
  v = cmpx<4>(v, d(32));
  v = cmpx<2>(v, d(32));
  v = cmpx<1>(v, d(32));
  v = cmpx<32>(v, DESC);
  v = cmpx<16>(v, DESC);
  v = cmpx<8>(v, DESC);
  v = cmpx<4>(v, DESC);
  v = cmpx<2>(v, DESC);
  v = cmpx<1>(v, DESC);
  return v;
}
// A bitonic sequence over the wave, sorted descending.
__device__ __forceinline__ u64 wave_merge_desc(u64 v) {
  v = cmpx<32>(v, true);
  v = cmpx<16>(v, true);
  v = cmpx<8>(v, true);
  v = cmpx<4>(v, true);
  v = cmpx<2>(v, true);
  v = cmpx<1>(v, true);
  return v;
}

// Finish a top-k row with k < 64 from at most kThreads gathered candidates
// (L.u.fin.ent[0, n), id order): every wave sorts 64 of them by (key desc, id
// asc), a tree of wave merges (each keeps the 64 largest of two sorted lists)
// leaves the row's 64 largest in wave 0, which applies top-k (ties kept), min_p
// and top-p to them and draws in id order.  The same sets and draw as
// finish_small_k.  Returns 1 when done, 0 when the row must go to the exact
// path, -1 when ties at kappa_k may reach past the 64 kept (the general
// finisher takes the row).
template <typename WPK>
__device__ __forceinline__ int finish_sorted(const Args& a, const RowP& p, int row, Lds& L, u32 n, u32 kmax,
                                             u32 below_max, u64 thr, WPK&& wpk) {
  const u32 t = threadIdx.x, w = wave_id(), l = lane_id();
  const u64 e = t < n ? L.u.fin.ent[t] : 0ull;
  u64 v = e ? (e & 0xffffffff00000000ull) | (u64)(~(u32)e) : 0ull;  // (key, ~id); 0 for no token
  v = wave_sort<true>(v);
  const u32 nw = uni((n + 63u) / 64u);  // waves holding candidates
  for (u32 step = 1, lev = 0; step < nw; step <<= 1, ++lev) {
    u64* buf = L.sel.hm + (lev & 1u) * kThreads;  // two buffers: one barrier per level
    buf[t] = v;
    lds_sync();
    if ((w & (2u * step - 1u)) == 0u && w + step < nw) {
      const u64 b = buf[(w + step) * 64u + 63u - l];  // the partner's list, reversed
      v = wave_merge_desc(b > v ? b : v);
    }
  }
  if (w == 0u) {
    const u32 key = (u32)(v >> 32), id = ~(u32)v;
    const bool have = v != 0ull;
    int res = 1;
    u32 kk = 1u;  // fewer candidates than k: every one of them (if none was left out)
    if (n < (u32)p.k) {
      if (below_max != 0u) res = 0;
    } else {
      kk = readlane(key, p.k - 1);
      // completeness: every token left out has a key of q below kappa_k
      if (below_max != 0u && skey(qdiv(f_of_key(below_max), p)) >= kk) res = 0;
      if (n > 64u && readlane(key, 63) == kk) res = -1;  // ties at kappa_k may go on past the 64
    }
    if (res == 1) {
      const bool inK = have && key >= kk;
      const u64 wv = inK ? wunpack(wpk(key)) : 0ull;
      const u64 rin = wave_incl_scan64(wv);
      const u64 S = readlane64(rin, 63);
      u64 W = S;
      u32 klo = kk, idlo = (u32)a.V;
      bool kept = inK;
      if (p.topp) {
        const u64 Tp = mul_frac(S, p.tp);
        kept = inK && rin - wv <= Tp;  // exclusive prefix within floor(top_p * S): a prefix of the order
        const u64 kb = __ballot(kept);
        const int last = 63 - __clzll((long long)kb);
        klo = readlane(key, last);
        idlo = readlane(id, last);
        W = readlane64(rin, last);
      }
      const u32 nkept = popc64(__ballot(kept && wv != 0ull));
      // the draw: the kept tokens in id order (lane of origin as payload)
      const u64 sv = wave_sort<false>(kept ? ((u64)id << 32) | l : ~0ull);
      const int src = (int)(u32)sv;
      const u32 wlo = (u32)__shfl((int)(u32)wv, src & 63), whi = (u32)__shfl((int)(u32)(wv >> 32), src & 63);
      const u64 wk = sv != ~0ull ? ((u64)whi << 32) | wlo : 0ull;
      const u64 inc = wave_incl_scan64(wk);
      const u64 tt = mul_frac(W, p.u);
      const u64 pb = __ballot(wk != 0ull && inc - wk <= tt && tt < inc);
      const long long pick = pb ? (long long)readlane((u32)(sv >> 32), __ffsll((long long)pb) - 1) : -1ll;
      if (pick < 0) res = 0;
      if (l == 0u && pick >= 0) write_result(a, row, p, pick, W, thr, kPathTopK, 0u, kmax, klo, idlo, nkept);
    }
    if (l == 0u) L.s.r[11] = (u32)res;
  }
  lds_sync();
  const int res = (int)L.s.r[11];
  lds_sync();
  return res;
}

// Finish a top-k row from its gathered candidates (L.u.fin.ent[0, n), id
// order): kappa_k (count select), weights and min_p, S, kappa_p (mass select),
// the draw by an id-order scan.  kmax is the row's largest key of q, klow a
// lower bound of the candidates' keys, below_max the largest z key left out by
// any chunk.  Returns false when the row must go to the exact path.
__device__ __forceinline__ bool finish_topk(const Args& a, const RowP& p, int row, Lds& L, u32 n, u32 kmax, u32 klow,
                                            u32 below_max, int c) {
  (void)c;
  const int SH = a.SH;
  const u64 thr = ceil_scaled(p.mp, 23 + SH);
  if (n == 0 || kmax == 0u) return false;
  const float qs = f_of_key(kmax);
  auto wpk = [&](u32 key) -> u32 {
    const u32 x = wpack_of(f_of_key(key), key, qs, kmax, SH);
    return wunpack(x) >= thr ? x : 0u;
  };
  auto wf = [&](u32 key) -> u64 { return wunpack(wpk(key)); };
  if (n <= (u32)kThreads && (u32)p.k < 64u) {
    const int r = finish_sorted(a, p, row, L, n, kmax, below_max, thr, wpk);
    if (r >= 0) return r != 0;
  }
  Held h;
  hold_entries(L, n, h);
  u32 wq[kFPer];
#pragma unroll
  for (int i = 0; i < kFPer; ++i) wq[i] = 0u;
  QS_TR(9);
  // kappa_k
  u32 kk, nk;  // nk: the size of K (tokens with key >= kk)
  int clean = -1;  // a select histogram buffer known to be cleared
  if (n < (u32)p.k) {
    if (below_max != 0u) return false;  // tokens left out could belong to K
    kk = 1u;
    nk = n;
  } else {
    // no closing barrier: what follows writes none of the scratch fields the
    // select's result is read from before its own first barrier
    const SelRes q = held_select<false, false>(a, L, h, wq, max(klow, 1u), kmax, (u64)p.k);
    clean = q.clean;
    kk = q.kappa;
    nk = q.cnt_above + q.cnt_at;
    // completeness: every token left out has a key of q below kappa_k
    if (!q.ok || (below_max != 0u && skey(qdiv(f_of_key(below_max), p)) >= kk)) {
      lds_sync();  // the exact path reuses the scratch fields just read
      return false;
    }
  }
  QS_TR(10);
  if (nk <= 64u) return finish_small_k(a, p, row, L, h, kk, nk, kmax, thr, wpk);
  // weights of K (packed); S and the count of nonzero weights (with top-p, as the
  // totals of the boundary's select)
  u64 S = 0;
  u32 nz = 0;
#pragma unroll
  for (int i = 0; i < kFPer; ++i) {
    if ((u32)i < h.per) {
      const u32 key = (u32)(h.e[i] >> 32);
      wq[i] = key >= kk ? wpk(key) : 0u;
      S += wunpack(wq[i]);
      nz += wq[i] ? 1u : 0u;
    }
  }
  if (!p.topp) block_sum2(S, nz, L.s);
  u32 klo = kk, jties = 0xffffffffu, kept = nz;
  u64 W = S, wt = 0;
  QS_TR(11);
  if (p.topp) {
    const SelRes q = held_select<true, false>(a, L, h, wq, kk, kmax, 0ull, p.tp, clean);
    S = q.total_mass;
    const u64 Tp = mul_frac(S, p.tp);
    if (!q.ok) {
      lds_sync();  // the exact path reuses the scratch fields just read
      return false;
    }
    klo = q.kappa;
    wt = wf(klo);  // every token at kappa_p has this weight
    const u64 jj = div_small(Tp - q.mass_above, wt) + 1ull;
    jties = (u32)(jj < (u64)q.cnt_at ? jj : (u64)q.cnt_at);
    W = q.mass_above + (u64)jties * wt;
    kept = q.cnt_above + jties;
  }
  QS_TR(12);
  // the draw: kept mass in id order, ties at klo counting wt each up to jties of them
  const bool ties_on = jties != 0xffffffffu;
  const u32 jt = ties_on ? jties : 0u;
  const u64 t = mul_frac(W, p.u);
  u64 m = 0;
  u32 tc = 0;
#pragma unroll
  for (int i = 0; i < kFPer; ++i) {
    if ((u32)i < h.per) {
      const u32 key = (u32)(h.e[i] >> 32);
      m += (ties_on ? key > klo : key >= klo) ? wunpack(wq[i]) : 0ull;
      tc += (ties_on && wq[i] && key == klo) ? 1u : 0u;
    }
  }
  u32 ttot;
  u64 mtot;
  if (threadIdx.x == 0) {  // ordered before the stores below by block_excl2's barriers
    L.s.r[11] = 0xffffffffu;
    L.s.r[12] = 0xffffffffu;
  }
  block_excl2(tc, m, L.s, &ttot, &mtot);
#pragma unroll
  for (int i = 0; i < kFPer; ++i) {
    if ((u32)i < h.per) {
      const u32 key = (u32)(h.e[i] >> 32);
      const bool tie = ties_on && wq[i] && key == klo;
      const u64 before = m + (u64)min(tc, jt) * wt;
      m += (ties_on ? key > klo : key >= klo) ? wunpack(wq[i]) : 0ull;
      tc += tie ? 1u : 0u;
      const u64 after = m + (u64)min(tc, jt) * wt;
      if (before <= t && t < after) L.s.r[11] = (u32)h.e[i];
      if (tie && tc == jties) L.s.r[12] = (u32)h.e[i];
    }
  }
  lds_sync();
  QS_TR(13);
  const u32 pick = L.s.r[11];
  const u32 idlo = ties_on ? L.s.r[12] : (u32)a.V;
  if (pick == 0xffffffffu) return false;
  write_result(a, row, p, (long long)pick, W, thr, kPathTopK, 0u, kmax, klo, idlo, kept);
  return true;
}

// Bins of the mass histogram over x = -d = q* - q past an offset x0: bins
// [0, n1) linear with n1 / x1 bins per unit up to x0 + x1, bins [n1, kNB) linear
// with s2 bins per unit past it; bin 0 holds the largest keys, everything past
// the range falls in the last bin.  Monotone in the key.
struct MassBins {
  float x0, x1, s1, s2;
  int n1;
  float c2;  // n1 - x1 * s2: the second segment is c2 + x * s2
};
static_assert(kNB <= 256, "a bin index fits a byte");
constexpr float kXMax = 44.5f;  // y = -x * log2(e) < -64 past it: weight 0
constexpr float kXFine = 12.0f; // first round: the finer segment, [0, kXFine)
__device__ __forceinline__ MassBins mass_bins_first(float D) {
  MassBins m;
  m.x0 = 0.0f;
  D = fminf(fmaxf(D, 0.0f), kXMax);
  if (D > 16.0f) {
    m.n1 = 3 * kNB / 4;
    m.x1 = kXFine;
    m.s1 = (float)m.n1 / kXFine;
    m.s2 = (float)(kNB - m.n1) / (D - kXFine);
  } else {
    m.n1 = kNB;
    m.x1 = D > 0x1p-60f ? D : 0.0f;
    m.s1 = D > 0x1p-60f ? (float)kNB / D : 0.0f;  // no spread: every token in bin 0
    m.s2 = 0.0f;
  }
  m.c2 = (float)m.n1 - m.x1 * m.s2;
  return m;
}
// The two segments make a concave map (s1 >= s2: 16 bins per unit, then at most
// 64 / 4), so the bin position is the smaller of the two lines.
__device__ __forceinline__ u32 mass_bin_d(float d, const MassBins& m) {
  const float x = -d - m.x0;
  const float f = fminf(x * m.s1, __builtin_fmaf(x, m.s2, m.c2));
  return min((u32)kNB - 1u, (u32)fmaxf(0.0f, f));
}
__device__ __forceinline__ u32 mass_bin(float q, u32 k, float qs, u32 ks, const MassBins& m) {
  return mass_bin_d((k == ks) ? 0.0f : q - qs, m);
}
// mass_bin_d for the first round's bins (x0 = 0), the same bin: x = -d, and the
// clamp to [0, kNB - 1] before the conversion (a dead token's NaN is not binned).
__device__ __forceinline__ u32 mass_bin_first(float d, const MassBins& m) {
  const float f = fminf(d * -m.s1, __builtin_fmaf(d, -m.s2, m.c2));
  return (u32)__builtin_amdgcn_fmed3f(f, 0.0f, (float)(kNB - 1));
}
// x at the far edge of bin b
__device__ __forceinline__ float bin_edge(const MassBins& m, u32 b) {
  const float e = (float)(b + 1);
  if ((int)b < m.n1) return m.x0 + (m.s1 > 0.0f ? e / m.s1 : 0.0f);
  return m.x0 + m.x1 + (m.s2 > 0.0f ? (e - (float)m.n1) / m.s2 : 3.0e38f);
}
// A lower bound of the nonzero weights in bin b: 2^(23 + SH) * 2^(-edge * log2 e)
// with room for the rounding of the bin computation, and never below 1 (every
// nonzero weight is at least 1).  A token with nonzero weight has x < kXMax, so
// the last bin of every range is bounded too.
__device__ __forceinline__ float bin_least_weight(const MassBins& m, u32 b, int SH) {
  const float xe = fminf(bin_edge(m, b) * 1.001f + 1e-6f, kXMax);
  return fmaxf(1.0f, 0.9f * exp2f((float)(23 + SH) - xe * kL2E));
}
// The bins of the next round: bin b of this one split into kNB.
__device__ __forceinline__ MassBins mass_bins_split(const MassBins& m, u32 b) {
  const float lo = b == 0u ? m.x0 : bin_edge(m, b - 1u);
  const float hi = bin_edge(m, b);
  MassBins n;
  n.x0 = lo;
  n.n1 = kNB;
  const float w = fminf(hi, kXMax) - lo;
  n.x1 = w > 0.0f ? w : 0.0f;
  n.s1 = w > 0x1p-60f ? (float)kNB / w : 0.0f;
  n.s2 = 0.0f;
  n.c2 = (float)kNB;
  return n;
}
// One wave re-reads segment s and returns, to every lane, the id of the token
// at which the inclusive id-order total of val(z, key, id) passes t (or -1).
// The chunk's history table must be built.
template <int DT, typename LT, typename VF>
__device__ __forceinline__ long long seg_find(const Args& a, const RowP& p, int row, const LT& L, int s, u64 t,
                                              VF&& val, u64* seg_total = nullptr) {
  constexpr int VL = Chunk<DT>::VL, J = Chunk<DT>::J;
  const int c = s / (kWaves * J), w = (s / J) % kWaves, j = s % J;
  const int l = lane_id();
  const int i0 = c * kCH + w * kWaveSpan + j * 64 * VL + l * VL;
  const size_t rowoff = (size_t)row * (size_t)a.row_stride;
  u32 x[4] = {0u, 0u, 0u, 0u};
  if (a.vec_ok && i0 + VL <= a.V) {
    const uint4 v = DT == QS_DTYPE_F32 ? gld((const uint4*)((const float*)a.logits + rowoff + i0))
                                       : gld((const uint4*)((const uint16_t*)a.logits + rowoff + i0));
    x[0] = v.x;
    x[1] = v.y;
    x[2] = v.z;
    x[3] = v.w;
  } else if (DT == QS_DTYPE_F32) {
    const float* q = (const float*)a.logits + rowoff;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (i0 + e < a.V) x[e] = __float_as_uint(gld(q + i0 + e));
  } else {
    const uint16_t* q = (const uint16_t*)a.logits + rowoff;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (i0 + e < a.V) x[e >> 1] |= (u32)gld(q + i0 + e) << ((e & 1) * 16);
  }
  u64 v[VL];
  u64 tot = 0;
#pragma unroll
  for (int e = 0; e < VL; ++e) {
    const int id = i0 + e;
    float z = DT == QS_DTYPE_F32 ? __uint_as_float(x[e]) : bf16_to_f32((x[e >> 1] >> ((e & 1) * 16)) & 0xffffu);
    if (p.pen) {
      const int li = id - c * kCH;
      const u32 n = (pen_table(L)[li >> 1] >> ((li & 1) * 16)) & 0xffffu;
      if (n) z = apply_penalty(z, n, p.rep, p.rrep, p.pres, p.freq);
    }
    v[e] = id < a.V ? val(z, id) : 0ull;
    tot += v[e];
  }
  const u64 inc = wave_incl_scan64(tot);
  if (seg_total) *seg_total = ((u64)readlane((u32)(inc >> 32), 63) << 32) | readlane((u32)inc, 63);
  u64 m = inc - tot;
  long long pick = -1;
#pragma unroll
  for (int e = 0; e < VL; ++e) {
    if (m <= t && t < m + v[e]) pick = i0 + e;
    m += v[e];
  }
  const u64 bal = __ballot(pick >= 0);
  if (!bal) return -1;
  const int src = __ffsll((long long)bal) - 1;
  return (long long)readlane((u32)pick, src);
}

// Per-row data of top-k-off rows: the row's bin masses [kRounds][kNB] u64
// (summed by atomics), the listed tokens [G][kLC], then the kept mass of every
// segment known before the final selection [G][kSegMax] (a segment is one
// wave's vector span of a chunk, 64 * VL ids: kWaves * J of them per chunk).
constexpr int kSegMax = 32;
__device__ __forceinline__ u64* row_hist(const Args& a, int row) { return row_data(a, row); }
__device__ __forceinline__ u64* list_base(const Args& a, int row) { return row_data(a, row) + (size_t)kRounds * kNB; }
__device__ __forceinline__ u64* seg_base(const Args& a, int row) { return list_base(a, row) + (size_t)a.G * kLC; }

// ---------------------------------------------------------------- the streaming kernel

// The chunk's candidate quota: nw waves hold logits of the row; each keeps
// at least kw tokens and the chunk at least kc, kc = mu + 4 sqrt(mu) + 2 for the
// mu = k * kCH / V tokens of the row's top k that a chunk holds on average.
// (A heuristic: it sets how many candidates the chunk writes, never the result;
// hardware reciprocal and square root suffice.)
struct Quota {
  int nw, kc, kw, jw;
};
__device__ __forceinline__ Quota topk_quota(const Args& a, const RowP& p, int c) {
  Quota q;
  const int vin = min(kCH, a.V - c * kCH);
  q.nw = min(kWaves, (vin + kWaveSpan - 1) / kWaveSpan);
  const float mu = (float)p.k * a.kmu;
  const float kc = ceilf(mu + 4.0f * __builtin_amdgcn_sqrtf(mu) + 2.0f);
  q.kc = min((int)uni((u32)(int)kc), p.k);
  // kw = ceil(kc / nw) and jw = ceil(kc / kw): by hardware reciprocals, which
  // can only round up (one more candidate wave or token, never fewer)
  const float kcf = (float)q.kc;
  q.kw = min(64, max(1, (int)uni((u32)(int)ceilf(kcf * __builtin_amdgcn_rcpf((float)q.nw)))));
  q.jw = min(q.nw, max(1, (int)uni((u32)(int)ceilf(kcf * __builtin_amdgcn_rcpf((float)q.kw)))));
  return q;
}
// The chunk threshold on 16-bit keys m16 (each thread's largest): tw, the
// kw-th largest per-thread maximum of each wave (lanes holding a maximum >= tw:
// at least kw), then tau, the jw-th largest tw over the waves, so that jw waves
// hold kw tokens >= tau each.  Uses L.s.v[][4].
__device__ __forceinline__ u32 topk_tau16(u32 m16, const Quota& q, Lds& L) {
  u32 tw = 0;
  for (int b = 15; b >= 0; --b) {
    const u32 cand = tw | (1u << b);
    if ((int)popc64(__ballot(m16 >= cand)) >= q.kw) tw = cand;
  }
  if (lane_id() == 0) L.s.v[wave_id()][4] = wave_id() < q.nw ? tw : 0u;
  lds_sync();
  u32 tv[kWaves];
#pragma unroll
  for (int i = 0; i < kWaves; ++i) tv[i] = uni(L.s.v[i][4]);
  static_assert(kWaves == 8, "sorting network for 8 waves");
  constexpr int net[19][2] = {{0, 2}, {1, 3}, {4, 6}, {5, 7}, {0, 4}, {1, 5}, {2, 6}, {3, 7}, {0, 1}, {2, 3},
                              {4, 5}, {6, 7}, {2, 4}, {3, 5}, {1, 4}, {3, 6}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
  for (int i = 0; i < 19; ++i) {
    const u32 x = tv[net[i][0]], y = tv[net[i][1]];
    tv[net[i][0]] = max(x, y);
    tv[net[i][1]] = min(x, y);
  }
  u32 tau = tv[0];
#pragma unroll
  for (int i = 1; i < kWaves; ++i) tau = (i == q.jw - 1) ? tv[i] : tau;
  return tau;
}

// What a top-k chunk's streaming leaves for topk_tail.
struct TkOut {
  u32 n, below, zmax, tau32;
};
// The slot of a top-k chunk after its region is written (n candidates, n =
// 0xffffffff for an overflow), by thread 0: below is the largest z key the
// chunk left out (an upper bound suffices: a larger one can only send the row
// to the exact path), zmax the chunk's largest z key, tau32 the z key at and
// above which every token of the chunk is in its region.
__device__ __forceinline__ void topk_slot(const Args& a, const RowP& p, const int row, const int c, const TkOut& t) {
  Slot* sl = row_slots(a, row);
  const u32 qmax = t.zmax ? skey(qdiv(f_of_key(t.zmax), p)) : 0u;
  const u32 qlow = skey(qdiv(f_of_key(t.tau32), p));
  stc(&sl[c].a, ((u64)t.below << 32) | t.n);
  stc(&sl[c].d, ((u64)qmax << 32) | qlow);
}

// The arrival of a workgroup that wrote nch chunks' slots of a top-k row, and in
// the row's last workgroup the gather and the finish.  Returns kNotLast in the
// other workgroups, else 0 or a reason to resolve the row by the exact path.
// With zk the regions and the slots hold z keys (the rows of topk_pk): the
// entries become keys of q as they are gathered, the chunk extremes after.
__device__ __forceinline__ u32 topk_last(const Args& a, const RowP& p, const int row, const int c, Lds& L, u32 nch,
                                         bool zk) {
  RowSync* sy = &a.sync[row];
  Slot* sl = row_slots(a, row);
  const int R = a.R;
  QS_TR(5);
  if (arrive_n(&sy->arrive, nch, L.s) != (u32)a.G - nch) return kNotLast;
  QS_TR(6);
  // ---- the row's last workgroup: gather and finish
  u32 mx[3];
  auto cnt_of = [&](int cc, u32(&v)[3]) -> u32 {
    const u64 x = ldc(&sl[cc].a), d = ldc(&sl[cc].d);
    v[0] = (u32)(x >> 32);  // largest z key left out
    v[1] = (u32)(d >> 32);  // largest key (of q, or of z with zk)
    v[2] = ~(u32)d;         // the complement of the key of the chunk's threshold
    return (u32)x;
  };
  auto qkey = [&](u32 zkey) -> u32 { return skey(qdiv(f_of_key(zkey), p)); };
  u32 tot;
  if (zk)
    tot = gather_lds(a, row_data(a, row), R, cnt_of, L, mx,
                     [&](u64 e) -> u64 { return ((u64)qkey((u32)(e >> 32)) << 32) | (u32)e; });
  else
    tot = gather_lds(a, row_data(a, row), R, cnt_of, L, mx);
  QS_TR(7);
  const u32 below_max = mx[0];
  const u32 qmax = zk ? (mx[1] ? qkey(mx[1]) : 0u) : mx[1], qlow = zk ? qkey(~mx[2]) : ~mx[2];
  QS_TR(8);
  u32 why = 0u;
  bool done = false;
  if (tot == 0xffffffffu)
    why = kStOverflow;
  else if (finish_topk(a, p, row, L, tot, qmax, qlow, below_max, c))
    done = true;
  else
    why = kStIncomplete;
  QS_TR(14);
  return done ? 0u : why;
}

// The streaming part of a top-k row: the chunk's candidates to its region.
template <int DT>
__device__ __forceinline__ TkOut topk_row(const Args& a, const RowP& p, const int row, const int c, Chunk<DT>& ch,
                                        Lds& L) {
  constexpr int E = kEPT, J = Chunk<DT>::J, VL = Chunk<DT>::VL;
    // z keys
  u32 kz[E];
  u32 m = 0;
  with_pen(p.pen, [&](auto pen) {
    constexpr bool PEN = decltype(pen)::value;
    u32 pw[kEPT / 2] = {};
    if constexpr (PEN) chunk_counts(L, ch, c, pw);
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < VL; ++e) {
        const u32 kx = skey(elem_zt<PEN>(ch, p, pw, j, e));  // 0 past V (NaN padding)
        kz[j * VL + e] = kx;
        m = max(m, kx);
      }
  });
  if (p.pen) lds_sync();
  QS_TR(2);
  const Quota qt = topk_quota(a, p, c);
  u32 tau = max(topk_tau16(m >> 16, qt, L) << 16, 1u);
  QS_TR(3);
  const int R = a.R;
  u32 n = 0, below = 0, zmax = 0;
  u64* reg = row_data(a, row) + (size_t)c * R;
  for (int attempt = 0; attempt < 2; ++attempt) {
    // positions in id order (wave, j, lane, e), the largest key left out and the
    // chunk's largest, with one exchange
    u32 cnt[J], ex[J], tj[J];
    u32 bl = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      u32 x = 0;
#pragma unroll
      for (int e = 0; e < VL; ++e) {
        const u32 kx = kz[j * VL + e];
        x += kx >= tau ? 1u : 0u;
        bl = kx < tau ? max(bl, kx) : bl;
      }
      cnt[j] = x;
    }
    u32 tot = 0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const u32 inc = wave_incl_scan(cnt[j]);
      ex[j] = inc - cnt[j];
      tj[j] = readlane(inc, 63);
      tot += tj[j];
    }
    bl = wave_max(bl);
    const u32 wm = wave_max(m);
    if (lane_id() == 0) {
      L.s.r[wave_id()] = tot;
      L.s.v[wave_id()][5] = bl;
      L.s.v[wave_id()][6] = wm;
    }
    lds_sync();
    u32 woff = 0;
    n = 0;
    below = 0;
    zmax = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      const u32 ti = L.s.r[i];
      woff += i < wave_id() ? ti : 0u;
      n += ti;
      below = max(below, L.s.v[i][5]);
      zmax = max(zmax, L.s.v[i][6]);
    }
    if (n > (u32)R) {
      lds_sync();  // the exchange is read: it may be written again
      if (attempt == 0) {
        tau = tau + 1u;  // ties at tau overflowed the region: strictly above it
        continue;
      }
      n = 0xffffffffu;
      break;
    }
    // each candidate straight to the region, as (key of q << 32 | id)
    u32 run = woff;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      u32 pos = run + ex[j];
#pragma unroll
      for (int e = 0; e < VL; ++e) {
        const u32 kx = kz[j * VL + e];
        if (kx >= tau) {
          const float q = qdiv(f_of_key(kx), p);
          stc(&reg[pos], ((u64)skey(q) << 32) | (u32)ch.id(j, e));
          ++pos;
        }
      }
      run += tj[j];
    }
    QS_TR(4);
    break;
  }
  return TkOut{n, below, zmax, tau};
}

// Top-k and greedy rows of bf16 logits without penalties: a workgroup serves
// kCPW consecutive chunks (chunk c0 = kCPW * i and the next kCPW - 1 of the row),
// all in step, on h keys (two per register), so that the row parameters, the
// exchanges between waves and the arrival are paid once per kCPW chunks.
constexpr int kCPW = 2;

// The bf16 bits of the value with h key h (h >= kHNegInf; -0 for 0x807e).
__host__ __device__ __forceinline__ u32 bf16_of_h(u32 h) {
  const u32 k = (h - 0x7fu) & 0xffffu;
  return k >= 0x8000u ? (k & 0x7fffu) : (~k & 0xffffu);
}

// h keys of a chunk's logits: hk[j * 4 + w] holds the keys of word w of vector
// j (elements 2w and 2w + 1 of the vector); returns the thread's largest.
__device__ __forceinline__ u32 chunk_hkeys(const Chunk<QS_DTYPE_BF16>& ch, u32 (&hk)[kEPT / 2]) {
  u32 m2 = 0;
#pragma unroll
  for (int j = 0; j < Chunk<QS_DTYPE_BF16>::J; ++j) {
    const uint4 v = ch.v[j];
    hk[j * 4 + 0] = hkey2(v.x);
    hk[j * 4 + 1] = hkey2(v.y);
    hk[j * 4 + 2] = hkey2(v.z);
    hk[j * 4 + 3] = hkey2(v.w);
  }
#pragma unroll
  for (int i = 0; i < kEPT / 2; ++i) m2 = pk_max_u16(m2, hk[i]);
  return max(m2 & 0xffffu, m2 >> 16);
}

// The streaming part of a top-k row for chunks c0 .. c0 + nch - 1 (nch <=
// kCPW): each chunk's candidates to its region and its slot.  Per logit pair one
// key, one maximum and one count step; the tokens at or above a chunk's
// threshold are written by the threads that hold them (a few per chunk); the
// largest key a chunk leaves out is bounded by its threshold's predecessor.
template <int NC>
__device__ __forceinline__ void topk_pk(const Args& a, const RowP& p, const int row, const int c0, const int nch,
                                        const Chunk<QS_DTYPE_BF16>* ch, Lds& L) {
  constexpr int NW = kEPT / 2, WPV = 4, J = Chunk<QS_DTYPE_BF16>::J;
  const int R = a.R;
  u32 hk[NC][NW];
  u32 m[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) m[k] = chunk_hkeys(ch[k], hk[k]);
  QS_TRA(2);
  // thresholds: per chunk tw (each wave's kw-th largest per-thread maximum),
  // then tau, the jw-th largest tw over the waves, all chunks in one exchange.
  // Every chunk but the row's last has the same quota.
  const Quota qf = topk_quota(a, p, 0);
  const Quota ql = c0 + NC > a.G - 1 ? topk_quota(a, p, a.G - 1) : qf;
  u32 tw[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) tw[k] = 0;
  for (int b = 15; b >= 0; --b) {
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int kw = c0 + k == a.G - 1 ? ql.kw : qf.kw;
      const u32 cand = tw[k] | (1u << b);
      if ((int)popc64(__ballot(m[k] >= cand)) >= kw) tw[k] = cand;
    }
  }
  if (lane_id() == 0) {
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int nw = c0 + k == a.G - 1 ? ql.nw : qf.nw;
      L.s.v[wave_id()][4 + k] = wave_id() < nw ? tw[k] : 0u;
    }
  }
  lds_sync();
  // the jw-th largest of the eight: lane k * 8 + i holds wave i's value of
  // chunk k; a bitonic sort of each group of eight lanes (descending) by DPP
  u32 tau[NC];
  {
    const int l = (int)lane_id();
    const int kk = min(l >> 3, NC - 1);
    u32 v = L.s.v[l & 7][4 + kk];
    // compare-exchange with the partner lane; the lane in the lower half of the
    // pair's block keeps the larger (a bitonic network with mirrored merges)
#define QS_CX(CTRL, lowbit)                                  \
  {                                                          \
    const u32 o = dpp_mov<CTRL, 0xF>(v);                     \
    v = (l & (lowbit)) == 0 ? max(v, o) : min(v, o);         \
  }
    QS_CX(0xB1, 1)   // quad_perm [1,0,3,2]: partner l ^ 1
    QS_CX(0x1B, 2)   // quad_perm [3,2,1,0]: partner l ^ 3
    QS_CX(0xB1, 1)
    QS_CX(0x141, 4)  // row_half_mirror: partner 7 - l within the 8
    QS_CX(0x4E, 2)   // quad_perm [2,3,0,1]: partner l ^ 2
    QS_CX(0xB1, 1)
#undef QS_CX
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const int jw = c0 + k == a.G - 1 ? ql.jw : qf.jw;
      tau[k] = max(readlane(v, k * 8 + jw - 1), kHNegInf);  // never a NaN
    }
  }
  QS_TRA(3);
  // counts per (chunk, vector) and their offsets in id order (wave, j, lane, e);
  // the chunk's total and largest key, all chunks in one exchange
  u32 pos[NC][J], n[NC], zmax[NC];
  u32 has = 0;  // bit k * J + j: this thread holds a candidate in vector j of chunk k
  for (int attempt = 0; attempt < 2; ++attempt) {
    has = 0;
#pragma unroll
    for (int k = 0; k < NC; ++k) {
      const u32 t1 = (tau[k] - 1u) * 0x10001u;
      u32 tot = 0;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        u32 acc = 0;
#pragma unroll
        for (int w = 0; w < WPV; ++w) acc = pk_add_u16(acc, pk_above(hk[k][j * WPV + w], t1));
        const u32 cn = (acc & 0xffffu) + (acc >> 16);
        has |= cn != 0u ? 1u << (k * J + j) : 0u;
        const u32 inc = wave_incl_scan(cn);
        pos[k][j] = tot + inc - cn;
        tot += readlane(inc, 63);
      }
      const u32 wm = wave_max(m[k]);
      if (lane_id() == 0) L.s.w[wave_id()][k] = ((u64)tot << 32) | wm;
    }
    lds_sync();
    // lane k * 8 + i takes wave i's (total, largest) of chunk k: prefix sums
    // and maxima within each group of eight lanes
    static_assert(NC * kWaves <= 16, "the chunks' groups fit one row of 16 lanes");
    bool over = false;
    {
      const int l = (int)lane_id();
      const u64 x = L.s.w[l & 7][min(l >> 3, NC - 1)];
      u32 t = (u32)(x >> 32), zm = (u32)x;
      const int gi = l & 7;  // position within the group
      // inclusive scan and running maximum over the group (row_shr within
      // the row of 16; contributions from the group below are masked)
      u32 s1 = dpp_mov<0x111, 0xF>(t), z1 = dpp_mov<0x111, 0xF>(zm);
      t += gi >= 1 ? s1 : 0u;
      zm = gi >= 1 ? max(zm, z1) : zm;
      s1 = dpp_mov<0x112, 0xF>(t);
      z1 = dpp_mov<0x112, 0xF>(zm);
      t += gi >= 2 ? s1 : 0u;
      zm = gi >= 2 ? max(zm, z1) : zm;
      s1 = dpp_mov<0x114, 0xF>(t);
      z1 = dpp_mov<0x114, 0xF>(zm);
      t += gi >= 4 ? s1 : 0u;
      zm = gi >= 4 ? max(zm, z1) : zm;
      const u32 incl = t, own = (u32)(x >> 32);
#pragma unroll
      for (int k = 0; k < NC; ++k) {
        n[k] = readlane(incl, k * 8 + 7);
        zmax[k] = readlane(zm, k * 8 + 7);
        const u32 woff = readlane(incl - own, k * 8 + wave_id());
#pragma unroll
        for (int j = 0; j < J; ++j) pos[k][j] += woff;
        over = over || (k < nch && n[k] > (u32)R);
      }
    }
    if (!over) break;
    lds_sync();  // the exchange is read: it may be written again
    if (attempt == 1) break;
#pragma unroll
    for (int k = 0; k < NC; ++k)
      if (n[k] > (u32)R) tau[k] += 1u;  // ties at tau overflowed the region: strictly above it
  }
  // each candidate straight to its chunk's region, as (key of q << 32 | id), by
  // the threads that hold one, in id order (j, word, half)
  const int base = ch[0].base;
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    if (k >= nch || n[k] > (u32)R) continue;
    u64* reg = row_data(a, row) + (size_t)(c0 + k) * R;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (has & (1u << (k * J + j))) {
        u32 ps = pos[k][j];
#pragma unroll
        for (int w = 0; w < WPV; ++w) {
          const u32 hw = hk[k][j * WPV + w];
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const u32 h = (hw >> (16 * hf)) & 0xffffu;
            if (h >= tau[k]) {
              const int id = base + k * kCH + j * 64 * Chunk<QS_DTYPE_BF16>::VL + 2 * w + hf;
              stc(&reg[ps], ((u64)key_of_h(h) << 32) | (u32)id);
              ++ps;
            }
          }
        }
      }
    }
  }
  QS_TRA(4);
  // slots with z keys (topk_last converts them)
  if (threadIdx.x < (u32)nch) {
    Slot* sl = row_slots(a, row);
    u32 nk = 0, t = 0, zm = 0;
#pragma unroll
    for (int k = 0; k < NC; ++k)
      if ((int)threadIdx.x == k) {
        nk = n[k] > (u32)R ? 0xffffffffu : n[k];
        t = tau[k];
        zm = zmax[k];
      }
    stc(&sl[c0 + threadIdx.x].a, ((u64)key_of_h(t - 1u) << 32) | nk);
    stc(&sl[c0 + threadIdx.x].d, ((u64)key_of_h(zm) << 32) | key_of_h(t));
  }
}

// The same for a greedy row: each chunk's (greedy key, ~id) to its slot.  The g
// key h - 0xfe (mod 2^16) puts the NaNs above +inf; the first index of the
// chunk's largest is found by the threads that hold it (with -0 equal to +0 and
// every NaN equal).  Logits past V (NaN padding) are masked to the lowest key.
template <int NC>
__device__ __forceinline__ void greedy_pk(const Args& a, const int row, const int c0, const int nch,
                                          const Chunk<QS_DTYPE_BF16>* ch, Lds& L) {
  constexpr int NW = kEPT / 2, WPV = 4, J = Chunk<QS_DTYPE_BF16>::J;
  constexpr u32 kGOff = 0xff02ff02u;  // -0xfe in both halves
  u32 gk[NC][NW];
  u32 gm[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    chunk_hkeys(ch[k], gk[k]);
    const bool last = c0 + k == a.G - 1;  // the chunk that may run past V
    u32 m2 = 0;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int w = 0; w < WPV; ++w) {
        u32 g = pk_add_u16(gk[k][j * WPV + w], kGOff);
        if (last) {
          const u32 lo = ch[k].valid(j, 2 * w) ? 0xffffu : 0u, hi = ch[k].valid(j, 2 * w + 1) ? 0xffff0000u : 0u;
          g &= lo | hi;
        }
        gk[k][j * WPV + w] = g;
        m2 = pk_max_u16(m2, g);
      }
    gm[k] = max(m2 & 0xffffu, m2 >> 16);
  }
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const u32 wmx = wave_max(gm[k]);
    if (lane_id() == 0) L.s.v[wave_id()][4 + k] = wmx;
  }
  lds_sync();
  u32 G[NC], first[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    G[k] = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) G[k] = max(G[k], L.s.v[i][4 + k]);
    // the keys equal to the largest: every NaN; -0 and +0 (g 0x7f80, 0x7f81)
    const u32 lo = G[k] >= 0xff02u ? 0xff02u : (G[k] == 0x7f81u ? 0x7f80u : G[k]);
    u32 id = 0xffffffffu;
    if (gm[k] >= lo) {
#pragma unroll
      for (int j = 0; j < J; ++j)
#pragma unroll
        for (int w = 0; w < WPV; ++w)
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const u32 g = (gk[k][j * WPV + w] >> (16 * hf)) & 0xffffu;
            const u32 i = (u32)ch[k].id(j, 2 * w + hf);
            id = (g >= lo && i < id) ? i : id;
          }
    }
    first[k] = wave_min(id);
  }
  lds_sync();  // the maxima are read: the exchange may be written again
  if (lane_id() == 0) {
#pragma unroll
    for (int k = 0; k < NC; ++k) L.s.v[wave_id()][4 + k] = first[k];
  }
  lds_sync();
  if (threadIdx.x == 0) {
    Slot* sl = row_slots(a, row);
#pragma unroll
    for (int k = 0; k < NC; ++k)
      if (k < nch) {
        u32 id = 0xffffffffu;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) id = min(id, L.s.v[i][4 + k]);
        u32 key;
        if (G[k] >= 0xff02u) {
          key = 0xffffffffu;  // NaN
        } else {
          key = key_of_h((G[k] + 0xfeu) & 0xffffu);
          if (key == 0x7fffffffu) key = 0x80000000u;  // -0 as +0
        }
        // a chunk of padding only has no id: key 0 loses to every real logit
        stc(&sl[c0 + k].a, id == 0xffffffffu ? 0ull : (((u64)key << 32) | (0xffffffffu - id)));
      }
  }
}

// A top-k-off row: keys, the row barrier, weights, the bracket rounds, and (in
// the row's last workgroup) the selection and the draw.  Returns as topk_row.
template <int DT>
__device__ __forceinline__ u32 mass_row(const Args& a, const RowP& p, const int row, const int c, Chunk<DT>& ch,
                                        Lds& L) {
  constexpr int E = kEPT, J = Chunk<DT>::J, VL = Chunk<DT>::VL;
  RowSync* sy = &a.sync[row];
  Slot* sl = row_slots(a, row);
  {
    u32 kr[E];
    chunk_qkeys<DT>(ch, p, L, c, kr);
    if (p.pen) lds_sync();  // the count table is read no more: the keys go over it
    u32 kmx = 0, kmn = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      kmx = max(kmx, kr[i]);
      if (kr[i]) kmn = min(kmn, kr[i]);
      L.u.kq[i * kThreads + threadIdx.x] = kr[i];
    }
    kmn = ~kmn;
    block_max2(kmx, kmn, L.s);
    kmn = ~kmn;
    if (threadIdx.x == 0) stc(&sl[c].a, ((u64)kmx << 32) | kmn);
  }
  QS_TR(2);
  (void)arrive(&sy->barA, L.s);
  bool ok = wait_count(a, row, &sy->barA, (u32)a.G, L.s);
  QS_TR(3);
  u32 kstar = 0, kmin = 0xffffffffu;
  if (ok) {
    for (int cc = threadIdx.x; cc < a.G; cc += kThreads) {
      const u64 v = ldc(&sl[cc].a);
      kstar = max(kstar, (u32)(v >> 32));
      kmin = min(kmin, (u32)v);
    }
    kmin = ~kmin;
    block_max2(kstar, kmin, L.s);
    kmin = ~kmin;
    QS_TR(4);
    if (kstar == 0u) {
      fail_row(a, row, kStIncomplete);  // no weights: resolved alone
      ok = false;
    }
  }
  const int SH = a.SH;
  const u64 thr = ceil_scaled(p.mp, 23 + SH);
  const u32 pthr = uni(packed_threshold(thr));
  const float qs = f_of_key(kstar);
  // first-round bins over x = q* - q in [0, D], D = min(q* - q_min, kXMax)
  MassBins mb = mass_bins_first(qs - f_of_key(kmin));
  u64 Tp = 0, A = 0;  // floor(top_p * S), the mass above the bracket
  if (ok) {
    // weights (packed, kept in registers), the chunk's mass and (top-p) the
    // first-round mass histogram, in one pass
    if (p.topp) {
      for (int b = threadIdx.x; b < kNB; b += kThreads) L.mh[b] = 0ull;
      lds_sync();
    }
    u32 wp[E];
    u32 bq[E / 4];  // each token's bin of the current round, four per word
    u64 Sc = 0;
    u32 nz = 0, inb = 0;
#pragma unroll
    for (int i = 0; i < E / 4; ++i) bq[i] = 0u;
    // A finite q* without min_p (the common row): the weight straight from
    // d = q - q* (weight_finite's clamp, no keys, no unpacking), packed for the
    // later rounds; the keyed form otherwise.
    const float flmin = -(float)(SH + 40);
    auto weigh = [&](auto plain) {
      constexpr bool PLAIN = decltype(plain)::value;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const u32 k = L.u.kq[i * kThreads + threadIdx.x];
        const float q = f_of_key(k);
        u32 x;
        u64 w;
        if constexpr (PLAIN) {
          const float d = q - qs;
          const float y = d * kL2E;
          const float fl = __builtin_floorf(y);
          const float f = y - fl;
          float pe = exp2_poly(f);
          pe = __builtin_amdgcn_fmed3f(pe, 1.0f, __uint_as_float(0x3fffffffu));
          const u32 m = 0x800000u | (__float_as_uint(pe) & 0x7fffffu);
          const int sx = (int)fmaxf(fl, flmin) + SH;
          w = ((u64)m << max(sx, 0)) >> max(-sx, 0);
          x = sx > -24 ? ((u32)(sx + 64) << 24) | m : 0u;  // wpack_of's form: w != 0 exactly then
        } else {
          x = wpack_of(q, k, qs, kstar, SH);
          x = x >= pthr ? x : 0u;
          w = wunpack(x);
        }
        wp[i] = x;
        Sc += w;
        nz += x ? 1u : 0u;
        inb |= (x ? 1u : 0u) << i;
        if (p.topp && x) {
          const u32 bi = PLAIN ? mass_bin_first(q - qs, mb) : mass_bin(q, k, qs, kstar, mb);
          bq[i / 4] |= bi << (8 * (i % 4));
          atomicAdd(&L.mh[bi], w);
        }
      }
    };
    if (qs - qs == 0.0f && pthr == 0u)
      weigh(Tag<true>{});
    else
      weigh(Tag<false>{});
    QS_TR(5);
    if (!p.topp) {  // every weight is kept: the segments' masses
      u64* sg = seg_base(a, row) + (size_t)c * kSegMax;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        u64 sj = 0;
#pragma unroll
        for (int e = 0; e < VL; ++e) sj += wunpack(wp[j * VL + e]);
        sj = wave_sum64(sj);
        if (lane_id() == 0) stc(&sg[wave_id() * J + j], sj);
      }
    }
    if (p.topp) {
      lds_sync();  // the histogram is complete (the chunk's sums are not needed: the lists replace them)
    } else {
      block_sum2(Sc, nz, L.s);
      if (threadIdx.x == 0) {
        stc(&sl[c].b, Sc);
        stc(&sl[c].c, (u64)nz);
      }
    }
    QS_TR(6);
    if (p.topp) {
      // Bracket the top-p boundary: each round, every workgroup adds its mass
      // histogram of the tokens still in the bracket to the row's (atomics),
      // waits for the row, and reads it; the bin holding the boundary is either
      // listed (few enough tokens, bounded by the bin's mass over its least
      // weight) or split again.  Every workgroup decides alike.
      u32 abv = 0;  // tokens above the bracket
      u64* hr = row_hist(a, row);
      bool listed = false;
      for (int r = 0; r < kRounds && ok && !listed; ++r) {
        if (r > 0) {
          for (int b = threadIdx.x; b < kNB; b += kThreads) L.mh[b] = 0ull;
          lds_sync();
#pragma unroll
          for (int i = 0; i < E / 4; ++i) bq[i] = 0u;
#pragma unroll
          for (int i = 0; i < E; ++i) {
            if ((inb >> i) & 1u) {
              const u32 k = L.u.kq[i * kThreads + threadIdx.x];
              const u32 bi = mass_bin(f_of_key(k), k, qs, kstar, mb);
              bq[i / 4] |= bi << (8 * (i % 4));
              atomicAdd(&L.mh[bi], wunpack(wp[i]));
            }
          }
          lds_sync();
        }
        QS_TR(7 + 4 * r);
        for (int b = threadIdx.x; b < kNB; b += kThreads) {
          const u64 v = L.mh[b];
          if (v) addc(&hr[(size_t)r * kNB + b], v);
        }
        (void)arrive(&sy->barB, L.s);
        QS_TR(8 + 4 * r);
        ok = wait_count(a, row, &sy->barB, (u32)a.G * (u32)(r + 1), L.s);
        QS_TR(9 + 4 * r);
        if (!ok) break;
        // the row's bins: the crossing bin and the mass above it, by one wave
        // (bins 4l .. 4l + 3 in lane l), the choice to the others through LDS
        if (threadIdx.x < 64) {
          static_assert(kNB == 256, "four bins per lane");
          const int l = (int)lane_id();
          u64 bm4[4], sb = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            bm4[i] = ldc(&hr[(size_t)r * kNB + 4 * l + i]);
            sb += bm4[i];
          }
          const u64 inc = wave_incl_scan64(sb);
          if (r == 0) Tp = mul_frac(readlane64(inc, 63), p.tp);
          const u64 target = Tp - A;
          u64 ex = inc - sb;
          if (l == 0) L.s.r[12] = 0xffffffffu;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (ex <= target && target < ex + bm4[i]) {
              const int b = 4 * l + i;
              L.s.r[12] = (u32)b;
              L.s.r64[12] = ex;
              // tokens of the bin: at most its mass over its least weight
              const float wl = bin_least_weight(mb, b, SH);
              L.s.r[13] = (float)bm4[i] <= wl * (float)kFCap ? 1u : 0u;
            }
            ex += bm4[i];
          }
          if (l == 0) L.s.r64[13] = Tp;
        }
        lds_sync();
        const u32 bsel = uni(L.s.r[12]);
        const u32 small = uni(L.s.r[13]);
        const u64 exs = uni64(L.s.r64[12]);
        Tp = uni64(L.s.r64[13]);
        lds_sync();
        if (bsel == 0xffffffffu || (!small && r + 1 == kRounds)) {
          fail_row(a, row, kStList);
          ok = false;
          break;
        }
        A += exs;
#pragma unroll
        for (int i = 0; i < E; ++i) {
          const u32 bi = (bq[i / 4] >> (8 * (i % 4))) & 0xffu;
          if (((inb >> i) & 1u) && bi < bsel) abv |= 1u << i;
          if (bi != bsel) inb &= ~(1u << i);
        }
        listed = small != 0u;
        mb = mass_bins_split(mb, bsel);
        QS_TR(10 + 4 * r);
      }
      if (ok) {
        // mass above the bracket (per segment too), and the bracket's tokens listed in
        // id order; the waves' totals, masses and counts in one exchange
        u64 above_w = 0;
        u32 cnt[J];
        u64* sg = seg_base(a, row) + (size_t)c * kSegMax;
#pragma unroll
        for (int j = 0; j < J; ++j) {
          cnt[j] = 0;
          u64 sj = 0;
#pragma unroll
          for (int e = 0; e < VL; ++e) {
            const int i = j * VL + e;
            sj += ((abv >> i) & 1u) ? wunpack(wp[i]) : 0ull;
            cnt[j] += (inb >> i) & 1u;
          }
          sj = wave_sum64(sj);
          above_w += sj;
          if (lane_id() == 0) stc(&sg[wave_id() * J + j], sj);
        }
        const u32 na_w = wave_sum((u32)__popc(abv));
        u32 ex[J], tot = 0;
        static_assert(J <= 4, "the exchange holds four vector counts per wave");
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const u32 inc = wave_incl_scan(cnt[j]);
          ex[j] = inc - cnt[j];
          const u32 tj = readlane(inc, 63);
          if (lane_id() == 0) L.s.v[wave_id()][j] = tj;
          tot += tj;
        }
        if (lane_id() == 0) {
          L.s.r[wave_id()] = tot;
          L.s.w[wave_id()][0] = above_w;
          L.s.v[wave_id()][4] = na_w;
        }
        lds_sync();
        u32 woff = 0, nl = 0;
#pragma unroll
        for (int i = 0; i < kWaves; ++i) {
          woff += i < wave_id() ? L.s.r[i] : 0u;
          nl += L.s.r[i];
        }
        u32 joff[J];
        {
          u32 run = woff;
#pragma unroll
          for (int j = 0; j < J; ++j) {
            joff[j] = run;
            run += L.s.v[wave_id()][j];
          }
        }
        u64 above = 0;
        u32 na = 0;
        if (threadIdx.x == 0) {
#pragma unroll
          for (int i = 0; i < kWaves; ++i) {
            above += L.s.w[i][0];
            na += L.s.v[i][4];
          }
        }
        u64* lst = list_base(a, row) + (size_t)c * kLC;
#pragma unroll
        for (int j = 0; j < J; ++j) {
          u32 pos = joff[j] + ex[j];
#pragma unroll
          for (int e = 0; e < VL; ++e) {
            const int i = j * VL + e;
            if ((inb >> i) & 1u) {
              if (pos < (u32)kLC) stc(&lst[pos], ((u64)L.u.kq[i * kThreads + threadIdx.x] << 32) | (u32)ch.id(j, e));
              ++pos;
            }
          }
        }
        if (threadIdx.x == 0) {
          if (nl > (u32)kLC) orc(&sy->status, kStOverflow);  // more than the bound allowed for
          stc(&sl[c].b, above);
          stc(&sl[c].c, ((u64)nl << 32) | na);
        }
      }
    }
  }
  QS_TR(19);
  if (arrive(&sy->arrive, L.s) != (u32)a.G - 1u) return kNotLast;
  QS_TR(20);
  // ---- the row's last workgroup: the selector
  if (p.topp) {  // every workgroup is past the row histograms: back to zero
    u64* hr = row_hist(a, row);
    for (int i = threadIdx.x; i < kRounds * kNB; i += kThreads) stc(&hr[i], 0ull);
  }
  // every chunk's segment masses, when they fit, in the same round trip as the
  // lists (the owner of the draw is known only after the selection)
  const int nsg = kWaves * J;
  const bool segpre = a.G * nsg <= kSegPre;
  constexpr int kSP = kSegPre / kThreads;
  u64 spv[kSP];
  if (segpre) {
#pragma unroll
    for (int i = 0; i < kSP; ++i) {
      const int f = (int)threadIdx.x + i * kThreads;
      spv[i] = f < a.G * nsg ? ldc(seg_base(a, row) + (size_t)(f / nsg) * kSegMax + (f % nsg)) : 0ull;
    }
  }
  // without top-p: the chunks' masses and counts, loaded before the status so
  // that both come back in one round trip (G <= kMaxG < kThreads: one per thread)
  u64 cmb = 0, cmc = 0;
  if (!p.topp && (int)threadIdx.x < a.G) {
    cmb = ldc(&sl[threadIdx.x].b);
    cmc = ldc(&sl[threadIdx.x].c);
  }
  const u32 st = ldc(&sy->status);
  if (segpre) {
#pragma unroll
    for (int i = 0; i < kSP; ++i) L.segm[threadIdx.x + i * kThreads] = spv[i];
  }
  if (st != 0u || kstar == 0u) return st ? st : kStIncomplete;
  // per-chunk kept masses and tie counts in L.cmass / L.cties
  u64 W = 0, wt = 0;
  u32 nlist = 0;  // listed tokens (in L.u.fin.ent, id order)
  u32 klo = 1u, jties = 0xffffffffu, kept = 0, idlo = (u32)a.V;
  bool fine = true;
  auto wpk = [&](u32 key) -> u32 {
    const u32 x = wpack_of(f_of_key(key), key, qs, kstar, SH);
    return wunpack(x) >= thr ? x : 0u;
  };
  auto wf = [&](u32 key) -> u64 { return wunpack(wpk(key)); };
  if (!p.topp) {
    static_assert(kMaxG <= kThreads, "one chunk per thread");
    u32 nzt = 0;
    if ((int)threadIdx.x < a.G) {
      L.cmass[threadIdx.x] = cmb;
      nzt = (u32)cmc;
      L.cties[threadIdx.x] = 0u;
    }
    kept = block_sum(nzt, L.s);
  } else {
    const u64 Ahi = A;
    u32 nat = 0;
    u32 mx[3];
    const u32 n = nlist = gather_lds(a, list_base(a, row), kLC, [&](int cc, u32(&)[3]) -> u32 {
      const u64 cv = ldc(&sl[cc].c);
      L.cmass[cc] = ldc(&sl[cc].b);
      nat = (u32)cv;
      return (u32)(cv >> 32);  // listed tokens of the chunk
    }, L, mx);
    QS_TR(21);
    if (n == 0xffffffffu || n == 0u) {
      fine = false;
    } else if (n <= 64u) {
      // A short list: one wave orders it by (key desc, id asc), keeps the prefix
      // whose exclusive mass stays within Tp - A, and adds the kept weights to
      // their chunks (no tie accounting: each kept token is known).
      nat = block_sum(nat, L.s);
      if (threadIdx.x < 64) {
        const u32 l = lane_id();
        const bool have = l < n;
        const u64 e = have ? L.u.fin.ent[l] : 0ull;
        const u32 key = (u32)(e >> 32), id = (u32)e;
        const u64 wv = have ? wf(key) : 0ull;
        u64 pre = 0;  // mass of the tokens before this one in (key desc, id asc) order
        for (u32 j = 0; j < n; ++j) {
          const u32 kj = readlane(key, (int)j), ij = readlane(id, (int)j);
          const u64 wj = readlane64(wv, (int)j);
          pre += (kj > key || (kj == key && ij < id)) ? wj : 0ull;
        }
        const u64 T1 = Tp - Ahi;
        const bool kp = have && wv != 0ull && pre <= T1;
        // the last kept token: the largest prefix among the kept
        const u64 lastpre = kp ? pre : 0ull;
        u64 mp = lastpre;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const u64 x = ((u64)(u32)__shfl_xor((int)(u32)(mp >> 32), o) << 32) | (u32)__shfl_xor((int)(u32)mp, o);
          mp = x > mp ? x : mp;
        }
        const u64 lb = __ballot(kp && pre == mp);
        const u32 nkp = popc64(__ballot(kp));
        const u64 inc = pre + wv;
        if (kp) atomicAdd(&L.cmass[id / (u32)kCH], wv);
        const int src = lb ? __ffsll((long long)lb) - 1 : 0;
        const u32 klast = readlane(key, src), ilast = readlane(id, src);
        const u64 wlast = readlane64(inc, src);
        if (l == 0u) {
          L.s.r[13] = lb ? nkp : 0u;
          L.s.r[14] = klast;
          L.s.r[15] = ilast;
          L.s.r64[14] = Ahi + wlast;
        }
      }
      for (int cc = threadIdx.x; cc < a.G; cc += kThreads) L.cties[cc] = 0u;
      lds_sync();
      const u32 nk = L.s.r[13];
      if (nk == 0u) {
        fine = false;  // the crossing lies outside the list: cannot happen
      } else {
        klo = L.s.r[14];
        idlo = L.s.r[15];
        W = L.s.r64[14];
        A = W;
        kept = nat + nk;
      }
      lds_sync();
    } else {
      // the exact boundary among the listed tokens (in id order in L.u.fin.ent)
      Held h;
      hold_entries(L, n, h);
      u32 wq[kFPer];
      u32 bkmax = 0, bkmin = 0u;
#pragma unroll
      for (int i = 0; i < kFPer; ++i) {
        wq[i] = 0u;
        if ((u32)i < h.per) {
          const u32 key = (u32)(h.e[i] >> 32);
          wq[i] = key ? wpk(key) : 0u;
          bkmax = max(bkmax, key);
          bkmin = key ? max(bkmin, ~key) : bkmin;
        }
      }
      block_max2_sum(bkmax, bkmin, nat, L.s);
      bkmin = ~bkmin;
      // (the per-chunk tie counts are cleared here: the select's barriers order it)
      for (int cc = threadIdx.x; cc < a.G; cc += kThreads) L.cties[cc] = 0u;
      const SelRes q = held_select<true>(a, L, h, wq, max(bkmin, 1u), bkmax, Tp - Ahi);
      if (!q.ok) {
        fine = false;
      } else {
        klo = q.kappa;
        wt = wf(klo);  // every token at kappa_p has this weight
        A = Ahi + q.mass_above;
        const u64 jj = div_small(Tp - A, wt) + 1ull;
        jties = (u32)(jj < (u64)q.cnt_at ? jj : (u64)q.cnt_at);
        W = A + (u64)jties * wt;
        kept = nat + q.cnt_above + jties;
        // per chunk: listed mass above kappa_p and ties at it; the jties-th tie's id
        u32 tcount = 0;
#pragma unroll
        for (int i = 0; i < kFPer; ++i) {
          if ((u32)i < h.per) {
            const u32 key = (u32)(h.e[i] >> 32);
            const int cc = (int)((u32)h.e[i] / (u32)kCH);
            if (wq[i] && key > klo) atomicAdd(&L.cmass[cc], wunpack(wq[i]));
            if (wq[i] && key == klo) {
              atomicAdd(&L.cties[cc], 1u);
              ++tcount;
            }
          }
        }
        // id of the jties-th tie in id order
        u32 ttot;
        u32 tex = block_excl(tcount, L.s, &ttot);
        if (threadIdx.x == 0) L.s.r[14] = (u32)a.V;
        lds_sync();
#pragma unroll
        for (int i = 0; i < kFPer; ++i) {
          if ((u32)i < h.per) {
            const u32 key = (u32)(h.e[i] >> 32);
            if (wq[i] && key == klo) {
              ++tex;
              if (tex == jties) L.s.r[14] = (u32)h.e[i];
            }
          }
        }
        lds_sync();
        idlo = L.s.r[14];
      }
    }
  }
  QS_TR(22);
  if (!fine) return kStList;
  // the chunk holding the draw: kept(c) = cmass[c] + min(ties(c), jties left) * wt;
  // one wave scans the chunks, four per lane
  if (threadIdx.x < 64) {
    const int l = (int)lane_id();
    u64 km[4];
    u32 tn[4], ts = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cc = 4 * l + i;
      km[i] = cc < a.G ? L.cmass[cc] : 0ull;
      tn[i] = cc < a.G ? L.cties[cc] : 0u;
      ts += tn[i];
    }
    u32 tb = wave_incl_scan(ts) - ts;
    u64 ks = 0;
    u64 kc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32 jl = jties == 0xffffffffu ? 0u : (jties > tb ? jties - tb : 0u);
      kc[i] = km[i] + (u64)min(tn[i], jl) * wt;
      ks += kc[i];
      tb += tn[i];
    }
    const u64 ki = wave_incl_scan64(ks);
    const u64 Wt = readlane64(ki, 63);
    if (!p.topp) W = Wt;
    const u64 t = mul_frac(W, p.u);
    u64 acc = ki - ks;
    tb = wave_incl_scan(ts) - ts;
    if (l == 0) L.s.r[15] = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32 jl = jties == 0xffffffffu ? 0u : (jties > tb ? jties - tb : 0u);
      if (acc <= t && t < acc + kc[i]) {
        L.s.r[15] = (u32)(4 * l + i);
        L.s.r64[13] = t - acc;
        L.s.r[7] = jl;
      }
      acc += kc[i];
      tb += tn[i];
    }
    if (l == 0) L.s.r64[14] = W;
  }
  lds_sync();
  const int owner = (int)L.s.r[15];
  const u64 tin = L.s.r64[13];
  const u32 jl = L.s.r[7];
  W = L.s.r64[14];
  lds_sync();
  if (owner < 0) return kStIncomplete;
  QS_TR(23);
  // the segment of the owner chunk holding the draw: the segments' masses known
  // before the selection, plus (top-p) the listed tokens kept
  (void)jl;
  const u64* sg = seg_base(a, row) + (size_t)owner * kSegMax;
  if ((int)threadIdx.x < nsg) L.cmass[threadIdx.x] = segpre ? L.segm[owner * nsg + threadIdx.x] : ldc(&sg[threadIdx.x]);
  lds_sync();
  if (p.topp) {
    for (u32 i = threadIdx.x; i < nlist; i += kThreads) {
      const u64 e = L.u.fin.ent[i];
      const u32 key = (u32)(e >> 32), id = (u32)e;
      if ((int)(id / (u32)kCH) == owner && (key > klo || (key == klo && id <= idlo))) {
        const u64 w = wf(key);
        if (w) atomicAdd(&L.cmass[(id - (u32)owner * kCH) / (64 * VL)], w);
      }
    }
    lds_sync();
  }
  if (threadIdx.x < 64) {
    const int l = (int)lane_id();
    const u64 m = l < nsg ? L.cmass[l] : 0ull;
    const u64 inc = wave_incl_scan64(m);
    const u64 bal = __ballot(m && inc - m <= tin && tin < inc);
    if (l == 0) L.s.r[15] = bal ? (u32)(__ffsll((long long)bal) - 1) : 0xffffffffu;
    const int src = bal ? __ffsll((long long)bal) - 1 : 0;
    const u64 ex = readlane64(inc - m, src);
    if (l == 0) L.s.r64[13] = tin - ex;
  }
  lds_sync();
  const u32 sloc = L.s.r[15];
  const u64 tin2 = L.s.r64[13];
  lds_sync();
  if (sloc == 0xffffffffu) return kStIncomplete;
  if (p.pen) pen_build(p, owner, L);
  QS_TR(24);
  if (threadIdx.x < 64) {
    const bool topp = p.topp;
    const long long id = seg_find<DT>(a, p, row, L, owner * nsg + (int)sloc, tin2, [&](float z, int i) -> u64 {
      const float q = qdiv(z, p);
      const u32 k = skey(q);
      u64 w = weight_of(q, k, qs, kstar, SH);
      w = w >= thr ? w : 0ull;
      if (!topp) return w;
      return (k > klo || (k == klo && (u32)i <= idlo)) ? w : 0ull;
    });
    if (threadIdx.x == 0) L.s.r[15] = id < 0 ? 0xffffffffu : (u32)id;
  }
  lds_sync();
  const u32 pk = L.s.r[15];
  lds_sync();
  if (pk == 0xffffffffu) return kStIncomplete;
  const long long pick = (long long)pk;
  write_result(a, row, p, pick, W, thr, p.topp ? kPathMassTopP : kPathMassAll, 0u, kstar, p.topp ? klo : 1u,
               p.topp ? idlo : (u32)a.V, kept);
  QS_TR(25);
  return 0u;
}

// 128 VGPRs at most: two 512-thread workgroups per CU.
template <int DT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_sample(Args a) {
  __shared__ Lds L;
  constexpr int E = kEPT, J = Chunk<DT>::J, VL = Chunk<DT>::VL;
  const int c = blockIdx.x;
  const int row = (int)uni(a.order ? (u32)sld(a.order + blockIdx.y) : blockIdx.y);
  if ((unsigned)row >= (unsigned)a.B) return;  // row_order must be a permutation of [0, B)
  QS_TR(0);
  // bf16 rows: the workgroup of chunk c = 0 mod kCPW (the lead) serves the next
  // kCPW - 1 chunks too for top-k and greedy rows without penalties.  Without
  // histories (no row has penalties) the other workgroups load their chunk once
  // the row parameters show that it is theirs; with histories they load it at
  // once (most such rows have penalties and need every workgroup).
  const bool lead = DT != QS_DTYPE_BF16 || c % kCPW == 0;
  const bool eager = lead || a.hist != nullptr;
  Chunk<DT> ch;
  if (eager) load_chunk<DT>(a, row, c, ch);
  int pre[kHistPre];  // the row's first history ids, loaded beside the chunk
  if (a.hist) {
    const int* h = a.hist + (size_t)row * a.H;
#pragma unroll
    for (int k = 0; k < kHistPre; ++k) {
      const int i = (int)threadIdx.x + k * kThreads;
      pre[k] = i < a.H ? gld(h + i) : -1;
    }
  }
  const RowP p = row_params(a, row);
  const bool packed_row = DT == QS_DTYPE_BF16 && !p.pen && (p.kind == kKindGreedy || p.kind == kKindTopK);
  if (!lead && packed_row) return;  // served by the lead
  if (!eager) load_chunk<DT>(a, row, c, ch);
  RowSync* sy = &a.sync[row];
  Slot* sl = row_slots(a, row);
  if (p.pen) pen_build_pre(p, c, L, pre);
  QS_TR(1);
  (void)E;
  (void)J;
  (void)VL;

  u32 nch = 1;  // chunks served by this workgroup
  bool packed = false;
  if constexpr (DT == QS_DTYPE_BF16) {
    if (packed_row) {
      nch = (u32)min(kCPW, a.G - c);
      Chunk<QS_DTYPE_BF16> chx[kCPW];
      chx[0] = ch;
#pragma unroll
      for (int k = 1; k < kCPW; ++k) load_chunk<QS_DTYPE_BF16>(a, row, c + k, chx[k]);
      if (p.kind == kKindGreedy)
        greedy_pk<kCPW>(a, row, c, (int)nch, chx, L);
      else
        topk_pk<kCPW>(a, p, row, c, (int)nch, chx, L);
      packed = true;
    }
  }

  if (p.kind == kKindGreedy) {
    if (!packed) {
      u64 best = 0;
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
      if (p.pen) lds_sync();
      best = block_max64(best, L.s);
      if (threadIdx.x == 0) stc(&sl[c].a, best);
    }
    QS_TR(2);
    if (arrive_n(&sy->arrive, nch, L.s) != (u32)a.G - nch) return;
    QS_TR(3);
    finish_greedy(a, p, row, L);
    reset_row(a, row);
    QS_TR(4);
    return;
  }

  u32 why;
  if (p.kind == kKindTopK) {
    if (!packed) {
      const TkOut t = topk_row<DT>(a, p, row, c, ch, L);
      if (threadIdx.x == 0) topk_slot(a, p, row, c, t);
    }
    why = topk_last(a, p, row, c, L, nch, packed);
  } else if (p.kind == kKindSingle) {
    if (p.pen) lds_sync();
    why = arrive(&sy->arrive, L.s) == (u32)a.G - 1u ? kWhyLargeK : kNotLast;
  } else {
    why = mass_row<DT>(a, p, row, c, ch, L);
  }
  if (why == kNotLast) return;
  if (why != 0u) resolve_single<DT>(kernel_args(), row, why, L);
  reset_row(a, row);
}

// ---------------------------------------------------------------- post-filter probabilities

template <int DT>
__global__ __launch_bounds__(kThreads) void k_probs(Args a) {
  __shared__ Lds L;
  const int c = blockIdx.x;
  const int row = blockIdx.y;
  Chunk<DT> ch;
  load_chunk<DT>(a, row, c, ch);
  const RowP p = row_params(a, row);
  RowRes r;
  r.id = gld(&a.res[row].id);
  r.W = gld(&a.res[row].W);
  r.thr = gld(&a.res[row].thr);
  r.kstar = gld(&a.res[row].kstar);
  r.klo = gld(&a.res[row].klo);
  r.idlo = gld(&a.res[row].idlo);
  float* out = a.out_probs + (size_t)row * a.V;
  if (p.kind == kKindGreedy) {
#pragma unroll
    for (int j = 0; j < Chunk<DT>::J; ++j)
#pragma unroll
      for (int e = 0; e < Chunk<DT>::VL; ++e)
        if (ch.valid(j, e)) gst(out + ch.id(j, e), ch.id(j, e) == (int)r.id ? 1.0f : 0.0f);
    return;
  }
  if (p.pen) pen_build(p, c, L);
  u32 kq[kEPT];
  chunk_qkeys<DT>(ch, p, L, c, kq);
  const float qs = f_of_key(r.kstar);
  const double Wd = (double)r.W;
#pragma unroll
  for (int j = 0; j < Chunk<DT>::J; ++j)
#pragma unroll
    for (int e = 0; e < Chunk<DT>::VL; ++e) {
      if (!ch.valid(j, e)) continue;
      const int i = j * Chunk<DT>::VL + e;
      const int id = ch.id(j, e);
      u64 w = r.kstar ? weight_of(f_of_key(kq[i]), kq[i], qs, r.kstar, a.SH) : 0ull;
      w = w >= r.thr ? w : 0ull;
      const bool kept = kq[i] > r.klo || (kq[i] == r.klo && (u32)id <= r.idlo);
      gst(out + id, (kept && w && r.W) ? (float)((double)w / Wd) : 0.0f);
    }
}

__global__ void k_zero(u32* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) gst(p + i, 0u);
}

}  // namespace qs
