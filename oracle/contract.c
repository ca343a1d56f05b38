/*
 * CPU oracle for the decode-step sampler -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this file's library, and only to check results or as the timed CPU baseline. The
 * product path (qedge_amd/) never calls it.
 *
 * What it restates. The reference sampler is BatchSampler.forward
 * (src/compute/sampler.py:25-41) behind ModelRunner._sample_gpu
 * (src/compute/model_runner.py:77-93):
 *   greedy rows (T <= 1e-5, sampler.py:30) take argmax of the logits
 *   (sampler.py:29,41: first index of the maximum, NaN counts as maximum);
 *   other rows take softmax(fp32(x) / T) (sampler.py:32), sort it descending
 *   (sampler.py:35), drop tokens whose exclusive prefix mass exceeds top_p
 *   (sampler.py:36-37) and draw one token (sampler.py:38,40).
 * The reference has no penalties, no top-k, no min_p filter and no seeded
 * draw; the extensions below follow the rules E1-E5 of this file, and the
 * parameter staging follows src/data/batch.py:149-175.
 *
 * The exact-integer contract, identical in the HIP kernels:
 *  R0  z_i = fp32(x_i).  Penalties (E1), only for tokens with history count
 *      c > 0, each step one IEEE fp32 operation:  z = z > 0 ? z / rep : z * rep;
 *      z = z - freq * (float)c;  z = z - pres.
 *  R1  greedy row iff T <= 1e-5f: id = first index of max z (NaN is maximum).
 *  R2  q_i = z_i / T, one IEEE fp32 division (sampler.py:32).  Order key:
 *      k_i = orderable bits of q_i (NaN -> 0, the lowest; -0 -> +0); a row is
 *      ordered by (k desc, id asc) -- the order torch.sort gives on the
 *      probabilities (sampler.py:35), ties taken in ascending id.
 *  R3  weights, anchored at the row maximum q* (the q of the largest key; a
 *      row whose every q is NaN has no weights):
 *        d_i = (k_i == k*) ? 0 : fl(q_i - q*)
 *        y_i = fl(d_i * L),  L = fp32(log2 e)
 *        w_i = 0 if q_i is NaN or !(y_i >= -64); otherwise
 *        n_i = floor(y_i), f_i = fl(y_i - n_i), P_i = poly(f_i) (fp32 FMA
 *        Horner of QS_P2), M_i = 24-bit mantissa of P_i clamped to [1, 2),
 *        s_i = n_i + SH:  w_i = s_i >= 0 ? M_i << s_i : M_i >> -s_i  (u64),
 *      with SH = 40 - ceil(log2 V), so that the largest weight, that of q*
 *      itself, is 2^(23+SH) and V weights sum to at most 2^63.
 *  R4  top-k (E2): if 0 < k < V, kappa = key at rank k-1 and the set K keeps
 *      k_i >= kappa (ties at the k-th value kept); otherwise K is the row.
 *  R5  min_p (E3): if min_p > 0, tokens with w_i < min_p * 2^(23+SH) (that is,
 *      p_i < min_p * p_max) have their weight replaced by 0.
 *  R6  top-p (sampler.py:35-37 restated exactly): S = sum of w over K;
 *      Tp = floor(top_p * S) (exact); walking K in order, keep a token iff its
 *      exclusive prefix mass <= Tp.  top_p >= 1 keeps the whole of K.
 *  R7  draw (E4): W = sum of kept w; t = floor(u * W), u clamped to
 *      [0, 1 - 2^-24]; walking kept tokens in ascending id, return the first
 *      whose inclusive prefix mass exceeds t.  W = 0 (a row of NaN) returns
 *      the R1 id.
 *  R8  post-filter probabilities (E5): p'_i = (float)((double)w_i / (double)W)
 *      for kept tokens, 0 elsewhere; the kept count counts kept tokens with
 *      w > 0.  A greedy row has p' = 1 at its id.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

#define QS_YMIN 64.0f

/* 2^f on [0, 1]: degree-6 Horner in fp32 with fused multiply-add; c0 = 1.
 * Derived by oracle/fit_exp2.py (iteratively reweighted least squares toward
 * the minimax relative error on Chebyshev nodes, rounded to fp32). */
static const float QS_P2[7] = {
    1.0f, 0x1.62e42cp-1f, 0x1.ebfd58p-3f, 0x1.c68912p-5f,
    0x1.3d0b92p-7f, 0x1.46d64cp-10f, 0x1.c5417ap-13f};

static const float QS_L2E = 0x1.715476p+0f; /* fp32(log2 e) */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float qso_exp2_poly(float f) {
  float p = QS_P2[6];
  p = fmaf(p, f, QS_P2[5]);
  p = fmaf(p, f, QS_P2[4]);
  p = fmaf(p, f, QS_P2[3]);
  p = fmaf(p, f, QS_P2[2]);
  p = fmaf(p, f, QS_P2[1]);
  p = fmaf(p, f, QS_P2[0]);
  return p;
}

static inline uint32_t mant24(float p) {
  if (!(p >= 1.0f)) p = 1.0f;
  if (p >= 2.0f) p = u2f(0x3fffffffu);
  return 0x800000u | (f2u(p) & 0x7fffffu);
}

uint32_t qso_key(float z) {
  if (z != z) return 0u;
  if (z == 0.0f) z = 0.0f;
  uint32_t u = f2u(z);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

float qso_z_of_key(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return u2f(u);
}

int qso_shift(int V) {
  int b = 0;
  while (b < 40 && ((int64_t)1 << b) < (int64_t)V) b++;
  return 40 - b;
}

/* R3: the weight of q given the row maximum q* (and its key). */
uint64_t qso_weight(float q, float qs, uint32_t ks, int SH) {
  if (q != q) return 0;
  float d = (qso_key(q) == ks) ? 0.0f : q - qs;
  float y = d * QS_L2E;
  if (!(y >= -QS_YMIN)) return 0;
  float fl = floorf(y);
  int n = (int)fl;
  float f = y - fl;
  uint64_t m = mant24(qso_exp2_poly(f));
  int s = n + SH;
  return s >= 0 ? m << s : m >> (-s);
}

/* floor(x * f) for f in [0, 1] given as an fp32 value, x < 2^64. */
static inline uint64_t mul_frac(uint64_t x, float f) {
  if (!(f > 0.0f)) return 0;
  uint32_t b = f2u(f);
  uint32_t e = (b >> 23) & 0xffu;
  uint32_t m = b & 0x7fffffu;
  int shift;
  if (e == 0) { shift = 149; } else { m |= 0x800000u; shift = 150 - (int)e; }
  if (shift >= 128) return 0;
  u128 prod = (u128)x * (u128)m;
  return (uint64_t)(prod >> shift);
}

/* ceil(f * 2^e) for f in [0, 1] as fp32 and e >= 0. */
uint64_t qso_ceil_scaled(float f, int e) {
  if (!(f > 0.0f)) return 0;
  uint32_t b = f2u(f);
  uint32_t ex = (b >> 23) & 0xffu;
  uint64_t m = b & 0x7fffffu;
  int sh; /* f = m * 2^-sh */
  if (ex == 0) { sh = 149; } else { m |= 0x800000u; sh = 150 - (int)ex; }
  sh -= e; /* f * 2^e = m * 2^-sh */
  if (sh <= 0) return m << (-sh);
  if (sh >= 64) return 1;
  uint64_t q = m >> sh;
  return q + ((m & (((uint64_t)1 << sh) - 1)) != 0);
}

static inline float load_logit(const void* base, int dtype, int64_t off) {
  if (dtype == 0) return ((const float*)base)[off];
  uint16_t h = ((const uint16_t*)base)[off];
  return u2f((uint32_t)h << 16);
}

static int cmp_desc_u64(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return (x < y) - (x > y);
}

/* Penalty application for one token with history count c (rule R0). */
static inline float apply_penalty(float z, int c, float rep, float pres, float freq) {
  if (c <= 0) return z;
  z = (z > 0.0f) ? (z / rep) : (z * rep);
  z = z - freq * (float)c;
  z = z - pres;
  return z;
}

/* Per-row record: what the tests compare beside the id. */
typedef struct {
  int32_t greedy_id;  /* R1 id, always computed */
  int32_t kept;       /* kept tokens with w > 0 */
  int32_t kend;       /* size of K */
  int32_t pend;       /* kept tokens (prefix of K in order) */
  uint32_t kstar;     /* key of q* (0: no weights) */
  uint32_t kappa;     /* key of the last kept token */
  uint32_t w_lo, w_hi; /* W */
  uint32_t s_lo, s_hi; /* S */
  uint32_t pad[6];
} qso_row_info;

/*
 * One row. Scratch buffers are owned by the caller (V entries each).
 * Returns the sampled id.
 */
static int64_t sample_row(const void* row, int dtype, int V, float T, float top_p, int top_k,
                          float min_p, float rep, float pres, float freq, const int32_t* hist, int H,
                          float u, float* z, uint64_t* comp, uint64_t* w, int32_t* cnt, uint8_t* kept,
                          float* probs, qso_row_info* info) {
  memset(info, 0, sizeof(*info));
  int has_pen = 0;
  if (hist && H > 0) {
    memset(cnt, 0, sizeof(int32_t) * (size_t)V);
    for (int h = 0; h < H; ++h) {
      int32_t id = hist[h];
      if (id >= 0 && id < V) { cnt[id]++; has_pen = 1; }
    }
  }
  for (int i = 0; i < V; ++i) {
    float v = load_logit(row, dtype, i);
    if (has_pen) v = apply_penalty(v, cnt[i], rep, pres, freq);
    z[i] = v;
  }
  /* R1: first index of the maximum; NaN counts as the maximum. */
  int arg = 0;
  {
    float best = z[0];
    int best_nan = (best != best);
    for (int i = 1; i < V && !best_nan; ++i) {
      float v = z[i];
      if (v != v) { arg = i; best_nan = 1; break; }
      if (v > best) { best = v; arg = i; }
    }
  }
  info->greedy_id = arg;
  if (T <= 1e-5f) {
    if (probs) for (int i = 0; i < V; ++i) probs[i] = (i == arg) ? 1.0f : 0.0f;
    info->kept = 1; info->kend = V; info->pend = 1;
    return arg;
  }
  /* R2: q = z / T in place; R3: q* */
  uint32_t ks = 0;
  for (int i = 0; i < V; ++i) {
    z[i] = z[i] / T;
    uint32_t k = qso_key(z[i]);
    if (k > ks) ks = k;
  }
  info->kstar = ks;
  const int SH = qso_shift(V);
  const float qs = qso_z_of_key(ks);
  for (int i = 0; i < V; ++i) {
    uint32_t k = qso_key(z[i]);
    w[i] = ks ? qso_weight(z[i], qs, ks, SH) : 0;
    comp[i] = ((uint64_t)k << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  }
  /* R2: (key desc, id asc) */
  qsort(comp, (size_t)V, sizeof(uint64_t), cmp_desc_u64);
  /* R4 top-k */
  int kend = V;
  if (top_k > 0 && top_k < V) {
    uint32_t kappa = (uint32_t)(comp[top_k - 1] >> 32);
    kend = top_k;
    while (kend < V && (uint32_t)(comp[kend] >> 32) == kappa) kend++;
  }
  info->kend = kend;
  /* R5 min_p */
  if (min_p > 0.0f) {
    uint64_t thr = qso_ceil_scaled(min_p, 23 + SH);
    for (int i = 0; i < V; ++i)
      if (w[i] < thr) w[i] = 0;
  }
  uint64_t S = 0;
  for (int p = 0; p < kend; ++p) S += w[0xffffffffu - (uint32_t)comp[p]];
  /* R6 top-p */
  int pend = kend;
  if (top_p < 1.0f) {
    uint64_t Tp = mul_frac(S, top_p);
    uint64_t excl = 0;
    pend = 0;
    while (pend < kend && excl <= Tp) {
      excl += w[0xffffffffu - (uint32_t)comp[pend]];
      pend++;
    }
  }
  memset(kept, 0, (size_t)V);
  uint64_t W = 0;
  int nk = 0;
  for (int p = 0; p < pend; ++p) {
    uint32_t id = 0xffffffffu - (uint32_t)comp[p];
    kept[id] = 1;
    W += w[id];
    if (w[id]) nk++;
  }
  info->kept = nk;
  info->pend = pend;
  info->kappa = pend > 0 ? (uint32_t)(comp[pend - 1] >> 32) : 0;
  info->w_lo = (uint32_t)W; info->w_hi = (uint32_t)(W >> 32);
  info->s_lo = (uint32_t)S; info->s_hi = (uint32_t)(S >> 32);
  /* R7 draw */
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = u2f(0x3f7fffffu);
  if (W == 0) {
    if (probs) for (int i = 0; i < V; ++i) probs[i] = 0.0f;
    info->kept = 0;
    return arg;
  }
  uint64_t t = mul_frac(W, u);
  int64_t pick = arg;
  uint64_t acc = 0;
  for (int i = 0; i < V; ++i) {
    if (!kept[i]) continue;
    acc += w[i];
    if (acc > t) { pick = i; break; }
  }
  if (probs) {
    double Wd = (double)W;
    for (int i = 0; i < V; ++i)
      probs[i] = kept[i] ? (float)((double)w[i] / Wd) : 0.0f;
  }
  return pick;
}

/*
 * Batched oracle. logits: [B, row_stride] of fp32 (dtype 0) or bf16 bits (1).
 * Any of top_p/top_k/min_p/rep/pres/freq/hist/u may be NULL (feature off).
 * hist: [B, H] int32 ids, entries outside [0, V) are padding.
 * out_probs: NULL or [B, V] fp32.  out_info: NULL or [B] records of 16 u32.
 */
int qso_sample(const void* logits, int dtype, int64_t row_stride, int B, int V, const float* T,
               const float* top_p, const int32_t* top_k, const float* min_p, const float* rep,
               const float* pres, const float* freq, const int32_t* hist, int H, const float* u,
               int64_t* out_ids, float* out_probs, uint32_t* out_info, int nthreads) {
  if (B < 0 || V <= 0 || !logits || !T || !out_ids) return -1;
  int status = 0;
  (void)nthreads;
#pragma omp parallel num_threads(nthreads > 0 ? nthreads : 1)
  {
    float* z = (float*)malloc(sizeof(float) * (size_t)V);
    uint64_t* comp = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
    uint64_t* w = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
    int32_t* cnt = (int32_t*)malloc(sizeof(int32_t) * (size_t)V);
    uint8_t* kept = (uint8_t*)malloc((size_t)V);
    if (!z || !comp || !w || !cnt || !kept) {
#pragma omp atomic write
      status = -2;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int r = 0; r < B; ++r) {
        const char* row = (const char*)logits + (size_t)r * (size_t)row_stride * (dtype ? 2 : 4);
        qso_row_info info;
        float rp = rep ? rep[r] : 1.0f, pp = pres ? pres[r] : 0.0f, fp = freq ? freq[r] : 0.0f;
        out_ids[r] = sample_row(row, dtype, V, T[r], top_p ? top_p[r] : 1.0f, top_k ? top_k[r] : 0,
                                min_p ? min_p[r] : 0.0f, rp, pp, fp,
                                hist ? hist + (size_t)r * (size_t)H : NULL, hist ? H : 0,
                                u ? u[r] : 0.0f, z, comp, w, cnt, kept,
                                out_probs ? out_probs + (size_t)r * (size_t)V : NULL, &info);
        if (out_info) memcpy(out_info + (size_t)r * 16, &info, sizeof(info));
      }
    }
    free(z); free(comp); free(w); free(cnt); free(kept);
  }
  return status;
}

/* One row after penalties and temperature (R0, R2, R3): per token z, q, key(q), w. */
void qso_row_weights(const void* row, int dtype, int V, float T, const int32_t* hist, int H,
                     float rep, float pres, float freq, uint32_t* key_out, float* z_out,
                     float* q_out, uint64_t* w_out) {
  int32_t* cnt = (int32_t*)calloc((size_t)V, sizeof(int32_t));
  int has_pen = 0;
  if (hist) for (int h = 0; h < H; ++h) if (hist[h] >= 0 && hist[h] < V) { cnt[hist[h]]++; has_pen = 1; }
  uint32_t ks = 0;
  for (int i = 0; i < V; ++i) {
    float v = load_logit(row, dtype, i);
    if (has_pen) v = apply_penalty(v, cnt[i], rep, pres, freq);
    z_out[i] = v;
    float q = v / T;
    q_out[i] = q;
    key_out[i] = qso_key(q);
    if (key_out[i] > ks) ks = key_out[i];
  }
  const int SH = qso_shift(V);
  const float qs = qso_z_of_key(ks);
  for (int i = 0; i < V; ++i) w_out[i] = ks ? qso_weight(q_out[i], qs, ks, SH) : 0;
  free(cnt);
}
