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
 * The reference has no penalties, no top-k and no seeded draw; the extensions
 * below (penalties, top-k, inverse-CDF draw on a host uniform) follow the
 * semantics stated in the rules E1-E4 of this file, and the parameter staging
 * rules follow src/data/batch.py:149-175.
 *
 * The exact-integer contract (rules), identical in the HIP kernels:
 *  R0  z_i = fp32(x_i).  Penalties (E1), only for tokens with history count c>0,
 *      each step one IEEE fp32 operation:  z = z>0 ? z/rep : z*rep;
 *      z = z - freq*(float)c;  z = z - pres.
 *  R1  greedy row iff T <= 1e-5f: id = first index of max z (NaN is maximum).
 *  R2  q_i = z_i / T, one IEEE fp32 division (sampler.py:32).  Order key:
 *      k_i = orderable bits of q_i (NaN -> lowest, -0 -> +0); rows are ordered
 *      by (k desc, id asc) -- the order torch.sort gives on the probabilities
 *      (sampler.py:35), ties taken in ascending id.
 *  R3  weights ("exp(q)" to 24 bits, free of any anchor):
 *        y_i = clamp((double)q_i * LOG2E, -2^30, 2^30)  (NaN -> -2^30)
 *        n_i = floor(y_i), f_i = y_i - n_i,  P = poly((float)f_i) ~ 2^f in [1,2)
 *        M_i = 24-bit mantissa of P;  exp(q_i) ~= M_i * 2^(n_i-23)
 *      Row scale N = max n_i; window: w_i = M_i << (n_i - N + 40) if
 *      n_i >= N-40 else 0 (u64, exact).  p_i = w_i / sum(w).
 *  R4  top-k (E2): if 0 < k < V, kappa = key at rank k-1; keep k_i >= kappa
 *      (top-k after temperature, ties at the k-th value kept).
 *  R5  top-p (sampler.py:35-37 restated exactly): S = sum of w over the top-k
 *      set; Tp = floor(top_p * S) (exact 128-bit); walking the top-k set in
 *      order, keep a token iff its exclusive prefix mass <= Tp.  top_p >= 1
 *      keeps the whole set.
 *  R6  draw (E3): W = sum of kept w; t = floor(u * W); walking kept tokens in
 *      ascending id, return the first whose inclusive prefix mass > t.
 *      u is clamped to [0, 1).
 *  R7  post-filter probabilities (E4): p'_i = (float)(w_i / W) in double for
 *      kept tokens, 0 elsewhere; the kept count counts kept tokens with w>0.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

#define QS_WINDOW 40
#define QS_YCLAMP 1073741824.0 /* 2^30 */

/* 2^f on [0,1]: degree-6 Horner in fp32 with fused multiply-add; c0 = 1. */
static const float QS_P2[7] = {
    1.0f, 0x1.62e42cp-1f, 0x1.ebfd5ap-3f, 0x1.c688f0p-5f,
    0x1.3d0c40p-7f, 0x1.46d326p-10f, 0x1.c54640p-13f};

static const double QS_LOG2E = 1.4426950408889634074;

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

static inline double y_of(float q) {
  if (q != q) return -QS_YCLAMP;
  double y = (double)q * QS_LOG2E;
  if (!(y >= -QS_YCLAMP)) y = -QS_YCLAMP;
  if (y > QS_YCLAMP) y = QS_YCLAMP;
  return y;
}

/* (n, M) such that exp(q) ~= M * 2^(n-23). */
void qso_detexp(const float* q, int count, int32_t* n_out, uint32_t* m_out) {
  for (int i = 0; i < count; ++i) {
    double y = y_of(q[i]);
    double fl = floor(y);
    double f = y - fl;
    n_out[i] = (int32_t)fl;
    m_out[i] = mant24(qso_exp2_poly((float)f));
  }
}

/* floor(x * f) for f in [0, 1] given as an fp32 value, x < 2^104. */
static inline u128 mul_frac(u128 x, float f) {
  if (!(f > 0.0f)) return 0;
  uint32_t b = f2u(f);
  uint32_t e = (b >> 23) & 0xffu;
  uint32_t m = b & 0x7fffffu;
  int shift;
  if (e == 0) { shift = 149; } else { m |= 0x800000u; shift = 150 - (int)e; }
  if (shift >= 128) return 0;
  u128 prod = x * (u128)m;
  return prod >> shift;
}

double qso_u128_to_double(uint64_t lo, uint64_t hi) {
  double d = (double)(uint32_t)(hi >> 32) * 0x1p96;
  d = d + (double)(uint32_t)hi * 0x1p64;
  d = d + (double)(uint32_t)(lo >> 32) * 0x1p32;
  d = d + (double)(uint32_t)lo;
  return d;
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

typedef struct {
  int32_t greedy_id;   /* argmax id (R1), always computed */
  int32_t n_max;       /* N */
  int32_t kept;        /* kept tokens with w > 0 */
  int32_t topk_end;    /* size of the top-k set */
  uint64_t w_lo, w_hi; /* W */
} qso_row_info;

/*
 * One row. Scratch buffers are owned by the caller (V entries each).
 * Returns the sampled id.
 */
static int64_t sample_row(const void* row, int dtype, int V, float T, float top_p, int top_k,
                          float rep, float pres, float freq, const int32_t* hist, int H, float u,
                          float* z, uint64_t* comp, uint64_t* w, int32_t* cnt, uint8_t* kept,
                          float* probs, qso_row_info* info) {
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
  info->kept = 0; info->topk_end = 0; info->w_lo = info->w_hi = 0; info->n_max = 0;
  if (T <= 1e-5f) {
    if (probs) for (int i = 0; i < V; ++i) probs[i] = (i == arg) ? 1.0f : 0.0f;
    info->kept = 1;
    return arg;
  }
  /* R2: q = z / T in place */
  for (int i = 0; i < V; ++i) z[i] = z[i] / T;
  /* R3 weights */
  int32_t N = INT32_MIN;
  for (int i = 0; i < V; ++i) {
    double y = y_of(z[i]);
    int32_t n = (int32_t)floor(y);
    if (n > N) N = n;
  }
  info->n_max = N;
  for (int i = 0; i < V; ++i) {
    double y = y_of(z[i]);
    double fl = floor(y);
    int32_t n = (int32_t)fl;
    if (n >= N - QS_WINDOW) {
      uint32_t m = mant24(qso_exp2_poly((float)(y - fl)));
      w[i] = (uint64_t)m << (n - N + QS_WINDOW);
    } else {
      w[i] = 0;
    }
    comp[i] = ((uint64_t)qso_key(z[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
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
  info->topk_end = kend;
  u128 S = 0;
  for (int p = 0; p < kend; ++p) S += w[0xffffffffu - (uint32_t)comp[p]];
  /* R5 top-p */
  int pend = kend;
  if (top_p < 1.0f) {
    u128 Tp = mul_frac(S, top_p);
    u128 excl = 0;
    pend = 0;
    while (pend < kend && excl <= Tp) {
      excl += w[0xffffffffu - (uint32_t)comp[pend]];
      pend++;
    }
  }
  memset(kept, 0, (size_t)V);
  u128 W = 0;
  int nk = 0;
  for (int p = 0; p < pend; ++p) {
    uint32_t id = 0xffffffffu - (uint32_t)comp[p];
    kept[id] = 1;
    W += w[id];
    if (w[id]) nk++;
  }
  info->kept = nk;
  info->w_lo = (uint64_t)W;
  info->w_hi = (uint64_t)(W >> 64);
  /* R6 draw */
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = u2f(0x3f7fffffu);
  u128 t = mul_frac(W, u);
  int64_t pick = -1;
  u128 acc = 0;
  for (int i = 0; i < V; ++i) {
    if (!kept[i]) continue;
    acc += w[i];
    if (acc > t) { pick = i; break; }
  }
  if (pick < 0) pick = arg; /* unreachable: W > 0 always (the top token has n = N) */
  if (probs) {
    double Wd = qso_u128_to_double((uint64_t)W, (uint64_t)(W >> 64));
    for (int i = 0; i < V; ++i)
      probs[i] = kept[i] ? (float)((double)w[i] / Wd) : 0.0f;
  }
  return pick;
}

/*
 * Batched oracle. logits: [B, row_stride] of fp32 (dtype 0) or bf16 bits (1).
 * Any of top_p/top_k/rep/pres/freq/hist/u may be NULL (feature off).
 * hist: [B, H] int32 ids, entries outside [0, V) are padding.
 * out_probs: NULL or [B, V] fp32.  out_info: NULL or [B] rows of 8 int32.
 */
int qso_sample(const void* logits, int dtype, int64_t row_stride, int B, int V, const float* T,
               const float* top_p, const int32_t* top_k, const float* rep, const float* pres,
               const float* freq, const int32_t* hist, int H, const float* u, int64_t* out_ids,
               float* out_probs, int32_t* out_info, int nthreads) {
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
        out_ids[r] = sample_row(row, dtype, V, T[r], top_p ? top_p[r] : 1.0f,
                                top_k ? top_k[r] : 0, rp, pp, fp,
                                hist ? hist + (size_t)r * (size_t)H : NULL, hist ? H : 0,
                                u ? u[r] : 0.0f, z, comp, w, cnt, kept,
                                out_probs ? out_probs + (size_t)r * (size_t)V : NULL, &info);
        if (out_info) {
          int32_t* o = out_info + (size_t)r * 8;
          o[0] = info.greedy_id; o[1] = info.n_max; o[2] = info.kept; o[3] = info.topk_end;
          o[4] = (int32_t)(uint32_t)info.w_lo; o[5] = (int32_t)(uint32_t)(info.w_lo >> 32);
          o[6] = (int32_t)(uint32_t)info.w_hi; o[7] = (int32_t)(uint32_t)(info.w_hi >> 32);
        }
      }
    }
    free(z); free(comp); free(w); free(cnt); free(kept);
  }
  return status;
}

/* One row after penalties and temperature (R0, R2, R3): per token z, q, key(q), n, M. */
void qso_row_weights(const void* row, int dtype, int V, float T, const int32_t* hist, int H,
                     float rep, float pres, float freq, int32_t* n_out, uint32_t* m_out,
                     uint32_t* key_out, float* z_out, float* q_out) {
  int32_t* cnt = (int32_t*)calloc((size_t)V, sizeof(int32_t));
  int has_pen = 0;
  if (hist) for (int h = 0; h < H; ++h) if (hist[h] >= 0 && hist[h] < V) { cnt[hist[h]]++; has_pen = 1; }
  for (int i = 0; i < V; ++i) {
    float v = load_logit(row, dtype, i);
    if (has_pen) v = apply_penalty(v, cnt[i], rep, pres, freq);
    z_out[i] = v;
    float q = v / T;
    q_out[i] = q;
    key_out[i] = qso_key(q);
    double y = y_of(q);
    double fl = floor(y);
    n_out[i] = (int32_t)fl;
    m_out[i] = mant24(qso_exp2_poly((float)(y - fl)));
  }
  free(cnt);
}
