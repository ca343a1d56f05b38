/*
 * qsampler -- decode-step token sampler for AMD MI355X (gfx950), C ABI.
 *
 * One shared library (qedge_amd/libqsampler.so).  Every pointer argument is a
 * device pointer owned by the caller, except where noted.  Calls are
 * asynchronous on `stream`, allocate nothing and never synchronise the host, so
 * a sequence of calls can be captured in a HIP graph.  Return value: 0 on
 * success, negative on an invalid argument or a HIP launch error; the message
 * is then available from qs_last_error().  No C++ exception crosses this ABI.
 *
 * Sampling contract (shared by the kernels and the CPU oracle; ids are exact):
 *  - z = fp32(logit), then the history penalties below, one IEEE fp32 step each.
 *  - greedy rows (temperature <= 1e-5): first index of max z, NaN is maximum.
 *  - sampling rows: q = z / T, one IEEE fp32 division (src/compute/sampler.py:32).
 *  - weights: exp(q) evaluated to a 24-bit mantissa M and exponent n
 *    (y = q*log2(e) in double, n = floor(y), M from a fixed fp32
 *    polynomial of y-n), scaled to a u64 relative to the row's largest n with
 *    a 40-octave window.
 *  - order: q descending, ties by ascending id.  top-k keeps q >= the k-th
 *    largest; top-p keeps the prefix whose exclusive mass <= floor(top_p*S)
 *    (exact 128-bit integers), S = mass of the top-k set.
 *  - draw: t = floor(u*W) over the kept mass W; kept tokens in ascending id,
 *    the first whose inclusive mass exceeds t.
 */
#ifndef QSAMPLER_H
#define QSAMPLER_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QS_DTYPE_F32 0
#define QS_DTYPE_BF16 1

/* flags for qs_sample */
#define QS_FLAG_ALL_GREEDY 1u /* every row greedy: argmax only
                                 (src/compute/model_runner.py:82,84-85) */
#define QS_FLAG_USE_TOP_P 2u  /* apply top_p; without it top_p is ignored
                                 (src/compute/sampler.py:34,39-40) */
#define QS_FLAG_NO_MASS_ROWS 4u /* host hint from the CPU-side parameters: every
                                   sampling row has 0 < top_k <= QS_TOPK_FAST_MAX
                                   (same kind of batch flag as use_top_p,
                                   src/compute/model_runner.py:82-83); skips the
                                   code that serves top-k-off rows (batches above
                                   64 rows: their launch).  If such a row is
                                   present anyway it is still resolved exactly,
                                   by a slower path. */

#define QS_TOPK_FAST_MAX 1024 /* top_k up to this value is resolved from
                                 per-chunk candidates in one pass */
#define QS_MAX_HISTORY 8192   /* longest token history per row (ids); the
                                 reference's max_model_len is 8192
                                 (src/config.py:49) */

/* Library version (major*10000 + minor*100 + patch). */
int qs_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* qs_last_error(void);

/*
 * Bytes of device workspace qs_sample/qs_argmax need for B rows of V logits
 * with H history ids per row (H = 0 without penalties).  The workspace is
 * zeroed once by qs_workspace_init and every call leaves it zeroed again.
 * Replaces the temporaries that BatchSampler.forward allocates per call
 * (src/compute/sampler.py:31-40).
 */
size_t qs_workspace_bytes(int B, int V, int logits_dtype, int H);

/* Zero a workspace (a fill kernel on `stream`, no memset node). */
int qs_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Sample one token per row.  Replaces BatchSampler.forward
 * (src/compute/sampler.py:25-41) as called by ModelRunner._sample_gpu
 * (src/compute/model_runner.py:77-93).
 *
 *  logits        [B, row_stride] fp32 or bf16 (row_stride >= V, in elements)
 *  temperature   f32[B]                       (src/data/batch.py:57,164)
 *  top_p         f32[B] or NULL               (src/data/batch.py:58,165)
 *  top_k         i32[B] or NULL; <= 0 or >= V disables (src/data/batch.py:154-157)
 *  rep_pen, pres_pen, freq_pen  f32[B] or NULL (extension; 1/0/0 = off)
 *  hist_ids      i32[B, H] or NULL; ids outside [0, V) are padding
 *  uniforms      f32[B] in [0, 1): the host's seeded uniform per row
 *  out_ids       i64[B]
 *  out_probs     f32[B, V] or NULL: post-filter probabilities (verification)
 *  out_kept      i32[B] or NULL: kept tokens with nonzero weight (needs out_probs)
 */
int qs_sample(const void* logits, int64_t row_stride, int logits_dtype, int B, int V,
              const float* temperature, const float* top_p, const int32_t* top_k,
              const float* rep_pen, const float* pres_pen, const float* freq_pen,
              const int32_t* hist_ids, int H, const float* uniforms, uint32_t flags,
              int64_t* out_ids, float* out_probs, int32_t* out_kept, void* workspace,
              size_t workspace_bytes, hipStream_t stream);

/*
 * Greedy ids only: first index of the maximum logit per row, NaN is maximum.
 * Replaces logits.argmax(-1) on the all-greedy path and inside the captured
 * decode graph (src/compute/model_runner.py:85,353).
 */
int qs_argmax(const void* logits, int64_t row_stride, int logits_dtype, int B, int V,
              int64_t* out_ids, void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QSAMPLER_H */
