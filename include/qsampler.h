/*
 * qsampler -- decode-step token sampler for AMD MI355X (gfx950), C ABI.
 *
 * One shared library (qedge_amd/libqsampler.so).  Every pointer argument is a
 * device pointer owned by the caller, except where noted.  Calls are
 * asynchronous on `stream`, allocate nothing and never synchronise the host, so
 * a sequence of calls can be captured in a HIP graph.  Two calls may run at
 * once only on distinct workspaces.  Return value: 0 on success, negative on
 * an invalid argument or a HIP launch error; the message is then available
 * from qs_last_error().  No C++ exception crosses this ABI.
 *
 * Sampling contract (shared by the kernels and the CPU oracle; ids are exact):
 *  - z = fp32(logit), then the history penalties of tokens with count c > 0,
 *    one IEEE fp32 step each: z > 0 ? z / rep : z * rep; z - freq*c; z - pres.
 *  - greedy rows (temperature <= 1e-5): first index of max z, NaN is maximum.
 *  - sampling rows: q = z / T, one IEEE fp32 division (src/compute/sampler.py:32).
 *  - weights, anchored at the row maximum q*: d = fl(q - q*), y = fl(d * log2e),
 *    2^y from a fixed fp32 polynomial to a 24-bit mantissa and the octave
 *    floor(y), as a u64 in which q* weighs 2^(23+SH), SH = 40 - ceil(log2 V);
 *    0 for y < -64 and NaN.  All sums are exact u64 integers.
 *  - order: q descending, ties by ascending id.  top-k keeps q >= the k-th
 *    largest; min_p zeroes weights below min_p * (weight of q*); top-p keeps
 *    the prefix whose exclusive mass <= floor(top_p * S), S = mass of the
 *    top-k set (src/compute/sampler.py:35-37 evaluated exactly).
 *  - draw: t = floor(u * W) over the kept mass W; kept tokens in ascending id,
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
#define QS_FLAG_ALL_GREEDY 1u /* every row greedy: argmax of the penalised logits
                                 (src/compute/model_runner.py:82,84-85) */
#define QS_FLAG_USE_TOP_P 2u  /* apply top_p; without it top_p is ignored
                                 (src/compute/sampler.py:34,39-40) */
#define QS_FLAG_NO_WAIT 4u    /* test hook: the row barriers of top-k-off rows give
                                 up at once, so those rows take the exact
                                 single-workgroup path (results are identical) */

#define QS_FLAG_SOLO 8u       /* resolve every row by one workgroup streaming it (no
                                 workgroup cooperation): faster for batches of hundreds
                                 of rows with top-k off; rows with top-k on take extra
                                 passes.  Ignored where a row spans more than 128
                                 chunks of 8192 logits (V > 1048576).  Results are
                                 identical. */

#define QS_TOPK_FAST_MAX 1024 /* top_k up to this value is resolved from
                                 per-chunk candidates in one pass; larger
                                 top_k by the exact single-workgroup path */
#define QS_MAX_HISTORY 65535  /* longest token history per row (ids) */

/* Library version (major*10000 + minor*100 + patch). */
int qs_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* qs_last_error(void);

/*
 * Bytes of device workspace for batches of up to max_B rows of V logits
 * (logits_dtype and H do not change the size).  A workspace serves any call
 * with B <= max_B.  It is zeroed once by qs_workspace_init and every call
 * leaves it zeroed again.  Replaces the temporaries that BatchSampler.forward
 * allocates per call (src/compute/sampler.py:31-40) and the fixed-address
 * batch buffers of src/data/batch.py:57-66.
 */
size_t qs_workspace_bytes(int max_B, int V, int logits_dtype, int H);

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
 *  min_p         f32[B] or NULL; 0 disables   (src/data/batch.py:60,158,167)
 *  rep_pen, pres_pen, freq_pen  f32[B] or NULL (extension; 1/0/0 = off)
 *  hist_ids      i32[B, H] or NULL; ids outside [0, V) are padding
 *  hist_len      i32[B] or NULL: row r uses hist_ids[r, 0:hist_len[r]]
 *  uniforms      f32[B] in [0, 1): the host's seeded uniform per row
 *  row_order     i32[B] or NULL: a permutation of the rows giving the order in
 *                which their work is dispatched (rows with top-k off first is
 *                fastest); results do not depend on it
 *  out_ids       i64[B]
 *  out_probs     f32[B, V] or NULL: post-filter probabilities (verification)
 *  out_kept      i32[B] or NULL: kept tokens with nonzero weight
 */
int qs_sample(const void* logits, int64_t row_stride, int logits_dtype, int B, int V,
              const float* temperature, const float* top_p, const int32_t* top_k, const float* min_p,
              const float* rep_pen, const float* pres_pen, const float* freq_pen,
              const int32_t* hist_ids, int H, const int32_t* hist_len, const float* uniforms,
              const int32_t* row_order, uint32_t flags, int64_t* out_ids, float* out_probs,
              int32_t* out_kept, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * qs_sample without a workspace argument, for callers that cannot allocate
 * device memory (code under graph capture, fixed serving loops, harnesses that
 * forbid allocation).  It has no counterpart in the reference.  The scratch is
 * the library's own device array of qs_static_scratch_bytes() bytes (32 MiB)
 * on each GPU, held until the process ends; a batch whose workspace would not
 * fit in it is rejected with an error.  The first call on a device clears the
 * array with a fill kernel on `stream`; every call leaves it cleared.  Calls
 * that overlap on one GPU share the array and race: serialise them.
 * Allocates nothing (no hipMalloc, no library allocation).
 */
int qs_sample_static(const void* logits, int64_t row_stride, int logits_dtype, int B, int V,
                     const float* temperature, const float* top_p, const int32_t* top_k, const float* min_p,
                     const float* rep_pen, const float* pres_pen, const float* freq_pen,
                     const int32_t* hist_ids, int H, const int32_t* hist_len, const float* uniforms,
                     const int32_t* row_order, uint32_t flags, int64_t* out_ids, float* out_probs,
                     int32_t* out_kept, hipStream_t stream);
size_t qs_static_scratch_bytes(void);

/*
 * Greedy ids only: first index of the maximum logit per row, NaN is maximum.
 * Replaces logits.argmax(-1) on the all-greedy path and inside the captured
 * decode graph (src/compute/model_runner.py:85,353).
 */
int qs_argmax(const void* logits, int64_t row_stride, int logits_dtype, int B, int V,
              int64_t* out_ids, void* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Decode-step bookkeeping after qs_sample, on the device (no host round trip),
 * one thread per row.  Replaces the GPU staging of ModelRunner._publish_sample_ids
 * (src/compute/model_runner.py:95-115), the copy of _read_sample_ids
 * (src/compute/model_runner.py:122-135) and the stop check of
 * Scheduler.postprocess (src/control/scheduler.py:304-322):
 *
 *  ids            i64[B] sampled ids (qs_sample's out_ids)
 *  slots          i32[B] or NULL: row r's id goes to pending[slots[r]] (NULL: slot r;
 *                 slots outside [0, n_pending) are skipped)
 *  pending        i64[n_pending] or NULL: the fixed next-token slots (model_runner.py:35-37)
 *  num_generated  i32[B]: completion tokens so far, incremented for rows with max_tokens > 0
 *  min_tokens     i32[B] or NULL (0);  max_tokens  i32[B];  ignore_eos  u8[B] or NULL (0)
 *  eos_id         end-of-sequence id (< 0: none)
 *  finished       u8[B] or NULL, out: max_tokens <= 0, or after the increment
 *                 n >= max_tokens, or (!ignore_eos && n >= min_tokens && id == eos_id)
 *  host_ids       i64[B] or NULL: the device address of a host-mapped pinned
 *                 buffer that receives the ids (the CPU mirror)
 */
int qs_step_finish(const int64_t* ids, int B, const int32_t* slots, int64_t* pending, int n_pending,
                   int32_t* num_generated, const int32_t* min_tokens, const int32_t* max_tokens,
                   const uint8_t* ignore_eos, int64_t eos_id, uint8_t* finished, int64_t* host_ids,
                   hipStream_t stream);

/*
 * Appends the sampled ids to the device-resident token history that qs_sample
 * reads (hist_ids [B, H], hist_len [B]): hist_ids[r, hist_len[r] % H] = ids[r],
 * hist_len[r] += 1, for rows with active[r] != 0 (active may be NULL: every
 * row).  The history is a ring of the last H ids; qs_sample uses the last
 * min(hist_len, H) of them.  Replaces Sequence.append_token's history
 * (src/data/sequence.py:177-179) for the penalties, so the ids are not
 * re-staged from the host each step.
 */
int qs_history_append(int32_t* hist_ids, int B, int H, int32_t* hist_len, const int64_t* ids,
                      const uint8_t* active, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QSAMPLER_H */
