// qsampler: decode-step token sampler for MI355X (gfx950), C ABI.
//
// Replaces BatchSampler.forward (src/compute/sampler.py:25-41) behind the
// ModelRunner._sample_gpu call site (src/compute/model_runner.py:77-93) and the
// greedy argmax sites (src/compute/model_runner.py:85,353).  The arithmetic
// contract is stated in include/qsampler.h; ids are exact integers.  One call
// is one launch of k_sample (plus k_probs when the probabilities are asked
// for); the kernels are in qs_kernels.hpp.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "qs_kernels.hpp"
#include "qs_solo.hpp"
#include "qs_step.hpp"
#include "qsampler.h"

namespace {

using namespace qs;

thread_local char g_err[512] = "";
#ifdef QS_TRACE
void* g_trace = nullptr;
#endif

int fail(const char* fmt, long long v = 0) {
  snprintf(g_err, sizeof(g_err), fmt, v);
  return -1;
}

struct Layout {
  int G, R, SH;
  long long dpr;  // u64 entries of per-row data
  size_t off_sync, off_res, off_slots, off_data, per_row, total;
};

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

int shift_of(int V) {
  int b = 0;
  while (b < 40 && (1ll << b) < (long long)V) ++b;
  return 40 - b;
}

bool layout_for(int B, int V, Layout* L) {
  if (V <= 0) return false;
  L->G = (V + kCH - 1) / kCH;
  if (L->G > kMaxG) return false;
  L->R = kRegionTotal / L->G;
  if (L->R > kRegionCap) L->R = kRegionCap;
  L->SH = shift_of(V);
  const long long cand = (long long)L->G * L->R;
  const long long mass = (long long)kRounds * kNB + (long long)L->G * (kLC + kSegMax);
  L->dpr = cand > mass ? cand : mass;
  // one row's block: counters, result, slots, data
  L->off_sync = 0;
  L->off_res = L->off_sync + sizeof(RowSync);
  L->off_slots = 0;
  L->per_row = 0;
  const size_t nB = (size_t)(B > 0 ? B : 1);
  size_t off = 0;
  L->off_sync = off;
  off = align_up(off + nB * sizeof(RowSync), 256);
  L->off_res = off;
  off = align_up(off + nB * sizeof(RowRes), 256);
  L->off_slots = off;
  off = align_up(off + nB * kMaxG * sizeof(Slot), 256);
  L->off_data = off;
  off = align_up(off + nB * (size_t)L->dpr * sizeof(u64), 256);
  L->total = off;
  return true;
}

// Workspaces are sized for a maximum batch; a call with fewer rows uses the
// first rows of every region, so the offsets are those of the maximum batch.
// The maximum is recovered from the workspace size.
int max_rows_of(size_t bytes, int V) {
  Layout L1;
  if (!layout_for(1, V, &L1)) return 0;
  const size_t per = sizeof(RowSync) + sizeof(RowRes) + kMaxG * sizeof(Slot) + (size_t)L1.dpr * sizeof(u64);
  int b = (int)(bytes / per) + 1;
  Layout L;
  while (b > 0 && (!layout_for(b, V, &L) || L.total > bytes)) --b;
  return b;
}

// Library-owned scratch for qs_sample_static (callers that cannot allocate).
// In host code `scratch` names a host-side stand-in: the device address of each
// GPU's copy comes from hipGetSymbolAddress, once per device.
constexpr size_t kStaticScratchBytes = size_t(32) << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];
constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

extern "C" {

int qs_version(void) { return 20000; }

#ifdef QS_TRACE
// Trace builds: [B, G, 16] u64 phase time stamps (device clock, 100 MHz) of the next calls.
void qs_trace_buffer(void* p) { g_trace = p; }
#endif

const char* qs_last_error(void) { return g_err; }

size_t qs_workspace_bytes(int B, int V, int logits_dtype, int H) {
  (void)logits_dtype;
  (void)H;
  Layout L;
  if (B < 0 || !layout_for(B, V, &L)) return 0;
  return L.total;
}

int qs_workspace_init(void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!workspace || workspace_bytes % 4 != 0) return fail("qs_workspace_init: null or unaligned workspace");
  const size_t n = workspace_bytes / 4;
  const int grid = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(k_zero, dim3(grid > 0 ? grid : 1), dim3(256), 0, stream, (u32*)workspace, n);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("qs_workspace_init: launch failed (%lld)", (long long)e);
  return 0;
}

int qs_sample(const void* logits, int64_t row_stride, int logits_dtype, int B, int V, const float* temperature,
              const float* top_p, const int32_t* top_k, const float* min_p, const float* rep_pen,
              const float* pres_pen, const float* freq_pen, const int32_t* hist_ids, int H,
              const int32_t* hist_len, const float* uniforms, const int32_t* row_order, uint32_t flags,
              int64_t* out_ids, float* out_probs, int32_t* out_kept, void* workspace, size_t workspace_bytes,
              hipStream_t stream) {
  g_err[0] = 0;
  if (B < 0) return fail("qs_sample: B < 0 (%lld)", B);
  if (B == 0) return 0;
  if (V <= 0) return fail("qs_sample: V must be positive (%lld)", V);
  if (logits_dtype != QS_DTYPE_F32 && logits_dtype != QS_DTYPE_BF16) return fail("qs_sample: unknown dtype %lld", logits_dtype);
  if (!logits || !out_ids || !workspace) return fail("qs_sample: logits, out_ids and workspace are required");
  if (row_stride < V) return fail("qs_sample: row_stride below V (%lld)", (long long)row_stride);
  if (!(flags & QS_FLAG_ALL_GREEDY) && !temperature) return fail("qs_sample: temperature is required");
  if (H < 0 || H > QS_MAX_HISTORY) return fail("qs_sample: history length out of range (%lld)", H);
  if ((H > 0) != (hist_ids != nullptr)) return fail("qs_sample: hist_ids and H must be given together");
  if (hist_len && !hist_ids) return fail("qs_sample: hist_len needs hist_ids");
  if (flags & ~(QS_FLAG_ALL_GREEDY | QS_FLAG_USE_TOP_P | QS_FLAG_NO_WAIT | QS_FLAG_SOLO))
    return fail("qs_sample: unknown flags 0x%llx", flags);
  Layout L;
  if (!layout_for(B, V, &L)) return fail("qs_sample: V too large (%lld)", V);
  const int maxB = max_rows_of(workspace_bytes, V);
  if (maxB < B) return fail("qs_sample: workspace holds %lld rows, fewer than B", maxB);
  Layout LM;
  layout_for(maxB, V, &LM);
  char* ws = (char*)workspace;
  Args a;
  memset(&a, 0, sizeof(a));
  a.logits = logits;
  a.row_stride = row_stride;
  a.B = B;
  a.V = V;
  a.G = L.G;
  a.R = L.R;
  a.SH = L.SH;
  a.kmu = (float)kCH / (float)V;
  a.H = H;
  const size_t esz = logits_dtype == QS_DTYPE_F32 ? 4 : 2;
  a.vec_ok = ((uintptr_t)logits % 16 == 0) && (((size_t)row_stride * esz) % 16 == 0);
  a.flags = flags;
  a.spin_limit = (flags & QS_FLAG_NO_WAIT) ? 0u : (1u << 20);
  a.temperature = temperature;
  a.top_p = top_p;
  a.top_k = top_k;
  a.min_p = min_p;
  a.rep = rep_pen;
  a.pres = pres_pen;
  a.freq = freq_pen;
  a.hist = hist_ids;
  a.hist_len = hist_len;
  a.uniforms = uniforms;
  a.order = row_order;
  a.out_ids = (long long*)out_ids;
  a.out_probs = out_probs;
  a.out_kept = out_kept;
  a.sync = (RowSync*)(ws + LM.off_sync);
  a.res = (RowRes*)(ws + LM.off_res);
  a.slots = (Slot*)(ws + LM.off_slots);
  a.data = (u64*)(ws + LM.off_data);
  a.data_per_row = LM.dpr;
#ifdef QS_TRACE
  a.trace = (u64*)g_trace;
#endif
  const dim3 grid(L.G, B), block(kThreads);
  const bool solo = (flags & QS_FLAG_SOLO) && L.G * kWaves <= kSoloSegs;  // one segment per wave and chunk
  if (solo) {
    // 16-byte vector loads need aligned rows and at least one whole vector
    const bool vec = a.vec_ok && a.V >= (logits_dtype == QS_DTYPE_F32 ? 4 : 8);
    if (logits_dtype == QS_DTYPE_F32) {
      if (vec)
        hipLaunchKernelGGL((k_solo<QS_DTYPE_F32, true>), dim3(B), block, 0, stream, a);
      else
        hipLaunchKernelGGL((k_solo<QS_DTYPE_F32, false>), dim3(B), block, 0, stream, a);
    } else {
      if (vec)
        hipLaunchKernelGGL((k_solo<QS_DTYPE_BF16, true>), dim3(B), block, 0, stream, a);
      else
        hipLaunchKernelGGL((k_solo<QS_DTYPE_BF16, false>), dim3(B), block, 0, stream, a);
    }
  } else if (logits_dtype == QS_DTYPE_F32) {
    hipLaunchKernelGGL(k_sample<QS_DTYPE_F32>, grid, block, 0, stream, a);
  } else {
    hipLaunchKernelGGL(k_sample<QS_DTYPE_BF16>, grid, block, 0, stream, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("qs_sample: launch failed (%lld)", (long long)e);
  if (out_probs) {
    if (logits_dtype == QS_DTYPE_F32)
      hipLaunchKernelGGL(k_probs<QS_DTYPE_F32>, grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL(k_probs<QS_DTYPE_BF16>, grid, block, 0, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return fail("qs_sample: probabilities launch failed (%lld)", (long long)e);
  }
  return 0;
}

int qs_sample_static(const void* logits, int64_t row_stride, int logits_dtype, int B, int V,
                     const float* temperature, const float* top_p, const int32_t* top_k, const float* min_p,
                     const float* rep_pen, const float* pres_pen, const float* freq_pen,
                     const int32_t* hist_ids, int H, const int32_t* hist_len, const float* uniforms,
                     const int32_t* row_order, uint32_t flags, int64_t* out_ids, float* out_probs,
                     int32_t* out_kept, hipStream_t stream) {
  g_err[0] = 0;
  if (B < 0) return fail("qs_sample_static: B < 0 (%lld)", B);
  if (B == 0) return 0;
  Layout L;
  if (V <= 0 || !layout_for(B, V, &L)) return fail("qs_sample_static: no layout for V = %lld", V);
  if (max_rows_of(kStaticScratchBytes, V) < B)
    return fail("qs_sample_static: the batch needs more than the static scratch (%lld bytes)",
                (long long)kStaticScratchBytes);
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail("qs_sample_static: no current device (%lld)", dev);
  if (!g_scratch_ptr[dev]) {
    // first call on this device: the address of its copy, cleared once by a fill kernel
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) return fail("qs_sample_static: hipGetSymbolAddress failed (%lld)", (long long)e);
    if (qs_workspace_init(ptr, kStaticScratchBytes, stream) != 0) return -1;
    g_scratch_ptr[dev] = ptr;
  }
  return qs_sample(logits, row_stride, logits_dtype, B, V, temperature, top_p, top_k, min_p, rep_pen, pres_pen,
                   freq_pen, hist_ids, H, hist_len, uniforms, row_order, flags, out_ids, out_probs, out_kept,
                   g_scratch_ptr[dev], kStaticScratchBytes, stream);
}

size_t qs_static_scratch_bytes(void) { return kStaticScratchBytes; }

int qs_argmax(const void* logits, int64_t row_stride, int logits_dtype, int B, int V, int64_t* out_ids,
              void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return qs_sample(logits, row_stride, logits_dtype, B, V, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                   nullptr, nullptr, 0, nullptr, nullptr, nullptr, QS_FLAG_ALL_GREEDY, out_ids, nullptr, nullptr,
                   workspace, workspace_bytes, stream);
}

int qs_step_finish(const int64_t* ids, int B, const int32_t* slots, int64_t* pending, int n_pending,
                   int32_t* num_generated, const int32_t* min_tokens, const int32_t* max_tokens,
                   const uint8_t* ignore_eos, int64_t eos_id, uint8_t* finished, int64_t* host_ids,
                   hipStream_t stream) {
  g_err[0] = 0;
  if (B < 0) return fail("qs_step_finish: B < 0 (%lld)", B);
  if (B == 0) return 0;
  if (!ids || !num_generated || !max_tokens) return fail("qs_step_finish: ids, num_generated and max_tokens are required");
  if (pending && n_pending <= 0) return fail("qs_step_finish: pending needs n_pending > 0 (%lld)", n_pending);
  StepArgs a;
  a.ids = (const long long*)ids;
  a.B = B;
  a.slots = slots;
  a.pending = (long long*)pending;
  a.n_pending = pending ? n_pending : 0;
  a.num_generated = num_generated;
  a.min_tokens = min_tokens;
  a.max_tokens = max_tokens;
  a.ignore_eos = ignore_eos;
  a.eos_id = eos_id;
  a.finished = finished;
  a.host_ids = (long long*)host_ids;
  hipLaunchKernelGGL(k_step_finish, dim3((B + 255) / 256), dim3(256), 0, stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("qs_step_finish: launch failed (%lld)", (long long)e);
  return 0;
}

int qs_history_append(int32_t* hist_ids, int B, int H, int32_t* hist_len, const int64_t* ids,
                      const uint8_t* active, hipStream_t stream) {
  g_err[0] = 0;
  if (B < 0) return fail("qs_history_append: B < 0 (%lld)", B);
  if (B == 0) return 0;
  if (H <= 0 || H > QS_MAX_HISTORY) return fail("qs_history_append: H out of range (%lld)", H);
  if (!hist_ids || !hist_len || !ids) return fail("qs_history_append: hist_ids, hist_len and ids are required");
  hipLaunchKernelGGL(k_history_append, dim3((B + 255) / 256), dim3(256), 0, stream, hist_ids, B, H, hist_len,
                     (const long long*)ids, active);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("qs_history_append: launch failed (%lld)", (long long)e);
  return 0;
}

}  // extern "C"
