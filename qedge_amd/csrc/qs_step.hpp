// Decode-step bookkeeping on the device, after the sampler: the pending-token
// slots, the per-row stop check and the token history.  One thread per row.
#pragma once

#include "qs_device.hpp"

namespace qs {

struct StepArgs {
  const long long* ids;     // [B] sampled ids
  int B;
  const int* slots;         // [B] pending slot of each row (or null: slot r)
  long long* pending;       // [n_pending] fixed next-token slots
  int n_pending;
  int* num_generated;       // [B] completion tokens so far (updated)
  const int* min_tokens;    // [B] or null (0)
  const int* max_tokens;    // [B]
  const unsigned char* ignore_eos;  // [B] or null (0)
  long long eos_id;         // < 0: no end-of-sequence token
  unsigned char* finished;  // [B] out
  long long* host_ids;      // [B] host-mapped mirror of the ids, or null
};

// Per row (src/control/scheduler.py:304-322 and src/compute/model_runner.py:95-115):
//   max_tokens <= 0: finished, nothing appended;
//   otherwise n = ++num_generated, finished = n >= max_tokens or
//   (!ignore_eos and n >= min_tokens and id == eos_id);
//   the id goes to its pending slot and to the host mirror either way.
__global__ void k_step_finish(StepArgs a) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= a.B) return;
  const long long id = gld(a.ids + r);
  const int slot = a.slots ? gld(a.slots + r) : r;
  if (a.pending && slot >= 0 && slot < a.n_pending) gst(a.pending + slot, id);
  const int maxt = gld(a.max_tokens + r);
  bool fin;
  if (maxt <= 0) {
    fin = true;
  } else {
    const int n = gld(a.num_generated + r) + 1;
    gst(a.num_generated + r, n);
    const int mint = a.min_tokens ? gld(a.min_tokens + r) : 0;
    const bool ign = a.ignore_eos ? gld(a.ignore_eos + r) != 0 : false;
    const bool hit_eos = !ign && n >= mint && a.eos_id >= 0 && id == a.eos_id;
    fin = hit_eos || n >= maxt;
  }
  if (a.finished) gst(a.finished + r, (unsigned char)(fin ? 1 : 0));
  if (a.host_ids) gst(a.host_ids + r, id);  // host-mapped memory
}

// Appends ids[r] to row r's history ring: hist[r, len % H] = id, len += 1.
// The sampler reads the last min(len, H) ids of a row (their order does not
// change the penalty counts).  Rows with active[r] == 0 are left alone.
__global__ void k_history_append(int* hist, int B, int H, int* hist_len, const long long* ids,
                                 const unsigned char* active) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= B) return;
  if (active && gld(active + r) == 0) return;
  const int len = gld(hist_len + r);
  const long long id = gld(ids + r);
  gst(hist + (size_t)r * H + (len % H), (int)id);
  gst(hist_len + r, len + 1 > 0 ? len + 1 : len);  // saturates at INT_MAX
}

}  // namespace qs
