"""Helpers: run a workload through the HIP sampler and the oracle."""
from __future__ import annotations

import numpy as np
import torch

from oracle import contract
from qedge_amd.sampler import Workspace, sample_into


def to_device(w, device):
    if w.dtype == "f32":
        logits = torch.from_numpy(np.ascontiguousarray(w.logits)).to(device)
    else:
        logits = torch.from_numpy(np.ascontiguousarray(w.logits).view(np.int16)).to(device).view(torch.bfloat16)
    t = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dt)
    return dict(logits=logits, temperatures=t(w.temperature, torch.float32), top_ps=t(w.top_p, torch.float32),
                top_ks=t(w.top_k, torch.int32), repetition_penalties=t(w.rep, torch.float32),
                presence_penalties=t(w.pres, torch.float32), frequency_penalties=t(w.freq, torch.float32),
                history=t(w.history, torch.int32))


def run_gpu(w, device, step=0, want_probs=True, all_greedy=False, use_top_p=True, ws=None, order=None, **extra):
    d = to_device(w, device)
    B, V = d["logits"].shape
    H = 0 if d["history"] is None else d["history"].shape[1]
    ws = ws or Workspace(B, V, d["logits"].dtype, H, device)
    u = torch.from_numpy(w.uniforms(step)).to(device)
    ids = torch.empty(B, dtype=torch.int64, device=device)
    probs = torch.empty((B, V), dtype=torch.float32, device=device) if want_probs else None
    kept = torch.empty(B, dtype=torch.int32, device=device) if want_probs else None
    logits = d.pop("logits")
    if order is not None:
        extra["row_order"] = torch.from_numpy(np.ascontiguousarray(order, dtype=np.int32)).to(device)
    sample_into(logits, ids, ws, uniforms=u, all_greedy=all_greedy, use_top_p=use_top_p,
                out_probs=probs, out_kept=kept, **d, **extra)
    torch.cuda.synchronize()
    return (ids.cpu().numpy(), None if probs is None else probs.cpu().numpy(),
            None if kept is None else kept.cpu().numpy())


def run_oracle(w, step=0, want_probs=True):
    return contract.sample_workload(w, step=step, want_probs=want_probs)


# Per-row resolution record of the last call.  The workspace starts with the
# row counters (640 bytes per row of the workspace's maximum batch), then the
# row results (128 bytes per row): word 13 is the path (1 greedy, 2 top-k,
# 3 top-k-off with top-p, 4 top-k-off without, 5 single workgroup), word 14 the
# reason a row went to the single-workgroup path (0: it did not).
def row_paths(ws, B):
    off = (ws.max_bs * 640 + 255) // 256 * 256
    raw = ws.buf[off: off + B * 128].cpu().numpy().view(np.uint32).reshape(B, 32)
    return raw[:, 13].copy(), raw[:, 14].copy()


def order_of(T, K, V):
    """The dispatch order SamplingBatch stages: top-k-off rows, top-k rows by descending k, greedy rows."""
    def kind(t, k):
        if t <= 1e-5:
            return 2
        return 1 if 0 < k < V and k <= 1024 else 0
    K = np.zeros(len(T), np.int32) if K is None else K
    return np.array([r for _, _, r in sorted((kind(T[r], K[r]), 0 if T[r] <= 1e-5 else -int(K[r]), r)
                                               for r in range(len(T)))], np.int32)
