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


def run_gpu(w, device, step=0, want_probs=True, all_greedy=False, use_top_p=True, ws=None):
    d = to_device(w, device)
    B, V = d["logits"].shape
    H = 0 if d["history"] is None else d["history"].shape[1]
    ws = ws or Workspace(B, V, d["logits"].dtype, H, device)
    u = torch.from_numpy(w.uniforms(step)).to(device)
    ids = torch.empty(B, dtype=torch.int64, device=device)
    probs = torch.empty((B, V), dtype=torch.float32, device=device) if want_probs else None
    kept = torch.empty(B, dtype=torch.int32, device=device) if want_probs else None
    logits = d.pop("logits")
    sample_into(logits, ids, ws, uniforms=u, all_greedy=all_greedy, use_top_p=use_top_p, mass_rows=w.mass_rows,
                out_probs=probs, out_kept=kept, **d)
    torch.cuda.synchronize()
    return (ids.cpu().numpy(), None if probs is None else probs.cpu().numpy(),
            None if kept is None else kept.cpu().numpy())


def run_oracle(w, step=0, want_probs=True):
    return contract.sample_workload(w, step=step, want_probs=want_probs)


# Per-row resolution record of the last call, from the row control blocks at
# the start of the workspace (256 bytes per row): word 30 is the path (0
# greedy, 1 top-k, 2 flat mass row, 3 single workgroup, 4 peaked mass row),
# word 32 the reason a row went to the single-workgroup path (0: it did not).
def row_paths(ws, B):
    raw = ws.buf[: B * 256].cpu().numpy().view(np.uint32).reshape(B, 64)
    return raw[:, 30].copy(), raw[:, 32].copy()
