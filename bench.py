#!/usr/bin/env python3
"""Decode-step sampler benchmark on one MI355X.

The JSON line's ``value`` is sampled rows/s on the heterogeneous batch (B=64
rows of V=248320 bf16 logits, per-row temperature / top-k / top-p, 10% greedy
rows, 10% top-k off), with µs per step and algorithmic HBM GB/s as a fraction
of the 8 TB/s HBM roofline.  ``workloads`` holds the same figures for every
synthetic config: the B=1 greedy and T=1 rows of the spiked fp32 config (each
alone, as a single request runs), the B=1 top-k/top-p/repetition row, the B=64
batch, the B=256 penalties batch and the B=1024 near-flat top-p batch.  The
torch-CPU restatement of the reference sampler is timed on the host cores over
a bounded sample of the B=64 batch, with all threads and with one thread.

A step is one ``qs_sample`` call over one batch.  Inputs are resident in HBM
before the timed region: the logits are held in several copies that the steps
rotate through, so that each step reads its batch from HBM rather than from
the 256 MB last-level cache.  Exactly K steps are captured in one HIP graph
(the way the decode loop runs) and the graph is replayed; the timed region is
bracketed by ``torch.cuda.synchronize()`` and measured with HIP events on the
stream the kernels run on.  One step is one kernel launch, so µs per step is
also the launch's average duration that the roofline fraction uses.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
Prints ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
WORKLOAD = "hetero_b64_bf16"
B1_WORKLOAD = "topk_topp_rep_bf16"
ROTATE_BYTES = 640 << 20  # rotate through >= 640 MB of logits copies (LLC is 256 MB)


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Case:
    """One workload staged on the device with R rotating copies of its inputs."""

    def __init__(self, name: str, device, rotate_bytes: int = ROTATE_BYTES, max_copies: int = 64, rows=None):
        import numpy as np
        import torch

        from qedge_amd import workloads as W
        from qedge_amd.sampler import Workspace

        self.w = w = W.make(name, rows=rows)
        self.name = name if rows is None else f"{name}[rows {','.join(str(r) for r in rows)}]"
        B, V = w.nrows, w.V
        self.B, self.V = B, V
        if w.dtype == "f32":
            base = torch.from_numpy(np.ascontiguousarray(w.logits)).to(device)
        else:
            base = torch.from_numpy(np.ascontiguousarray(w.logits).view(np.int16)).to(device).view(torch.bfloat16)
        nbytes = base.numel() * base.element_size()
        self.R = R = max(1, min(max_copies, math.ceil(rotate_bytes / nbytes)))
        self.logits = [base] + [base.clone() for _ in range(R - 1)]
        t = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dt)
        topk_on = bool(np.any((w.top_k > 0) & (w.top_k < V)))  # as SamplingBatch.use_top_k
        self.params = dict(temperatures=t(w.temperature, torch.float32), top_ps=t(w.top_p, torch.float32),
                           top_ks=t(w.top_k, torch.int32) if topk_on else None,
                           repetition_penalties=t(w.rep, torch.float32),
                           presence_penalties=t(w.pres, torch.float32),
                           frequency_penalties=t(w.freq, torch.float32), history=t(w.history, torch.int32))
        self.uniforms = [t(w.uniforms(s), torch.float32) for s in range(R)]
        H = 0 if w.history is None else w.history.shape[1]
        self.ws = Workspace(B, V, base.dtype, H, device)
        self.order = t(dispatch_order(w), torch.int32)
        self.ids = torch.empty(B, dtype=torch.int64, device=device)
        self.alg_bytes = w.algorithmic_bytes()

    def step(self, i: int) -> None:
        from qedge_amd.sampler import sample_into

        r = i % self.R
        sample_into(self.logits[r], self.ids, self.ws, uniforms=self.uniforms[r], use_top_p=True,
                    row_order=self.order, **self.params)


def dispatch_order(w):
    """The row order the host stages beside the parameters (qedge_amd.batch.SamplingBatch):
    rows with top-k off first, then top-k rows by descending k, greedy rows last."""
    import numpy as np

    def kind(t, k):
        if t <= 1e-5:
            return 2
        return 1 if 0 < k < w.V and k <= 1024 else 0

    rank = sorted((kind(w.temperature[r], w.top_k[r]), 0 if w.temperature[r] <= 1e-5 else -int(w.top_k[r]), r)
                  for r in range(w.nrows))
    return np.array([r for _, _, r in rank], np.int32)


def time_graph(case: Case, steps: int, warmup: int, repeats: int = 3):
    """µs/step over replays of one graph holding exactly ``steps`` steps; median of ``repeats``."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(max(warmup, 1)):
            case.step(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            case.step(i)
    torch.cuda.synchronize()
    g.replay()  # warm the graph
    torch.cuda.synchronize()
    results = []
    stream = torch.cuda.current_stream()
    for _ in range(repeats):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        g.replay()
        stop.record(stream)
        torch.cuda.synchronize()
        results.append(start.elapsed_time(stop) * 1000.0 / steps)
    del g
    return statistics.median(results), steps, results


def time_eager(case: Case, steps: int):
    """Host-inclusive µs per call (ctypes launch from Python, no graph)."""
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        case.step(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e6 / steps


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(name: str, budget_s: float = 20.0):
    """The torch-CPU restatement of the reference sampler on this host's cores:
    median ms/step with torch's default thread count, then with one thread."""
    import numpy as np
    import torch

    from oracle import torch_ref
    from qedge_amd import workloads as W

    w = W.make(name)
    if w.dtype == "f32":
        logits = torch.from_numpy(np.ascontiguousarray(w.logits))
    else:
        logits = torch.from_numpy(np.ascontiguousarray(w.logits).view(np.int16)).view(torch.bfloat16)
    t = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    kw = dict(top_ks=t(w.top_k, torch.int32), rep=t(w.rep, torch.float32), pres=t(w.pres, torch.float32),
              freq=t(w.freq, torch.float32), history=t(w.history, torch.int32))
    T, P = t(w.temperature, torch.float32), t(w.top_p, torch.float32)
    gen = torch.Generator().manual_seed(0)

    def timed(budget: float, max_steps: int):
        times = []
        with torch.inference_mode():
            torch_ref.extended_forward(logits, T, P, use_top_p=True, generator=gen, **kw)  # warm-up
            t_start = time.perf_counter()
            while len(times) < max_steps:
                t0 = time.perf_counter()
                torch_ref.extended_forward(logits, T, P, use_top_p=True, generator=gen, **kw)
                times.append(time.perf_counter() - t0)
                if time.perf_counter() - t_start > budget and len(times) >= 3:
                    break
        return statistics.median(times), len(times)

    threads = torch.get_num_threads()
    med, n = timed(budget_s * 0.5, 20)
    torch.set_num_threads(1)
    try:
        med1, n1 = timed(budget_s * 0.5, 10)
    finally:
        torch.set_num_threads(threads)
    return {
        "value": round(w.nrows / med, 3),
        "unit": "rows/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{name}: B={w.nrows} rows per step, median of {n} timed steps after one warm-up step; "
                   f"torch-CPU restatement of the reference op sequence with top-k/top-p and penalties "
                   f"(oracle/torch_ref.extended_forward) on {threads} threads of {os.cpu_count()} host CPUs "
                   f"({_cpu_model()}); also {n1} steps on one thread"),
        "ms_per_step": round(med * 1e3, 3),
        "one_thread": {"value": round(w.nrows / med1, 3), "unit": "rows/s", "cores": 1,
                       "ms_per_step": round(med1 * 1e3, 3)},
        "host_cpus": os.cpu_count(),
        "cpu_model": _cpu_model(),
    }


def counter_run(case: Case, steps: int, calib_mib: int = 1024, calib_runs: int = 4) -> dict:
    """Short eager run for hardware-counter passes (rocprofv3 --pmc).

    ``steps`` sampler calls, each on a different logits copy, then
    ``calib_runs`` plain device copies of ``calib_mib`` MiB (torch's copy
    kernel): their counters per dispatch are the scale that turns the
    sampler's counters into HBM bytes.
    """
    import torch

    for i in range(3):
        case.step(i)
    torch.cuda.synchronize()
    for i in range(steps):
        case.step(3 + i)
    torch.cuda.synchronize()
    n = calib_mib << 18  # float32 elements
    src = torch.empty(n, dtype=torch.float32, device=case.ids.device).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(calib_runs):
        dst.copy_(src)
    torch.cuda.synchronize()
    return {"mode": "counters", "workload": case.name, "sampler_calls": steps + 3,
            "calibration_copy_bytes": n * 4, "calibration_runs": calib_runs}


def traffic_from_profile(name: str):
    """HBM bytes per launch measured by rocprofv3 --pmc, if a summary is committed."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("hbm_bytes_per_launch")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default=WORKLOAD)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-b1", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--counters", type=int, default=0, metavar="N",
                    help="only run N eager sampler calls and a calibration copy (for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures the sampler on one GPU only: every row is independent, so N GPUs "
              "would each run this same kernel on B/N rows; run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 2
    from qedge_amd import _lib

    _lib.load()
    dev = torch.device("cuda:0")
    _log(f"device {torch.cuda.get_device_name(dev)}; staging {args.workload}")
    case = Case(args.workload, dev)
    if args.counters > 0:
        print(json.dumps(counter_run(case, args.counters)), flush=True)
        return 0
    _log(f"B={case.B} V={case.V} copies={case.R}; warmup {args.warmup}, steps {args.steps}")
    torch.cuda.synchronize()
    us, steps_done, reps = time_graph(case, args.steps, args.warmup)
    _log(f"graph replay: {us:.3f} us/step (repeats {[round(r, 3) for r in reps]})")
    eager_us = time_eager(case, min(args.steps, 500))
    _log(f"eager (host-inclusive): {eager_us:.3f} us/call")

    # every synthetic config (the spiked fp32 one as its two single-request rows)
    workloads = []
    b1 = None
    if not args.no_b1:
        plan = [("greedy_spikes_f32", [0]), ("greedy_spikes_f32", [1]), (B1_WORKLOAD, None),
                (WORKLOAD, None), ("penalties_b256_bf16", None), ("flat_topp_b1024_f32", None)]
        for name, rows in plan:
            if name == args.workload and rows is None:
                c, w_us, w_steps = case, us, steps_done
            else:
                c = Case(name, dev, rows=rows)
                w_steps = min(args.steps, 400 if c.B <= 64 else 100)
                w_us, _, _ = time_graph(c, w_steps, min(args.warmup, 20))
            gbs = c.alg_bytes / (w_us * 1e-6) / 1e9
            entry = {"workload": c.name, "B": c.B, "logits": c.w.dtype, "us_per_step": round(w_us, 3),
                     "rows_per_s": round(c.B / (w_us * 1e-6), 3), "hbm_gbs": round(gbs, 3),
                     "roofline_frac": round(gbs / HBM_PEAK_GBS, 5), "steps": w_steps}
            workloads.append(entry)
            _log(f"{c.name}: {w_us:.3f} us/step, {gbs:.1f} GB/s")
            if c is not case:
                del c
                torch.cuda.empty_cache()
        b1 = {"workload": B1_WORKLOAD, "us_per_step": next(e["us_per_step"] for e in workloads
                                                             if e["workload"] == B1_WORKLOAD)}

    cpu = None
    if not args.no_cpu_baseline:
        _log("cpu baseline ...")
        cpu = cpu_baseline(args.workload, args.cpu_budget)
        _log(f"cpu baseline: {cpu['ms_per_step']} ms/step on {cpu['cores']} threads, "
             f"{cpu['one_thread']['ms_per_step']} ms/step on one")

    sec = us * 1e-6
    achieved = case.alg_bytes / sec / 1e9
    out = {
        "metric": "sampled rows/s + HBM GB/s (B=64,V=248320 bf16); us/step at B=1",
        "value": round(case.B / sec, 3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps_done,
        "warmup": args.warmup,
        "ms_per_step": round(us / 1000.0, 6),
        "us_per_step": round(us, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": args.workload, "B": case.B, "V": case.V, "logits": case.w.dtype,
                   "algorithmic_bytes_per_step": case.alg_bytes, "rotating_copies": case.R,
                   "timing": "one HIP graph of exactly `steps` steps, replayed; HIP events",
                   "eager_us_per_call": round(eager_us, 3)},
        "hbm_gbs": round(achieved, 3),
        "b1": b1,
        "workloads": workloads,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": traffic_from_profile(args.workload)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
