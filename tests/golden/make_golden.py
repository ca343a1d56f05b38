"""Writes tests/golden/oracle_vectors.npz: inputs and oracle outputs of small
mixed problems, and the oracle's outputs on row subsets of the five workloads.

A drift guard for the oracle and for the workload generator: test_golden.py
re-derives everything and compares bit for bit.  Regenerate only when the
sampling contract changes on purpose:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import contract  # noqa: E402
from qedge_amd import workloads as W  # noqa: E402

WORKLOAD_ROWS = {
    "greedy_spikes_f32": [0, 1],
    "topk_topp_rep_bf16": [0],
    "hetero_b64_bf16": [0, 5, 16, 27, 39, 63],
    "penalties_b256_bf16": [0, 128, 255],
    "flat_topp_b1024_f32": [0, 1023],
}


def digest(row: np.ndarray) -> int:
    """Order-sensitive 64-bit digest of a row's raw bits (workload drift guard)."""
    h = np.ascontiguousarray(row).view(np.uint16).astype(np.uint64)
    with np.errstate(over="ignore"):
        v = (h + np.uint64(0x9E3779B9)) * (np.arange(h.size, dtype=np.uint64) * np.uint64(2) + np.uint64(1))
    return int(np.bitwise_xor.reduce(v))


def mixed_problem(seed: int, B: int, V: int, dtype: str):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((B, V)) * rng.uniform(0.05, 4.0, (B, 1))).astype(np.float32)
    x[0, 7] = np.nan
    x[1, :] = np.round(x[1, :] * 2) / 2  # heavy ties
    logits = W.bf16_bits(x) if dtype == "bf16" else x
    T = rng.uniform(0.1, 1.5, B).astype(np.float32)
    T[2] = 0.0
    P = rng.uniform(0.3, 1.0, B).astype(np.float32)
    K = rng.integers(0, V // 2, B).astype(np.int32)
    rep = rng.uniform(0.9, 1.3, B).astype(np.float32)
    pres = rng.uniform(0.0, 0.5, B).astype(np.float32)
    freq = rng.uniform(0.0, 0.5, B).astype(np.float32)
    hist = rng.integers(-3, V + 3, (B, 32)).astype(np.int32)
    u = rng.random(B).astype(np.float32)
    return dict(logits=logits, T=T, P=P, K=K, rep=rep, pres=pres, freq=freq, hist=hist, u=u)


def solve(prob, dtype):
    return contract.sample(prob["logits"], dtype, prob["T"], prob["P"], prob["K"], prob["rep"], prob["pres"],
                           prob["freq"], prob["hist"], prob["u"], want_probs=True)


def main():
    out = {}
    for tag, (seed, B, V, dtype) in {"mix_f32": (11, 12, 777, "f32"), "mix_bf16": (12, 12, 1500, "bf16")}.items():
        prob = mixed_problem(seed, B, V, dtype)
        res = solve(prob, dtype)
        for k, v in prob.items():
            out[f"{tag}/{k}"] = v
        out[f"{tag}/ids"] = res.ids
        out[f"{tag}/kept"] = res.kept
        out[f"{tag}/probs"] = res.probs
    for name, rows in WORKLOAD_ROWS.items():
        w = W.make(name, rows=rows)
        res = contract.sample_workload(w, want_probs=True)
        out[f"{name}/ids"] = res.ids
        out[f"{name}/kept"] = res.kept
        out[f"{name}/topk_end"] = res.kend
        out[f"{name}/W_hex"] = np.array([format(x, "x") for x in res.W])
        out[f"{name}/probs_sum"] = res.probs.astype(np.float64).sum(axis=1)
        out[f"{name}/logits_digest"] = np.array([digest(r) for r in w.logits], dtype=np.uint64)
    path = os.path.join(HERE, "oracle_vectors.npz")
    np.savez_compressed(path, **out)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
