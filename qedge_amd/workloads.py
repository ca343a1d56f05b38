"""Deterministic synthetic sampler workloads (the five decode-step shapes).

Every value is derived from raw ``numpy.random.PCG64`` output bits and this
module's own transforms (Box-Muller in float64, Gumbel by double logarithm,
Zipf by inverse CDF, bf16 by round-to-nearest-even of the fp32 bits), so the
inputs do not depend on numpy's distribution code.  Each row of each tensor has
its own stream, so any subset of rows is identical to the same rows of the full
workload.

"N(0, s)" is read as standard deviation ``s``.

Shapes (vocabulary V = 248320):

* ``greedy_spikes_f32``: B=1 fp32 N(0,2) with 5 planted spikes at +12.0; one
  greedy row and one T=1.0 full-vocabulary row (the default single-request
  path of the reference engine).
* ``topk_topp_rep_bf16``: B=1 bf16 N(0,3); T=0.7, top_k=20, top_p=0.8,
  repetition penalty 1.05 over 2048 uniform history ids.
* ``hetero_b64_bf16``: B=64 bf16 Gumbel(0,1)*s, s~U[1,4]; per-row T~U[0.1,1.5],
  top_k~U{1..1000} with 6 rows top_k=0 (off), top_p~U[0.5,1.0], 6 greedy rows.
* ``penalties_b256_bf16``: B=256 bf16 N(0,2); repetition 1.1, presence 0.5,
  frequency 0.3 over 4096 Zipf(1.1) history ids per row; T=0.8, top_p=0.95.
* ``flat_topp_b1024_f32``: B=1024 fp32 N(0,0.05); top_p=0.95, T=1.0.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

VOCAB = 248320
SEED_BASE = 0x5A3D0000

# stream kinds
_LOGITS, _PARAMS, _HIST, _UNIF, _PERM = 0, 1, 2, 3, 4


def _raw(seed: int, kind: int, index: int, n: int) -> np.ndarray:
    ss = np.random.SeedSequence(entropy=seed, spawn_key=(kind, index))
    return np.random.PCG64(ss).random_raw(n).astype(np.uint64)


def _unit(bits: np.ndarray) -> np.ndarray:
    """[0, 1) doubles with 53 random bits."""
    return (bits >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def _open_unit(bits: np.ndarray) -> np.ndarray:
    """(0, 1) doubles."""
    return ((bits >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def _normal(seed: int, kind: int, index: int, n: int) -> np.ndarray:
    half = (n + 1) // 2
    b = _raw(seed, kind, index, 2 * half)
    u1 = _open_unit(b[:half])
    u2 = _unit(b[half:])
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * half, dtype=np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return out[:n]


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 (nearest, ties to even); returns uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return rounded.astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def uniform_f32(seed: int, row: int, step: int) -> np.float32:
    """The host uniform of a row at a decode step: 24 random bits, in [0, 1)."""
    b = _raw(seed, _UNIF, row * 1_000_003 + step, 1)[0]
    return np.float32(float(int(b) >> 40) * (1.0 / 16777216.0))


@dataclass
class Workload:
    name: str
    B: int
    V: int
    dtype: str  # "f32" or "bf16"
    seed: int
    rows: list[int]
    logits: np.ndarray  # float32 [b, V] or uint16 bf16 bits [b, V]
    temperature: np.ndarray
    top_p: np.ndarray
    top_k: np.ndarray
    rep: np.ndarray | None = None
    pres: np.ndarray | None = None
    freq: np.ndarray | None = None
    history: np.ndarray | None = None  # int32 [b, H]
    notes: dict = field(default_factory=dict)

    @property
    def nrows(self) -> int:
        return len(self.rows)

    def uniforms(self, step: int) -> np.ndarray:
        return np.array([uniform_f32(self.seed, r, step) for r in self.rows], dtype=np.float32)

    @property
    def mass_rows(self) -> bool:
        """Host-side batch flag: some sampling row has top-k off (or above the fast limit)."""
        k = self.top_k.astype(np.int64)
        fast = (k > 0) & (k <= 1024) & (k < self.V)
        return bool(np.any((self.temperature > 1e-5) & ~fast))

    def logits_f32(self) -> np.ndarray:
        return self.logits if self.dtype == "f32" else bf16_to_f32(self.logits)

    @property
    def bytes_per_logit(self) -> int:
        return 4 if self.dtype == "f32" else 2

    def algorithmic_bytes(self) -> int:
        """B*V*sizeof(logit) + history ids*4 + per-row params, uniform and id out."""
        b = self.nrows * self.V * self.bytes_per_logit
        if self.history is not None:
            b += self.history.size * 4
        return b + self.nrows * (24 + 4 + 8)


WORKLOADS = (
    "greedy_spikes_f32",
    "topk_topp_rep_bf16",
    "hetero_b64_bf16",
    "penalties_b256_bf16",
    "flat_topp_b1024_f32",
)
FULL_B = {
    "greedy_spikes_f32": 2,  # row 0 greedy, row 1 T=1.0 over the same logits
    "topk_topp_rep_bf16": 1,
    "hetero_b64_bf16": 64,
    "penalties_b256_bf16": 256,
    "flat_topp_b1024_f32": 1024,
}


def _rows_arg(name: str, rows) -> list[int]:
    if rows is None:
        return list(range(FULL_B[name]))
    return [int(r) for r in rows]


def make(name: str, rows=None, V: int = VOCAB) -> Workload:
    """Build a workload (all rows, or the given row indices)."""
    idx = _rows_arg(name, rows)
    seed = SEED_BASE + WORKLOADS.index(name) + 1
    b = len(idx)
    if name == "greedy_spikes_f32":
        base = _normal(seed, _LOGITS, 0, V) * 2.0
        pos_bits = _raw(seed, _PARAMS, 0, 64)
        spikes: list[int] = []
        for bits in pos_bits:
            p = int(bits % np.uint64(V))
            if p not in spikes:
                spikes.append(p)
            if len(spikes) == 5:
                break
        base[spikes] = 12.0
        row = base.astype(np.float32)
        logits = np.stack([row for _ in idx])
        temp = np.array([0.0 if r == 0 else 1.0 for r in idx], dtype=np.float32)
        return Workload(name, FULL_B[name], V, "f32", seed, idx, logits, temp,
                        np.ones(b, np.float32), np.zeros(b, np.int32),
                        notes={"spikes": sorted(spikes)})
    if name == "topk_topp_rep_bf16":
        logits = np.stack([bf16_bits((_normal(seed, _LOGITS, r, V) * 3.0).astype(np.float32)) for r in idx])
        hist = np.stack([(_raw(seed, _HIST, r, 2048) % np.uint64(V)).astype(np.int32) for r in idx])
        return Workload(name, FULL_B[name], V, "bf16", seed, idx, logits,
                        np.full(b, 0.7, np.float32), np.full(b, 0.8, np.float32),
                        np.full(b, 20, np.int32), rep=np.full(b, 1.05, np.float32),
                        pres=np.zeros(b, np.float32), freq=np.zeros(b, np.float32), history=hist)
    if name == "hetero_b64_bf16":
        B = FULL_B[name]
        pb = _raw(seed, _PARAMS, 0, 8 * B)
        u = _unit(pb)
        scale = 1.0 + 3.0 * u[0:B]
        temp = (0.1 + 1.4 * u[B:2 * B]).astype(np.float32)
        top_k = (1 + (pb[2 * B:3 * B] % np.uint64(1000))).astype(np.int32)
        top_p = (0.5 + 0.5 * u[3 * B:4 * B]).astype(np.float32)
        order = np.argsort(pb[4 * B:5 * B], kind="stable")
        top_k[order[:B // 10]] = 0
        order2 = np.argsort(pb[5 * B:6 * B], kind="stable")
        temp[order2[:B // 10]] = 0.0
        rows = []
        for r in idx:
            g = -np.log(-np.log(_open_unit(_raw(seed, _LOGITS, r, V))))
            rows.append(bf16_bits((g * scale[r]).astype(np.float32)))
        return Workload(name, B, V, "bf16", seed, idx, np.stack(rows), temp[idx], top_p[idx], top_k[idx],
                        notes={"topk_off_rows": sorted(int(i) for i in order[:B // 10]),
                               "greedy_rows": sorted(int(i) for i in order2[:B // 10])})
    if name == "penalties_b256_bf16":
        logits = np.stack([bf16_bits((_normal(seed, _LOGITS, r, V) * 2.0).astype(np.float32)) for r in idx])
        ranks = np.arange(1, V + 1, dtype=np.float64)
        cdf = np.cumsum(ranks ** -1.1)
        cdf /= cdf[-1]
        perm = np.argsort(_raw(seed, _PERM, 0, V), kind="stable").astype(np.int32)
        hist = []
        for r in idx:
            uu = _unit(_raw(seed, _HIST, r, 4096))
            rk = np.minimum(np.searchsorted(cdf, uu, side="right"), V - 1)
            hist.append(perm[rk])
        return Workload(name, FULL_B[name], V, "bf16", seed, idx, logits,
                        np.full(b, 0.8, np.float32), np.full(b, 0.95, np.float32),
                        np.zeros(b, np.int32), rep=np.full(b, 1.1, np.float32),
                        pres=np.full(b, 0.5, np.float32), freq=np.full(b, 0.3, np.float32),
                        history=np.stack(hist).astype(np.int32))
    if name == "flat_topp_b1024_f32":
        logits = np.stack([(_normal(seed, _LOGITS, r, V) * 0.05).astype(np.float32) for r in idx])
        return Workload(name, FULL_B[name], V, "f32", seed, idx, logits,
                        np.ones(b, np.float32), np.full(b, 0.95, np.float32), np.zeros(b, np.int32))
    raise KeyError(name)
