"""Device-resident sampling parameters for a batch of requests.

Mirrors the sampling part of ``Batch`` (src/data/batch.py:57-66, 75-88,
149-175): fixed-address device buffers sized for ``max_bs`` rows, refilled
through reusable pinned host staging with non-blocking copies, skipped when the
parameter signature is unchanged, and the host-side batch flags derived from the
CPU parameters (no device read).  The extensions add the penalty buffers, the
token-history matrix and the per-step host uniforms.

Normalisation (src/data/batch.py:152-158): top_p None -> 1.0; top_k None or
<= 0 -> V (off), else min(k, V); min_p None -> 0.  Values are rounded to fp32
once, on staging.
"""
from __future__ import annotations

import numpy as np
import torch

from .sampling_params import SamplingParams

_GOLDEN = 0x9E3779B97F4A7C15
_MASK64 = (1 << 64) - 1


def _splitmix64(x: np.ndarray) -> np.ndarray:
    """splitmix64 finaliser (Steele, Lea, Flood 2014), vectorised over uint64."""
    with np.errstate(over="ignore"):
        z = x + np.uint64(_GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def seeded_uniforms(seeds: np.ndarray, step: int) -> np.ndarray:
    """One uniform in [0, 1) per row from (seed, step): 24 random bits, float32 exact."""
    s = np.asarray(seeds, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = s * np.uint64(_GOLDEN) + np.uint64((step * 0xD1B54A32D192ED03) & _MASK64)
    bits = _splitmix64(x) >> np.uint64(40)
    return (bits.astype(np.float64) * (1.0 / 16777216.0)).astype(np.float32)


class SamplingBatch:
    """Sampling parameters of up to ``max_bs`` rows on ``device``."""

    def __init__(self, max_bs: int, vocab_size: int, device: torch.device, max_history: int = 0,
                 fast_topk: int = 1024):
        self.max_bs, self.vocab_size, self.device = max_bs, vocab_size, device
        self.fast_topk = fast_topk
        f32 = dict(dtype=torch.float32, device=device)
        self.temperatures = torch.zeros(max_bs, **f32)
        self.top_ps = torch.zeros(max_bs, **f32)
        self.top_ks = torch.zeros(max_bs, dtype=torch.int32, device=device)
        self.min_ps = torch.zeros(max_bs, **f32)
        self.repetition_penalties = torch.ones(max_bs, **f32)
        self.presence_penalties = torch.zeros(max_bs, **f32)
        self.frequency_penalties = torch.zeros(max_bs, **f32)
        self.uniforms = torch.zeros(max_bs, **f32)
        self.row_order = torch.zeros(max_bs, dtype=torch.int32, device=device)
        self.max_history = max_history
        self.history = (torch.full((max_bs, max_history), -1, dtype=torch.int32, device=device)
                        if max_history > 0 else None)
        self._staging: dict[tuple[int, torch.dtype], torch.Tensor] = {}
        self._staged: dict[tuple[int, torch.dtype], object] = {}  # event of the last copy out of each buffer
        self._signature: tuple | None = None
        self._order_sig: tuple | None = None
        self._rng = np.random.default_rng()
        self.bs = 0
        self.all_greedy = True
        self.any_greedy = False
        self.use_top_k = False
        self.use_top_p = False
        self.use_min_p = False
        self.use_penalties = False
        self.mass_rows = False
        self.max_top_k = 0

    def _cp(self, dst: torch.Tensor, data, dtype: torch.dtype) -> None:
        """Write ``data`` into reusable pinned staging, then a non-blocking H2D copy (:75-88).

        The staging buffer is rewritten only after the previous copy out of it
        has completed (an event recorded after each copy), so a step never
        overwrites the values of a step whose copy is still queued."""
        flat = dst.reshape(-1)
        key = (flat.data_ptr(), dtype)
        cpu = self._staging.get(key)
        pin = flat.is_cuda
        if cpu is None or cpu.numel() < flat.numel():
            cpu = torch.empty(flat.numel(), dtype=dtype, pin_memory=pin)
            self._staging[key] = cpu
            self._staged.pop(key, None)
        ev = self._staged.get(key)
        if ev is not None:
            ev.synchronize()
        arr = np.asarray(data).reshape(-1)
        cpu.numpy()[: arr.size] = arr
        flat[: arr.size].copy_(cpu[: arr.size], non_blocking=True)
        if pin:
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(flat.device))
            self._staged[key] = ev

    def fill(self, params: list[SamplingParams], histories: list[list[int]] | None = None,
             step: int = 0) -> None:
        """Stage the rows' parameters (and token histories) for the next sampler call."""
        bs = len(params)
        if bs > self.max_bs:
            raise ValueError(f"batch of {bs} exceeds max_bs={self.max_bs}")
        V = self.vocab_size
        temps = [float(s.temperature) for s in params]
        top_ps = [1.0 if s.top_p is None else float(s.top_p) for s in params]
        top_ks = [V if (s.top_k is None or s.top_k <= 0) else min(int(s.top_k), V) for s in params]
        min_ps = [0.0 if s.min_p is None else float(s.min_p) for s in params]
        reps = [float(s.repetition_penalty) for s in params]
        pres = [float(s.presence_penalty) for s in params]
        freq = [float(s.frequency_penalty) for s in params]
        signature = tuple(zip(temps, top_ps, top_ks, min_ps, reps, pres, freq))
        if signature != self._signature:
            self._cp(self.temperatures[:bs], np.array(temps, np.float32), torch.float32)
            self._cp(self.top_ps[:bs], np.array(top_ps, np.float32), torch.float32)
            self._cp(self.top_ks[:bs], np.array(top_ks, np.int32), torch.int32)
            self._cp(self.min_ps[:bs], np.array(min_ps, np.float32), torch.float32)
            self._cp(self.repetition_penalties[:bs], np.array(reps, np.float32), torch.float32)
            self._cp(self.presence_penalties[:bs], np.array(pres, np.float32), torch.float32)
            self._cp(self.frequency_penalties[:bs], np.array(freq, np.float32), torch.float32)
            self._signature = signature
        # host flags from the CPU values (src/data/batch.py:169-174, src/compute/model_runner.py:82-83)
        greedy = [t <= 1e-5 for t in temps]
        self.bs = bs
        self.all_greedy = all(greedy)
        self.any_greedy = any(greedy)
        self.use_top_k = any(k < V for k in top_ks)
        self.use_top_p = any(p < 1.0 for p in top_ps)
        self.use_min_p = any(m > 0.0 for m in min_ps)
        self.max_top_k = max(top_ks) if self.use_top_k else 0
        self.use_penalties = any(s.uses_penalties for s in params)
        self.mass_rows = any(not g and not (0 < k <= self.fast_topk and k < V) for g, k in zip(greedy, top_ks))
        # dispatch order: rows with top-k off first (their workgroups cooperate), then
        # top-k rows by descending k, greedy rows last; results do not depend on it
        def kind(g: bool, k: int) -> int:
            if g:
                return 2
            return 1 if 0 < k < V and k <= self.fast_topk else 0

        rank = sorted((kind(g, k), 0 if g else -k, r) for r, (g, k) in enumerate(zip(greedy, top_ks)))
        order = np.array([r for _, _, r in rank], dtype=np.int32)
        if signature != self._order_sig:
            self._cp(self.row_order[:bs], order, torch.int32)
            self._order_sig = signature
        # history ids, padded with -1 (ignored by the sampler); only when some row uses penalties
        if histories is not None and self.use_penalties:
            if self.history is None:
                raise ValueError("SamplingBatch was built without history buffers (max_history=0)")
            H = self.max_history
            mat = np.full((bs, H), -1, dtype=np.int32)
            for r, h in enumerate(histories):
                tail = np.asarray(h[-H:], dtype=np.int64)
                mat[r, : tail.size] = tail
            self._cp(self.history[:bs], mat, torch.int32)
        # the step's uniforms: seeded rows are reproducible, the rest come from the host RNG
        u = self._rng.random(bs, dtype=np.float64).astype(np.float32)
        u = np.minimum(u, np.float32(np.nextafter(np.float32(1.0), np.float32(0.0))))
        seeded = np.array([s.seed is not None for s in params])
        if seeded.any():
            seeds = np.array([0 if s.seed is None else s.seed for s in params], dtype=np.uint64)
            u = np.where(seeded, seeded_uniforms(seeds, step), u)
        self._cp(self.uniforms[:bs], u.astype(np.float32), torch.float32)

    def sampler_kwargs(self, with_history: bool = True) -> dict:
        """Keyword arguments for ``BatchSampler.forward`` / ``sample_into`` (rows [:bs])."""
        bs = self.bs
        kw = dict(temperatures=self.temperatures[:bs], top_ps=self.top_ps[:bs], uniforms=self.uniforms[:bs],
                  all_greedy=self.all_greedy, use_top_p=self.use_top_p, row_order=self.row_order[:bs])
        if self.use_top_k:
            kw["top_ks"] = self.top_ks[:bs]
        if self.use_min_p:
            kw["min_ps"] = self.min_ps[:bs]
        if self.use_penalties:
            kw.update(repetition_penalties=self.repetition_penalties[:bs],
                      presence_penalties=self.presence_penalties[:bs],
                      frequency_penalties=self.frequency_penalties[:bs])
            if with_history and self.history is not None:
                kw["history"] = self.history[:bs]
        return kw
