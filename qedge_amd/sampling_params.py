"""Per-request sampling parameters.

Mirrors ``SamplingParams`` (src/sampling_params.py:6-30): the same fields,
defaults and validation errors (``ValueError``), plus the sampler's extensions:
history penalties (repetition, presence, frequency) and a per-request seed for
the host uniforms the draw consumes.
"""
from __future__ import annotations

import math
from dataclasses import dataclass


@dataclass
class SamplingParams:
    temperature: float = 0.0          # <= 1e-5 means greedy (src/compute/sampler.py:30)
    top_p: float | None = None        # None: off (src/data/batch.py:153)
    top_k: int | None = None          # None: off; 0 is rejected (src/sampling_params.py:27-28)
    min_p: float | None = None        # None: off; keeps p >= min_p * p_max (staged as in src/data/batch.py:158)
    max_tokens: int = 128
    min_tokens: int = 0
    ignore_eos: bool = False
    # extensions
    repetition_penalty: float = 1.0   # z / rp for z > 0, z * rp otherwise, on tokens in the history
    presence_penalty: float = 0.0     # subtracted once from tokens in the history
    frequency_penalty: float = 0.0    # subtracted per occurrence in the history
    seed: int | None = None           # seeds the host uniform of every step

    def __post_init__(self) -> None:
        # the same accepted domain as src/sampling_params.py:16-30
        if self.max_tokens < 0:
            raise ValueError(f"SamplingParams: max_tokens={self.max_tokens} is negative")
        if self.min_tokens < 0:
            raise ValueError(f"SamplingParams: min_tokens={self.min_tokens} is negative")
        if self.min_tokens > self.max_tokens:
            raise ValueError(f"SamplingParams: min_tokens={self.min_tokens} is above max_tokens={self.max_tokens}")
        if self.temperature < 0:
            raise ValueError(f"SamplingParams: temperature={self.temperature} is negative")
        if self.top_p is not None and not (0.0 < self.top_p <= 1.0):
            raise ValueError(f"SamplingParams: top_p={self.top_p} lies outside (0, 1]")
        if self.top_k is not None and self.top_k == 0:
            raise ValueError("SamplingParams: top_k=0 is not accepted (None turns top-k off)")
        if self.min_p is not None and not (0.0 <= self.min_p <= 1.0):
            raise ValueError(f"SamplingParams: min_p={self.min_p} lies outside [0, 1]")
        if not (math.isfinite(self.repetition_penalty) and self.repetition_penalty > 0.0):
            raise ValueError(f"SamplingParams: repetition_penalty={self.repetition_penalty} is not a positive number")
        if not math.isfinite(self.presence_penalty):
            raise ValueError(f"SamplingParams: presence_penalty={self.presence_penalty} is not finite")
        if not math.isfinite(self.frequency_penalty):
            raise ValueError(f"SamplingParams: frequency_penalty={self.frequency_penalty} is not finite")
        if self.seed is not None and not (0 <= self.seed < 2**63):
            raise ValueError(f"SamplingParams: seed={self.seed} lies outside [0, 2**63)")

    @property
    def greedy(self) -> bool:
        return self.temperature <= 1e-5

    @property
    def uses_penalties(self) -> bool:
        return self.repetition_penalty != 1.0 or self.presence_penalty != 0.0 or self.frequency_penalty != 0.0
