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
    min_p: float | None = None        # validated and staged, not applied (as in the reference)
    max_tokens: int = 128
    min_tokens: int = 0
    ignore_eos: bool = False
    # extensions
    repetition_penalty: float = 1.0   # z / rp for z > 0, z * rp otherwise, on tokens in the history
    presence_penalty: float = 0.0     # subtracted once from tokens in the history
    frequency_penalty: float = 0.0    # subtracted per occurrence in the history
    seed: int | None = None           # seeds the host uniform of every step

    def __post_init__(self) -> None:
        # src/sampling_params.py:16-30
        if self.max_tokens < 0:
            raise ValueError(f"max_tokens must be >= 0, got {self.max_tokens}")
        if self.min_tokens < 0:
            raise ValueError(f"min_tokens must be >= 0, got {self.min_tokens}")
        if self.min_tokens > self.max_tokens:
            raise ValueError("min_tokens must not exceed max_tokens")
        if self.temperature < 0:
            raise ValueError(f"temperature must be >= 0, got {self.temperature}")
        if self.top_p is not None and not (0.0 < self.top_p <= 1.0):
            raise ValueError(f"top_p must be in (0, 1], got {self.top_p}")
        if self.top_k is not None and self.top_k == 0:
            raise ValueError("top_k=0 is invalid; use None to disable")
        if self.min_p is not None and not (0.0 <= self.min_p <= 1.0):
            raise ValueError(f"min_p must be in [0, 1], got {self.min_p}")
        if not (math.isfinite(self.repetition_penalty) and self.repetition_penalty > 0.0):
            raise ValueError(f"repetition_penalty must be finite and > 0, got {self.repetition_penalty}")
        if not math.isfinite(self.presence_penalty):
            raise ValueError(f"presence_penalty must be finite, got {self.presence_penalty}")
        if not math.isfinite(self.frequency_penalty):
            raise ValueError(f"frequency_penalty must be finite, got {self.frequency_penalty}")
        if self.seed is not None and not (0 <= self.seed < 2**63):
            raise ValueError(f"seed must be in [0, 2**63), got {self.seed}")

    @property
    def greedy(self) -> bool:
        return self.temperature <= 1e-5

    @property
    def uses_penalties(self) -> bool:
        return self.repetition_penalty != 1.0 or self.presence_penalty != 0.0 or self.frequency_penalty != 0.0
