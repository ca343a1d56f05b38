"""Derivation of the exp2 polynomial of the sampling contract -- TEST INFRASTRUCTURE.

The contract's weight rule evaluates 2^f for f in [0, 1) as a degree-6
polynomial with c0 = 1 in fp32 fused multiply-adds (oracle/contract.c QS_P2,
qedge_amd/csrc/qs_device.hpp).  The coefficients c1..c6 come from this fit:

  * 4097 Chebyshev nodes on [0, 1];
  * least squares on the relative error (2^f - 1 - sum c_j f^j) / 2^f, with
    c0 = 1 held fixed so that 2^0 is exactly 1 (the row maximum's weight is
    then exactly a power of two);
  * 60 rounds of reweighting that raise the weight of nodes in proportion to
    their error, which drives the fit toward equal-ripple (minimax) error;
  * each coefficient rounded to the nearest fp32.

Run as a script it prints the coefficients as C hex-float literals.  The test
suite re-runs the fit and checks the committed coefficients against it.
"""
from __future__ import annotations

import numpy as np


def fit(degree: int = 6, nodes: int = 4097, rounds: int = 60) -> list[float]:
    k = np.arange(nodes)
    x = 0.5 - 0.5 * np.cos(np.pi * (k + 0.5) / nodes)
    y = np.exp2(x)
    A = np.stack([x ** j for j in range(1, degree + 1)], axis=1) / y[:, None]
    b = (y - 1.0) / y
    w = np.ones(nodes)
    c = np.zeros(degree)
    for _ in range(rounds):
        c, *_ = np.linalg.lstsq(A * w[:, None], b * w, rcond=None)
        e = np.abs(A @ c - b)
        w = w * (1.0 + e / e.max())
        w /= w.max()
    return [1.0] + [float(np.float32(v)) for v in c]


def horner_f32(coef: list[float], f: np.ndarray) -> np.ndarray:
    """fp32 Horner with a fused multiply-add per step (exact product, one rounding)."""
    f = np.asarray(f, dtype=np.float32).astype(np.float64)
    p = np.full(f.shape, np.float32(coef[-1]), dtype=np.float32)
    for c in reversed(coef[:-1]):
        p = (p.astype(np.float64) * f + np.float64(np.float32(c))).astype(np.float32)
    return p


if __name__ == "__main__":
    for c in fit():
        print(float(np.float32(c)).hex())
