"""ctypes front of the CPU oracle (oracle/contract.c) -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this module, to check results or as the timed CPU baseline.  The product
path never does.

The oracle restates src/compute/sampler.py:25-41 (with the staging rules of
src/data/batch.py:149-175) as the exact-integer contract documented at the top
of contract.c; the HIP kernels implement the same contract.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        lib.qso_sample.restype = ctypes.c_int
        lib.qso_sample.argtypes = [P, ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                   P, P, P, P, P, P, P, P, ctypes.c_int, P, P, P, P, ctypes.c_int]
        lib.qso_weight.restype = ctypes.c_uint64
        lib.qso_weight.argtypes = [ctypes.c_float, ctypes.c_float, ctypes.c_uint32, ctypes.c_int]
        lib.qso_shift.restype = ctypes.c_int
        lib.qso_shift.argtypes = [ctypes.c_int]
        lib.qso_ceil_scaled.restype = ctypes.c_uint64
        lib.qso_ceil_scaled.argtypes = [ctypes.c_float, ctypes.c_int]
        lib.qso_exp2_poly.restype = ctypes.c_float
        lib.qso_exp2_poly.argtypes = [ctypes.c_float]
        lib.qso_key.restype = ctypes.c_uint32
        lib.qso_key.argtypes = [ctypes.c_float]
        lib.qso_z_of_key.restype = ctypes.c_float
        lib.qso_z_of_key.argtypes = [ctypes.c_uint32]
        lib.qso_row_weights.restype = None
        lib.qso_row_weights.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_float, P, ctypes.c_int,
                                        ctypes.c_float, ctypes.c_float, ctypes.c_float, P, P, P, P]
        _lib = lib
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


@dataclass
class OracleResult:
    ids: np.ndarray        # int64 [B]
    probs: np.ndarray | None  # float32 [B, V] post-filter probabilities
    greedy_ids: np.ndarray  # int32 [B]
    kept: np.ndarray       # int32 [B] kept tokens with nonzero weight
    kend: np.ndarray       # int32 [B] size of the top-k set K
    pend: np.ndarray       # int32 [B] kept tokens (a prefix of K in order)
    kstar: np.ndarray      # uint32 [B] key of the row maximum q*
    kappa: np.ndarray      # uint32 [B] key of the last kept token
    W: list[int]           # exact kept mass per row
    S: list[int]           # exact mass of K per row


def sample(logits: np.ndarray, dtype: str, temperature, top_p=None, top_k=None, rep=None,
           pres=None, freq=None, history=None, uniforms=None, want_probs=False,
           threads: int | None = None, min_p=None) -> OracleResult:
    """Run the contract on [B, V] logits (float32, or uint16 bf16 bits)."""
    lib = _load()
    logits = np.ascontiguousarray(logits)
    B, V = logits.shape
    dt = 0 if dtype == "f32" else 1
    if dt == 0:
        assert logits.dtype == np.float32
    else:
        assert logits.dtype == np.uint16
    T = _c(temperature, np.float32)
    tp = _c(top_p, np.float32)
    tk = _c(top_k, np.int32)
    mp = _c(min_p, np.float32)
    rp, pp, fp = _c(rep, np.float32), _c(pres, np.float32), _c(freq, np.float32)
    hist = _c(history, np.int32)
    H = 0 if hist is None else hist.shape[1]
    u = _c(uniforms, np.float32)
    ids = np.zeros(B, dtype=np.int64)
    probs = np.zeros((B, V), dtype=np.float32) if want_probs else None
    info = np.zeros((B, 16), dtype=np.uint32)
    nt = threads if threads is not None else (os.cpu_count() or 1)
    rc = lib.qso_sample(_ptr(logits), dt, V, B, V, _ptr(T), _ptr(tp), _ptr(tk), _ptr(mp), _ptr(rp), _ptr(pp),
                        _ptr(fp), _ptr(hist), H, _ptr(u), _ptr(ids), _ptr(probs), _ptr(info), nt)
    if rc != 0:
        raise RuntimeError(f"oracle failed: {rc}")
    W = [int(info[r, 6]) | (int(info[r, 7]) << 32) for r in range(B)]
    S = [int(info[r, 8]) | (int(info[r, 9]) << 32) for r in range(B)]
    i32 = info.view(np.int32)
    return OracleResult(ids, probs, i32[:, 0].copy(), i32[:, 1].copy(), i32[:, 2].copy(), i32[:, 3].copy(),
                        info[:, 4].copy(), info[:, 5].copy(), W, S)


def sample_workload(w, step: int = 0, want_probs: bool = False, threads: int | None = None) -> OracleResult:
    return sample(w.logits, w.dtype, w.temperature, w.top_p, w.top_k, w.rep, w.pres, w.freq,
                  w.history, w.uniforms(step), want_probs=want_probs, threads=threads,
                  min_p=getattr(w, "min_p", None))


def shift(V: int) -> int:
    """SH of the weight rule: the row maximum weighs 2**(23 + SH)."""
    return int(_load().qso_shift(int(V)))


def weight(q: float, qstar: float, V: int) -> int:
    """The contract weight of q in a row whose maximum is qstar (rule R3)."""
    lib = _load()
    return int(lib.qso_weight(float(q), float(qstar), key(qstar), shift(V)))


def weights(q: np.ndarray, V: int) -> np.ndarray:
    """Contract weights of a row of q values (its maximum taken from the row)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    ks = max(key(float(v)) for v in q)
    qs = z_of_key(ks)
    lib = _load()
    SH = shift(V)
    return np.array([lib.qso_weight(float(v), qs, ks, SH) for v in q], dtype=np.uint64)


def ceil_scaled(f: float, e: int) -> int:
    """ceil(f * 2**e) for an fp32 f in [0, 1]."""
    return int(_load().qso_ceil_scaled(float(f), int(e)))


def exp2_poly(f: float) -> float:
    return float(_load().qso_exp2_poly(float(f)))


def key(z: float) -> int:
    return int(_load().qso_key(float(z)))


def z_of_key(k: int) -> float:
    return float(_load().qso_z_of_key(int(k)))


def row_weights(row: np.ndarray, dtype: str, temperature: float, history=None, rep=1.0, pres=0.0, freq=0.0):
    """Per-token (z, q, key(q), w) after penalties and temperature, as the contract defines them."""
    lib = _load()
    row = np.ascontiguousarray(row)
    V = row.shape[0]
    hist = _c(history, np.int32)
    k = np.zeros(V, np.uint32)
    z = np.zeros(V, np.float32)
    q = np.zeros(V, np.float32)
    w = np.zeros(V, np.uint64)
    lib.qso_row_weights(_ptr(row), 0 if dtype == "f32" else 1, V, float(temperature), _ptr(hist),
                        0 if hist is None else hist.size, float(rep), float(pres), float(freq),
                        _ptr(k), _ptr(z), _ptr(q), _ptr(w))
    return z, q, k, w
