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
                                   P, P, P, P, P, P, P, ctypes.c_int, P, P, P, P, ctypes.c_int]
        lib.qso_detexp.restype = None
        lib.qso_detexp.argtypes = [P, ctypes.c_int, P, P]
        lib.qso_exp2_poly.restype = ctypes.c_float
        lib.qso_exp2_poly.argtypes = [ctypes.c_float]
        lib.qso_key.restype = ctypes.c_uint32
        lib.qso_key.argtypes = [ctypes.c_float]
        lib.qso_z_of_key.restype = ctypes.c_float
        lib.qso_z_of_key.argtypes = [ctypes.c_uint32]
        lib.qso_row_weights.restype = None
        lib.qso_row_weights.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_float, P, ctypes.c_int,
                                        ctypes.c_float, ctypes.c_float, ctypes.c_float, P, P, P, P, P]
        lib.qso_u128_to_double.restype = ctypes.c_double
        lib.qso_u128_to_double.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
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
    n_max: np.ndarray      # int32 [B] row scale N
    kept: np.ndarray       # int32 [B] kept tokens with nonzero weight
    topk_end: np.ndarray   # int32 [B]
    W: list[int]           # exact kept mass per row


def sample(logits: np.ndarray, dtype: str, temperature, top_p=None, top_k=None, rep=None,
           pres=None, freq=None, history=None, uniforms=None, want_probs=False,
           threads: int | None = None) -> OracleResult:
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
    rp, pp, fp = _c(rep, np.float32), _c(pres, np.float32), _c(freq, np.float32)
    hist = _c(history, np.int32)
    H = 0 if hist is None else hist.shape[1]
    u = _c(uniforms, np.float32)
    ids = np.zeros(B, dtype=np.int64)
    probs = np.zeros((B, V), dtype=np.float32) if want_probs else None
    info = np.zeros((B, 8), dtype=np.int32)
    nt = threads if threads is not None else (os.cpu_count() or 1)
    rc = lib.qso_sample(_ptr(logits), dt, V, B, V, _ptr(T), _ptr(tp), _ptr(tk), _ptr(rp), _ptr(pp), _ptr(fp),
                        _ptr(hist), H, _ptr(u), _ptr(ids), _ptr(probs), _ptr(info), nt)
    if rc != 0:
        raise RuntimeError(f"oracle failed: {rc}")
    iu = info.view(np.uint32)
    W = [int(iu[r, 4]) | (int(iu[r, 5]) << 32) | (int(iu[r, 6]) << 64) | (int(iu[r, 7]) << 96)
         for r in range(B)]
    return OracleResult(ids, probs, info[:, 0].copy(), info[:, 1].copy(), info[:, 2].copy(),
                        info[:, 3].copy(), W)


def sample_workload(w, step: int = 0, want_probs: bool = False, threads: int | None = None) -> OracleResult:
    return sample(w.logits, w.dtype, w.temperature, w.top_p, w.top_k, w.rep, w.pres, w.freq,
                  w.history, w.uniforms(step), want_probs=want_probs, threads=threads)


def detexp(q: np.ndarray):
    """(n, M) with exp(q) ~= M * 2**(n-23), per the contract's weight rule."""
    lib = _load()
    q = np.ascontiguousarray(q, dtype=np.float32)
    n = np.zeros(q.size, np.int32)
    m = np.zeros(q.size, np.uint32)
    lib.qso_detexp(_ptr(q), q.size, _ptr(n), _ptr(m))
    return n, m


def exp2_poly(f: float) -> float:
    return float(_load().qso_exp2_poly(float(f)))


def key(z: float) -> int:
    return int(_load().qso_key(float(z)))


def z_of_key(k: int) -> float:
    return float(_load().qso_z_of_key(int(k)))


def row_weights(row: np.ndarray, dtype: str, temperature: float, history=None, rep=1.0, pres=0.0, freq=0.0):
    """Per-token (z, q, key(q), n, M) after penalties and temperature, as the contract defines them."""
    lib = _load()
    row = np.ascontiguousarray(row)
    V = row.shape[0]
    hist = _c(history, np.int32)
    n = np.zeros(V, np.int32)
    m = np.zeros(V, np.uint32)
    k = np.zeros(V, np.uint32)
    z = np.zeros(V, np.float32)
    q = np.zeros(V, np.float32)
    lib.qso_row_weights(_ptr(row), 0 if dtype == "f32" else 1, V, float(temperature), _ptr(hist),
                        0 if hist is None else hist.size, float(rep), float(pres), float(freq),
                        _ptr(n), _ptr(m), _ptr(k), _ptr(z), _ptr(q))
    return z, q, k, n, m


def u128_to_double(x: int) -> float:
    return float(_load().qso_u128_to_double(x & ((1 << 64) - 1), x >> 64))
