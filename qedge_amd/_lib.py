"""ctypes binding of qedge_amd/libqsampler.so (declarations: include/qsampler.h).

The library must be built (``python -m qedge_amd.build``); loading fails loudly
otherwise -- there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  -- loads the HIP runtime the library binds to

from .build import OUT as LIB_PATH

QS_DTYPE_F32 = 0
QS_DTYPE_BF16 = 1
QS_FLAG_ALL_GREEDY = 1
QS_FLAG_USE_TOP_P = 2
QS_FLAG_NO_WAIT = 4
QS_FLAG_SOLO = 8
QS_TOPK_FAST_MAX = 1024
QS_MAX_HISTORY = 65535

EXPORTS = ("qs_version", "qs_last_error", "qs_workspace_bytes", "qs_workspace_init", "qs_sample", "qs_argmax",
           "qs_history_append", "qs_step_finish", "qs_sample_static", "qs_static_scratch_bytes")

_lib = None


class SamplerError(RuntimeError):
    pass


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise SamplerError(f"{LIB_PATH} is missing: build it with `python -m qedge_amd.build`")
    lib = ctypes.CDLL(LIB_PATH)
    P, I, I64, U32, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint32, ctypes.c_size_t
    lib.qs_version.restype = I
    lib.qs_version.argtypes = []
    lib.qs_last_error.restype = ctypes.c_char_p
    lib.qs_last_error.argtypes = []
    lib.qs_workspace_bytes.restype = SZ
    lib.qs_workspace_bytes.argtypes = [I, I, I, I]
    lib.qs_workspace_init.restype = I
    lib.qs_workspace_init.argtypes = [P, SZ, P]
    lib.qs_sample.restype = I
    lib.qs_sample.argtypes = [P, I64, I, I, I,          # logits, row_stride, dtype, B, V
                              P, P, P, P,               # temperature, top_p, top_k, min_p
                              P, P, P,                  # rep, pres, freq
                              P, I, P,                  # hist_ids, H, hist_len
                              P, P, U32,                # uniforms, row_order, flags
                              P, P, P,                  # out_ids, out_probs, out_kept
                              P, SZ, P]                 # workspace, bytes, stream
    lib.qs_argmax.restype = I
    lib.qs_argmax.argtypes = [P, I64, I, I, I, P, P, SZ, P]
    lib.qs_sample_static.restype = I
    lib.qs_sample_static.argtypes = lib.qs_sample.argtypes[:-3] + [P]  # no workspace: the library's scratch
    lib.qs_static_scratch_bytes.restype = SZ
    lib.qs_static_scratch_bytes.argtypes = []
    lib.qs_step_finish.restype = I
    lib.qs_step_finish.argtypes = [P, I, P, P, I,            # ids, B, slots, pending, n_pending
                                   P, P, P, P, I64,          # num_generated, min, max, ignore_eos, eos_id
                                   P, P, P]                  # finished, host_ids, stream
    lib.qs_history_append.restype = I
    lib.qs_history_append.argtypes = [P, I, I, P, P, P, P]   # hist, B, H, hist_len, ids, active, stream
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != 0:
        raise SamplerError(load().qs_last_error().decode() or f"qsampler error {rc}")
