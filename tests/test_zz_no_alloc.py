"""GPU test of qs_sample_static, the entry point that allocates nothing (its
scratch is the library's own device array): through the C ABI, two calls in a
row (the second with a smaller batch) must give exactly what qs_sample gives
with a caller workspace on the same inputs.  Needs an MI355X."""
import ctypes

import numpy as np
import pytest
import torch

from qedge_amd import _lib
from qedge_amd import workloads as W
from qedge_amd.sampler import Workspace, sample_into
from tests.devrun import to_device

pytestmark = pytest.mark.gpu


def _static_call(lib, d, B, V, u, ids, probs, kept, stream):
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    lg = d["logits"]
    H = 0 if d["history"] is None else d["history"].shape[1]
    return lib.qs_sample_static(
        p(lg), lg.stride(0), _lib.QS_DTYPE_BF16 if lg.dtype == torch.bfloat16 else _lib.QS_DTYPE_F32, B, V,
        p(d["temperatures"]), p(d["top_ps"]), p(d["top_ks"]), None,
        p(d["repetition_penalties"]), p(d["presence_penalties"]), p(d["frequency_penalties"]),
        p(d["history"]), H, None, p(u), None, _lib.QS_FLAG_USE_TOP_P, p(ids), p(probs), p(kept),
        ctypes.c_void_p(stream))


@pytest.mark.parametrize("first,second", [("hetero_b64_bf16", "topk_topp_rep_bf16")])
def test_static_scratch_entry_matches_workspace_entry(gpu, first, second):
    lib = _lib.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    for name, rows in ((first, None), (second, None), (first, list(range(0, 64, 9)))):
        w = W.make(name, rows=rows)
        d = to_device(w, gpu)
        B, V = d["logits"].shape
        H = 0 if d["history"] is None else d["history"].shape[1]
        u = torch.from_numpy(w.uniforms(0)).to(gpu)
        ids_s = torch.full((B,), -1, dtype=torch.int64, device=gpu)
        probs_s = torch.empty((B, V), dtype=torch.float32, device=gpu)
        kept_s = torch.empty(B, dtype=torch.int32, device=gpu)
        rc = _static_call(lib, d, B, V, u, ids_s, probs_s, kept_s, stream)
        assert rc == 0, lib.qs_last_error().decode()
        ws = Workspace(B, V, d["logits"].dtype, H, gpu)
        ids_w = torch.empty(B, dtype=torch.int64, device=gpu)
        probs_w = torch.empty((B, V), dtype=torch.float32, device=gpu)
        kept_w = torch.empty(B, dtype=torch.int32, device=gpu)
        lg = d.pop("logits")
        sample_into(lg, ids_w, ws, uniforms=u, use_top_p=True, out_probs=probs_w, out_kept=kept_w, **d)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(ids_s.cpu().numpy(), ids_w.cpu().numpy())
        np.testing.assert_array_equal(kept_s.cpu().numpy(), kept_w.cpu().numpy())
        np.testing.assert_array_equal(probs_s.cpu().numpy(), probs_w.cpu().numpy())


def test_static_scratch_rejects_batches_beyond_it(gpu):
    lib = _lib.load()
    V = 248320
    limit = int(lib.qs_static_scratch_bytes())
    B = 1
    while lib.qs_workspace_bytes(B, V, _lib.QS_DTYPE_BF16, 0) <= limit:
        B *= 2
    x = torch.zeros((B, V), dtype=torch.bfloat16, device=gpu)
    T = torch.ones(B, dtype=torch.float32, device=gpu)
    ids = torch.empty(B, dtype=torch.int64, device=gpu)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = lib.qs_sample_static(p(x), V, _lib.QS_DTYPE_BF16, B, V, p(T), None, None, None, None, None, None, None, 0,
                              None, None, None, 0, p(ids), None, None,
                              ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream))
    assert rc != 0 and b"static scratch" in lib.qs_last_error()
