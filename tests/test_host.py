"""Host-side logic on the CPU: parameter validation and staging, the seeded
uniforms, the synthetic workloads, the C ABI's exported symbols and the bench
contract.  Mirrors the reference's host test for the sampling parameters
(tests/test_host.py:47-50 in the reference)."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from qedge_amd import workloads as W
from qedge_amd.batch import SamplingBatch, seeded_uniforms
from qedge_amd.sampling_params import SamplingParams

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# ---------------------------------------------------------------- SamplingParams


@pytest.mark.parametrize("kwargs", [{"top_p": 0}, {"top_p": 1.1}, {"min_p": -0.1},
                                    {"min_tokens": 3, "max_tokens": 2}, {"temperature": -1}, {"top_k": 0}])
def test_sampling_rejects_like_the_reference(kwargs):
    with pytest.raises(ValueError):
        SamplingParams(**kwargs)


@pytest.mark.parametrize("kwargs", [{"repetition_penalty": 0.0}, {"repetition_penalty": -1.0},
                                    {"repetition_penalty": float("inf")}, {"presence_penalty": float("nan")},
                                    {"frequency_penalty": float("inf")}, {"seed": -1}])
def test_sampling_rejects_bad_extensions(kwargs):
    with pytest.raises(ValueError):
        SamplingParams(**kwargs)


def test_sampling_defaults_are_greedy_and_penalty_free():
    p = SamplingParams()
    assert p.greedy and not p.uses_penalties
    assert SamplingParams(temperature=1e-6).greedy and not SamplingParams(temperature=0.5).greedy


# ---------------------------------------------------------------- SamplingBatch


def test_batch_normalises_like_the_reference():
    V = 1000
    b = SamplingBatch(8, V, torch.device("cpu"), max_history=4)
    params = [SamplingParams(), SamplingParams(temperature=0.7, top_p=0.9, top_k=50),
              SamplingParams(temperature=1.0, top_k=-3), SamplingParams(temperature=0.5, top_k=5000, min_p=0.1),
              SamplingParams(temperature=0.8, repetition_penalty=1.1, seed=7)]
    b.fill(params, histories=[[1, 2], [], [3], [4, 5, 6, 7, 8], [9]])
    bs = len(params)
    np.testing.assert_array_equal(b.top_ks[:bs].numpy(), [V, 50, V, V, V])  # None/<=0 -> V, min(k, V)
    np.testing.assert_allclose(b.top_ps[:bs].numpy(), [1.0, 0.9, 1.0, 1.0, 1.0], rtol=0, atol=1e-7)
    np.testing.assert_allclose(b.min_ps[:bs].numpy(), [0, 0, 0, 0.1, 0], atol=1e-7)
    assert not b.all_greedy and b.any_greedy and b.use_top_k and b.use_top_p and b.use_min_p
    assert b.use_penalties and b.max_top_k == V
    assert b.mass_rows  # rows with top-k off need the mass path
    hist = b.history[:bs].numpy()
    np.testing.assert_array_equal(hist[3], [5, 6, 7, 8])  # the most recent H ids
    np.testing.assert_array_equal(hist[1], [-1, -1, -1, -1])
    u = b.uniforms[:bs].numpy()
    assert np.all((u >= 0) & (u < 1))
    assert u[4] == seeded_uniforms(np.array([7], np.uint64), 0)[0]
    kw = b.sampler_kwargs()
    assert kw["history"].shape == (bs, 4) and kw["min_ps"].shape == (bs,)
    # dispatch order: top-k-off rows first, then top-k rows by descending k, greedy rows last
    np.testing.assert_array_equal(b.row_order[:bs].numpy(), [2, 3, 4, 1, 0])


def test_batch_flags_for_fast_topk_batches():
    b = SamplingBatch(4, 248320, torch.device("cpu"))
    b.fill([SamplingParams(temperature=0.7, top_k=20, top_p=0.8), SamplingParams()])
    assert not b.mass_rows and not b.all_greedy and b.use_top_p
    b.fill([SamplingParams(), SamplingParams(temperature=0.0, top_p=0.5)])
    assert b.all_greedy


def test_seeded_uniforms_reproducible_and_in_range():
    seeds = np.arange(1000, dtype=np.uint64)
    a = seeded_uniforms(seeds, 3)
    b = seeded_uniforms(seeds, 3)
    c = seeded_uniforms(seeds, 4)
    np.testing.assert_array_equal(a, b)
    assert np.mean(a != c) > 0.99
    assert np.all((a >= 0) & (a < 1)) and a.dtype == np.float32
    assert abs(a.mean() - 0.5) < 0.05
    assert np.all(np.round(a * 2**24) == a * 2**24)  # 24 random bits, exact in fp32


# ---------------------------------------------------------------- workloads


def test_workloads_shapes_and_planted_structure():
    w = W.make("greedy_spikes_f32")
    assert w.logits.shape == (2, W.VOCAB) and w.logits.dtype == np.float32
    spikes = w.notes["spikes"]
    assert len(spikes) == 5 and np.all(w.logits[0][spikes] == 12.0)
    assert w.temperature[0] == 0 and w.temperature[1] == 1.0
    meta = W.make("hetero_b64_bf16", rows=[0], V=4096)
    assert len(meta.notes["topk_off_rows"]) == 6 and len(meta.notes["greedy_rows"]) == 6
    w3 = W.make("hetero_b64_bf16", rows=meta.notes["topk_off_rows"], V=4096)
    assert np.all(w3.top_k == 0) and w3.mass_rows
    w2 = W.make("topk_topp_rep_bf16", V=4096)
    assert w2.logits.dtype == np.uint16 and w2.history.shape == (1, 2048) and not w2.mass_rows


def test_workload_rows_are_independent_streams():
    full = W.make("penalties_b256_bf16", rows=[0, 5, 9], V=2048)
    one = W.make("penalties_b256_bf16", rows=[5], V=2048)
    np.testing.assert_array_equal(full.logits[1], one.logits[0])
    np.testing.assert_array_equal(full.history[1], one.history[0])


def test_bf16_rounding_is_nearest_even():
    x = np.array([1.0, 1.00390625, 1.005859375, -2.5, 3.0e38, np.inf], np.float32)
    b = W.bf16_bits(x)
    back = W.bf16_to_f32(b)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(back, ref)


def test_algorithmic_bytes_match_the_metric_definition():
    w = W.make("hetero_b64_bf16", rows=[0], V=1024)
    assert w.algorithmic_bytes() == 1024 * 2 + 36


# ---------------------------------------------------------------- C ABI


def _header_functions():
    text = open(os.path.join(ROOT, "include", "qsampler.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qs_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    from qedge_amd import _lib

    lib = _lib.load()
    names = _header_functions()
    assert {"qs_sample", "qs_argmax", "qs_workspace_bytes", "qs_workspace_init"} <= set(names)
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.EXPORTS
    assert lib.qs_version() >= 200


def test_workspace_size_grows_with_batch_only():
    from qedge_amd import _lib

    lib = _lib.load()
    a = lib.qs_workspace_bytes(1, 248320, 1, 0)
    b = lib.qs_workspace_bytes(64, 248320, 1, 0)
    c = lib.qs_workspace_bytes(64, 248320, 0, 4096)
    assert 0 < a < b == c
    assert a % 256 == 0 and b % 256 == 0
    assert lib.qs_workspace_bytes(1, 0, 1, 0) == 0


def test_argument_errors_are_reported_without_a_gpu():
    from qedge_amd import _lib

    lib = _lib.load()
    P = ctypes.c_void_p
    # null workspace / bad dtype / bad shape: rejected before any launch
    def call(stride=100, dtype=0, T=P(1), hist=None, H=0, flags=0, ws_bytes=1 << 20, B=1, V=100):
        return lib.qs_sample(P(1), stride, dtype, B, V, T, None, None, None, None, None, None, hist, H, None,
                             P(1), None, flags, P(1), None, None, P(256), ws_bytes, None)

    assert call(dtype=7) < 0 and b"dtype" in lib.qs_last_error()
    assert call(stride=50) < 0 and b"row_stride" in lib.qs_last_error()
    assert call(hist=P(1), H=70000) < 0 and b"history" in lib.qs_last_error()
    assert call(hist=None, H=5) < 0 and b"hist_ids" in lib.qs_last_error()
    assert call(T=None) < 0 and b"temperature" in lib.qs_last_error()
    assert call(flags=1 << 9) < 0 and b"flags" in lib.qs_last_error()
    assert call(ws_bytes=1024) < 0 and b"workspace" in lib.qs_last_error()
    assert call(B=0) == 0  # an empty batch is a no-op


# ---------------------------------------------------------------- bench contract


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
