"""Pins the CPU oracle (oracle/contract.c) against closed forms, library routines
and the reference's own rules, so the GPU parity tests compare against a
trustworthy checker.  CPU only.

What each rule is checked against:
  weights exp(q)        float64 math.exp (closed form)
  orderable keys        numpy float ordering, NaN lowest, -0 == +0
  greedy                torch.argmax (first maximum, NaN is maximum)
  post-filter probs     float64 softmax over the kept set
  top-k set             torch.topk's k-th value, ties kept
  top-p set             the reference rule (src/compute/sampler.py:35-37) in
                        float64 on the same q; and torch's own fp32 pipeline
  draw                  the inverse-CDF measure of every id over a fine u grid;
                        chi-square against torch.multinomial
  penalties             transformers' RepetitionPenaltyLogitsProcessor; numpy
                        closed forms for presence / frequency
"""
import math

import numpy as np
import pytest
import torch

from oracle import contract, torch_ref
from qedge_amd import workloads as W


def _row_problem(rng, V, dtype="f32", scale=2.0, ties=False):
    x = rng.standard_normal(V).astype(np.float32) * np.float32(scale)
    if ties:
        x = np.round(x * 4) / 4
        x = x.astype(np.float32)
    if dtype == "bf16":
        return W.bf16_bits(x)
    return x


def _f32(logits, dtype):
    return logits if dtype == "f32" else W.bf16_to_f32(logits)


# ---------------------------------------------------------------- weights


def test_exp2_poly_close_to_exp2():
    f = np.linspace(0.0, 1.0, 4001, endpoint=False).astype(np.float32)
    got = np.array([contract.exp2_poly(float(v)) for v in f])
    ref = np.exp2(f.astype(np.float64))
    assert np.max(np.abs(got - ref) / ref) < 1.5e-7


def test_weights_close_to_exp():
    q = np.concatenate([np.linspace(-80, 80, 20001), [0.0, -0.0, 1e-30, -1e-30, 88.0, -87.0]]).astype(np.float32)
    n, m = contract.detexp(q)
    val = m.astype(np.float64) * np.exp2(n.astype(np.float64) - 23.0)
    ref = np.exp(q.astype(np.float64))
    assert np.all((m >= 1 << 23) & (m < 1 << 24))
    assert np.max(np.abs(val - ref) / ref) < 2e-7


# ---------------------------------------------------------------- keys


def test_keys_order_like_floats():
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10,
                           np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40, 3.4e38, -3.4e38], np.float32)])
    keys = np.array([contract.key(float(v)) for v in vals], dtype=np.uint64)
    order_k = np.lexsort((np.arange(vals.size), keys))
    srt = vals[order_k]
    assert np.all(np.diff(srt.astype(np.float64)) >= 0)
    assert contract.key(0.0) == contract.key(-0.0)
    assert contract.key(float("nan")) == 0
    assert contract.key(float("-inf")) > 0
    for v in vals[:200]:
        if v != 0:
            assert contract.z_of_key(contract.key(float(v))) == v


# ---------------------------------------------------------------- greedy


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_greedy_is_torch_argmax(dtype):
    rng = np.random.default_rng(2)
    B, V = 24, 517
    rows = []
    for r in range(B):
        x = rng.standard_normal(V).astype(np.float32)
        if r % 3 == 0:
            x[rng.integers(0, V, 4)] = x.max() + 1  # tied maxima
        if r % 5 == 1:
            x[rng.integers(0, V, 2)] = np.nan
        rows.append(W.bf16_bits(x) if dtype == "bf16" else x)
    logits = np.stack(rows)
    res = contract.sample(logits, dtype, np.zeros(B, np.float32))
    ref = torch.from_numpy(_f32(logits, dtype)).argmax(dim=-1).numpy()
    np.testing.assert_array_equal(res.ids, ref)


# ---------------------------------------------------------------- probabilities


def _kept_mask(res):
    return res.probs > 0


def test_probs_are_softmax_of_q():
    rng = np.random.default_rng(3)
    B, V = 16, 700
    logits = np.stack([_row_problem(rng, V, scale=3.0) for _ in range(B)])
    T = rng.uniform(0.2, 1.5, B).astype(np.float32)
    res = contract.sample(logits, "f32", T, uniforms=rng.random(B).astype(np.float32), want_probs=True)
    for r in range(B):
        q = (logits[r] / T[r]).astype(np.float32).astype(np.float64)
        p = np.exp(q - q.max())
        p /= p.sum()
        p[p < 2.0 ** -41] = 0.0  # below the 40-octave window the contract gives weight 0
        np.testing.assert_allclose(res.probs[r], p, rtol=3e-7, atol=1e-12)


# ---------------------------------------------------------------- top-k


def test_topk_set_matches_torch_topk():
    rng = np.random.default_rng(4)
    B, V = 40, 333
    logits = np.stack([_row_problem(rng, V, dtype="bf16", ties=True) for _ in range(B)])
    T = rng.uniform(0.3, 1.2, B).astype(np.float32)
    K = rng.integers(1, V, B).astype(np.int32)
    res = contract.sample(logits, "bf16", T, top_k=K, uniforms=rng.random(B).astype(np.float32),
                          want_probs=True)
    z = _f32(logits, "bf16")
    for r in range(B):
        q = torch.from_numpy((z[r] / T[r]).astype(np.float32))
        kth = torch.topk(q, int(K[r])).values[-1]
        want = (q >= kth).numpy()
        assert res.topk_end[r] == want.sum()
        got = res.probs[r] > 0
        # every top-k token inside the 40-octave weight window survives, nothing else
        y = q.numpy().astype(np.float64) * (1.0 / math.log(2.0))
        in_window = np.floor(y) >= math.floor(y.max()) - 40
        np.testing.assert_array_equal(got, want & in_window)


# ---------------------------------------------------------------- top-p


def _exact_topp(q, top_p):
    """The reference rule (src/compute/sampler.py:35-37) in float64 on the same q."""
    q64 = q.astype(np.float64)
    p = np.exp(q64 - q64.max())
    p /= p.sum()
    order = np.lexsort((np.arange(q.size), -q64))
    ps = p[order]
    excl = np.cumsum(ps) - ps
    kept = np.zeros(q.size, bool)
    kept[order[excl <= top_p]] = True
    ex = np.empty_like(excl)
    ex[order] = excl
    return kept, ex


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_topp_set_is_the_reference_rule(dtype):
    rng = np.random.default_rng(5)
    B, V = 48, 600
    logits = np.stack([_row_problem(rng, V, dtype=dtype, scale=rng.uniform(0.05, 4.0)) for _ in range(B)])
    T = rng.uniform(0.2, 1.5, B).astype(np.float32)
    P = rng.uniform(0.05, 0.999, B).astype(np.float32)
    res = contract.sample(logits, dtype, T, top_p=P, uniforms=rng.random(B).astype(np.float32),
                          want_probs=True)
    z = _f32(logits, dtype)
    near = 0
    for r in range(B):
        q = (z[r] / T[r]).astype(np.float32)
        want, excl = _exact_topp(q, float(P[r]))
        got = res.probs[r] > 0
        diff = np.nonzero(got != (want & (np.exp(q.astype(np.float64) - q.max()) > 2.0 ** -41)))[0]
        # the only admissible differences: exclusive mass within the weights' error of top_p
        assert np.all(np.abs(excl[diff] - P[r]) < 1e-6), (r, diff[:5], excl[diff][:5] - P[r])
        near += diff.size
    assert near <= 2


def test_topp_against_torch_pipeline_on_workloads():
    """Differences from torch's own fp32 softmax/cumsum are explained by its rounding."""
    for name, rows in [("hetero_b64_bf16", list(range(0, 64, 9))), ("penalties_b256_bf16", [0, 1]),
                       ("flat_topp_b1024_f32", [0, 1]), ("topk_topp_rep_bf16", None)]:
        w = W.make(name, rows=rows)
        ref = contract.sample_workload(w, want_probs=True)
        t = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dt)
        st = torch_ref.filter_rows(torch.from_numpy(w.logits_f32()), t(w.temperature, torch.float32),
                                   t(w.top_p, torch.float32), t(w.top_k, torch.int32), t(w.rep, torch.float32),
                                   t(w.pres, torch.float32), t(w.freq, torch.float32), t(w.history, torch.int32))
        for i in range(w.nrows):
            if bool(st.greedy[i]):
                assert ref.ids[i] == int(st.z[i].argmax())
                continue
            got = ref.probs[i] > 0
            want = st.kept[i].numpy()
            diff = np.nonzero(got != want)[0]
            if diff.size == 0:
                continue
            # exact float64 exclusive masses on the same q, restricted to the top-k set
            q = (st.z[i].numpy() / w.temperature[i]).astype(np.float32)
            k = int(w.top_k[i])
            if 0 < k < w.V:
                kth = np.sort(q)[::-1][k - 1]
                q = np.where(q >= kth, q, -np.inf).astype(np.float32)
            _, excl = _exact_topp(q, float(w.top_p[i]))
            torch_err = np.abs(st.excl[i].numpy()[diff].astype(np.float64) - excl[diff])
            slack = np.abs(excl[diff] - float(w.top_p[i]))
            assert np.all(slack <= torch_err + 4 * np.spacing(np.float32(w.top_p[i]))), (name, i)
            # probabilities still agree to the stated tolerance where both keep the token
            both = got & want
            tol = 1e-5 if w.dtype == "f32" else 2e-3
            assert np.max(np.abs(ref.probs[i][both] - st.post[i].numpy()[both]), initial=0) < tol


# ---------------------------------------------------------------- draw


def test_draw_is_an_inverse_cdf_in_id_order():
    rng = np.random.default_rng(6)
    V = 23
    x = rng.standard_normal(V).astype(np.float32)
    grid = 4096
    u = ((np.arange(grid) + 0.5) / grid).astype(np.float32)
    logits = np.repeat(x[None, :], grid, axis=0)
    T = np.full(grid, 0.9, np.float32)
    P = np.full(grid, 0.8, np.float32)
    res = contract.sample(logits, "f32", T, top_p=P, uniforms=u, want_probs=True)
    p = res.probs[0]
    assert np.all(np.diff(res.ids) >= 0)  # ascending id as u grows
    counts = np.bincount(res.ids, minlength=V) / grid
    np.testing.assert_allclose(counts, p, atol=1.0 / grid + 1e-6)
    assert set(np.unique(res.ids)) == set(np.nonzero(p > 0)[0])
    # u = 0 gives the lowest kept id; u just below 1 the highest
    ends = contract.sample(logits[:2], "f32", T[:2], top_p=P[:2],
                           uniforms=np.array([0.0, np.nextafter(np.float32(1), np.float32(0))], np.float32))
    kept_ids = np.nonzero(p > 0)[0]
    assert ends.ids[0] == kept_ids.min() and ends.ids[1] == kept_ids.max()


def test_draw_distribution_matches_multinomial():
    rng = np.random.default_rng(7)
    V, n = 40, 20000
    x = (rng.standard_normal(V) * 1.5).astype(np.float32)
    logits = np.repeat(x[None, :], n, axis=0)
    T = np.full(n, 1.0, np.float32)
    P = np.full(n, 0.9, np.float32)
    res = contract.sample(logits, "f32", T, top_p=P, uniforms=rng.random(n).astype(np.float32), want_probs=True)
    p = res.probs[0].astype(np.float64)
    kept = p > 0
    obs = np.bincount(res.ids, minlength=V)[kept]
    g = torch.Generator().manual_seed(0)
    mult = torch.multinomial(torch.from_numpy(p), n, replacement=True, generator=g).numpy()
    obs_m = np.bincount(mult, minlength=V)[kept]
    from scipy.stats import chisquare
    assert chisquare(obs, n * p[kept]).pvalue > 1e-3
    assert chisquare(obs_m, n * p[kept]).pvalue > 1e-3


# ---------------------------------------------------------------- penalties


def test_repetition_penalty_matches_transformers():
    from transformers import RepetitionPenaltyLogitsProcessor

    rng = np.random.default_rng(8)
    V, H = 300, 64
    x = (rng.standard_normal(V) * 2).astype(np.float32)
    hist = rng.integers(0, V, H).astype(np.int32)
    for rp in (1.05, 1.3, 0.8):
        z, _, _, _, _ = contract.row_weights(x, "f32", 1.0, history=hist, rep=rp)
        proc = RepetitionPenaltyLogitsProcessor(penalty=rp)
        ref = proc(torch.from_numpy(hist[None, :].astype(np.int64)), torch.from_numpy(x[None, :].copy()))[0].numpy()
        np.testing.assert_array_equal(z, ref)


def test_presence_frequency_penalties_closed_form():
    rng = np.random.default_rng(9)
    V, H = 250, 200
    x = (rng.standard_normal(V) * 2).astype(np.float32)
    hist = np.concatenate([rng.integers(0, V, H), [-1, V, V + 5]]).astype(np.int32)  # out-of-range ids are padding
    rp, pres, freq = np.float32(1.1), np.float32(0.5), np.float32(0.3)
    z, q, _, _, _ = contract.row_weights(x, "f32", 0.8, history=hist, rep=float(rp), pres=float(pres),
                                         freq=float(freq))
    c = np.bincount(hist[(hist >= 0) & (hist < V)], minlength=V)
    want = x.copy()
    seen = c > 0
    want[seen] = np.where(x[seen] > 0, x[seen] / rp, x[seen] * rp).astype(np.float32)
    want[seen] = (want[seen] - (freq * c[seen].astype(np.float32))).astype(np.float32)
    want[seen] = (want[seen] - pres).astype(np.float32)
    np.testing.assert_array_equal(z, want)
    np.testing.assert_array_equal(q, (want / np.float32(0.8)).astype(np.float32))


def test_torch_reference_penalties_agree_with_oracle():
    w = W.make("penalties_b256_bf16", rows=[3])
    z, *_ = contract.row_weights(w.logits[0], "bf16", float(w.temperature[0]), history=w.history[0],
                                 rep=float(w.rep[0]), pres=float(w.pres[0]), freq=float(w.freq[0]))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    zt = torch_ref.apply_penalties(t(w.logits_f32()), t(w.history), t(w.rep), t(w.pres), t(w.freq))[0].numpy()
    np.testing.assert_array_equal(z, zt)


# ---------------------------------------------------------------- edge cases


def test_top_p_tiny_keeps_only_the_top_token():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((4, 100)).astype(np.float32)
    res = contract.sample(x, "f32", np.ones(4, np.float32), top_p=np.full(4, 1e-6, np.float32),
                          uniforms=rng.random(4).astype(np.float32), want_probs=True)
    np.testing.assert_array_equal(res.ids, x.argmax(axis=1))
    np.testing.assert_array_equal(res.kept, np.ones(4))


def test_flat_row_ties_resolve_to_lowest_ids():
    x = np.zeros((3, 64), np.float32)
    res = contract.sample(x, "f32", np.ones(3, np.float32), top_p=np.array([0.25, 0.5, 0.999], np.float32),
                          uniforms=np.array([0.99, 0.0, 0.5], np.float32), want_probs=True)
    # with 64 equal weights, top_p keeps floor(top_p*64)+1 tokens (exclusive mass <= top_p), lowest ids first
    for r, tp in enumerate([0.25, 0.5, 0.999]):
        n = math.floor(tp * 64) + 1
        assert res.kept[r] == min(n, 64)
        assert np.all(res.probs[r][:n] > 0) and np.all(res.probs[r][n:] == 0)


def test_nan_and_inf_logits_never_drawn():
    x = np.zeros((2, 50), np.float32)
    x[:, 3] = np.nan
    x[:, 4] = -np.inf
    x[:, 5] = 5.0
    res = contract.sample(x, "f32", np.ones(2, np.float32), uniforms=np.array([0.0, 0.999], np.float32),
                          want_probs=True)
    assert res.probs[:, 3].max() == 0 and res.probs[:, 4].max() == 0
    assert 3 not in res.ids and 4 not in res.ids
    g = contract.sample(x, "f32", np.zeros(2, np.float32))
    np.testing.assert_array_equal(g.ids, [3, 3])  # greedy: NaN is the maximum
