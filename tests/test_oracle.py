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


def test_exp2_coefficients_are_the_documented_fit():
    from oracle import fit_exp2

    fitted = fit_exp2.fit()
    committed = [contract.exp2_poly(0.0)]
    # recover c1..c6 from the committed polynomial through its values is ill-posed; compare
    # the polynomials instead: the committed one and the re-run fit agree to 2 fp32 ulps
    f = np.linspace(0.0, 1.0, 20001, dtype=np.float32)
    got = np.array([contract.exp2_poly(float(v)) for v in f], dtype=np.float32)
    ref = fit_exp2.horner_f32(fitted, f)
    ulps = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert committed[0] == 1.0 and ulps.max() <= 2


def test_exp2_poly_close_to_exp2():
    f = np.linspace(0.0, 1.0, 40001, endpoint=False).astype(np.float32)
    got = np.array([contract.exp2_poly(float(v)) for v in f])
    ref = np.exp2(f.astype(np.float64))
    assert np.max(np.abs(got - ref) / ref) < 7e-8
    assert contract.exp2_poly(0.0) == 1.0


@pytest.mark.parametrize("V", [248320, 4096, 151936, 2])
def test_weights_close_to_exp(V):
    SH = contract.shift(V)
    assert SH == 40 - math.ceil(math.log2(V))
    wmax = 2 ** (23 + SH)
    for qs in (0.0, 7.25, -3.5, 118.0, 1e-3):
        d = np.concatenate([-np.geomspace(1e-7, 50.0, 4000), np.linspace(-44, 0, 4001)])
        q = (np.float32(qs) + d.astype(np.float32)).astype(np.float32)
        q = q[q <= np.float32(qs)]
        w = np.array([contract.weight(float(v), qs, V) for v in q], dtype=np.float64)
        ref = np.exp(q.astype(np.float64) - float(np.float32(qs)))
        # error budget: fl(q - q*), fl(d * L), fl(y - n), the polynomial, the 24-bit mantissa, the shift
        dd = np.abs(q.astype(np.float64) - float(np.float32(qs)))
        tol = ref * (4e-7 + 1.2e-7 * dd) + 1.0 / wmax
        assert np.all(np.abs(w / wmax - ref) <= tol), (qs, np.max(np.abs(w / wmax - ref) - tol))
    assert contract.weight(3.0, 3.0, V) == wmax
    assert contract.weight(float("nan"), 3.0, V) == 0
    assert contract.weight(float("-inf"), 3.0, V) == 0
    assert contract.weight(3.0 - 45.0, 3.0, V) == 0  # y below -64
    # V weights of the maximum sum to at most 2**63
    assert V * wmax <= 2 ** 63


def test_weights_monotone_in_q():
    rng = np.random.default_rng(11)
    q = np.sort(np.concatenate([rng.uniform(-50, 5, 20000), rng.uniform(-1e-6, 0, 2000)]).astype(np.float32))
    q = np.concatenate([q, np.array([5.0], np.float32)])
    w = contract.weights(q, 248320)
    assert np.all(np.diff(w.astype(np.float64)) >= 0)
    # equal q, equal weight
    assert contract.weight(1.0, 5.0, 248320) == contract.weight(1.0, 5.0, 248320)


def test_ceil_scaled_is_exact():
    for f in (1.0, 0.5, 0.1, 0.3, 1e-7, 0.999999, 2.0 ** -30, 1e-40):
        f32 = np.float32(f)
        for e in (0, 10, 45, 62):
            want = math.ceil(float(f32) * 2 ** e) if float(f32) * 2 ** e < 2 ** 64 else None
            if want is None:
                continue
            # exact rational ceiling
            from fractions import Fraction
            exact = Fraction(float(f32)) * 2 ** e
            assert contract.ceil_scaled(float(f32), e) == math.ceil(exact), (f, e)


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
        d = q - q.max()
        p = np.exp(d)
        p /= p.sum()
        # the weights' error grows with the distance d from the row maximum (fl(q - q*), fl(d * L))
        tol = p * (6e-7 + 1.5e-7 * np.abs(d)) + 1e-15
        assert np.all(np.abs(res.probs[r] - p) <= tol), r


# ---------------------------------------------------------------- top-k and min_p


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
        assert res.kend[r] == want.sum()
        np.testing.assert_array_equal(res.probs[r] > 0, want)


def test_min_p_keeps_p_at_least_min_p_times_pmax():
    rng = np.random.default_rng(12)
    B, V = 64, 800
    logits = np.stack([_row_problem(rng, V, scale=rng.uniform(0.5, 3.0)) for _ in range(B)])
    T = rng.uniform(0.4, 1.3, B).astype(np.float32)
    MP = rng.uniform(0.0, 0.6, B).astype(np.float32)
    MP[::7] = 0.0
    res = contract.sample(logits, "f32", T, min_p=MP, uniforms=rng.random(B).astype(np.float32),
                          want_probs=True)
    for r in range(B):
        q = (logits[r] / T[r]).astype(np.float32).astype(np.float64)
        ratio = np.exp(q - q.max())  # p / p_max
        got = res.probs[r] > 0
        # closed form: kept iff p >= min_p * p_max; only ratios within the weights' error may differ
        want = ratio >= float(MP[r])
        diff = got != want
        assert np.all(np.abs(ratio[diff] - float(MP[r])) <= 5e-7 * max(float(MP[r]), 1e-30)), r
        if MP[r] == 0:
            assert got.all()


def test_min_p_then_top_p_over_the_remaining_mass():
    rng = np.random.default_rng(13)
    V = 500
    x = (rng.standard_normal(V) * 2).astype(np.float32)
    base = contract.sample(x[None], "f32", np.ones(1, np.float32), min_p=np.array([0.05], np.float32),
                           want_probs=True, uniforms=np.array([0.3], np.float32))
    kept_mp = base.probs[0] > 0
    both = contract.sample(x[None], "f32", np.ones(1, np.float32), min_p=np.array([0.05], np.float32),
                           top_p=np.array([0.7], np.float32), want_probs=True, uniforms=np.array([0.3], np.float32))
    # top-p runs on the renormalised min_p set: the float64 rule on that set
    q = x.astype(np.float64)
    qm = np.where(kept_mp, q, -np.inf)
    want, _ = _exact_topp(qm.astype(np.float32), 0.7)
    np.testing.assert_array_equal(both.probs[0] > 0, want & kept_mp)


# ---------------------------------------------------------------- top-p


def _exact_topp(q, top_p, scale=1.0):
    """The reference rule (src/compute/sampler.py:35-37) in float64 on the same q.

    ``scale`` multiplies the exact probabilities (Sigma p = scale), which is how
    torch's fp32 softmax differs from the exact one to first order."""
    q64 = q.astype(np.float64)
    p = np.exp(q64 - np.max(q64))
    p /= p.sum()
    p *= scale
    order = np.lexsort((np.arange(q.size), -q64))
    ps = p[order]
    excl = np.cumsum(ps) - ps
    kept = np.zeros(q.size, bool)
    kept[order[excl <= top_p]] = True
    kept &= p > 0
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
        diff = np.nonzero(got != want)[0]
        # the only admissible differences: exclusive mass within the weights' error of top_p
        assert np.all(np.abs(excl[diff] - P[r]) < 1e-6), (r, diff[:5], excl[diff][:5] - P[r])
        near += diff.size
    assert near <= 2


def _torch_state(w):
    t = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    return torch_ref.filter_rows(torch.from_numpy(w.logits_f32()), t(w.temperature, torch.float32),
                                 t(w.top_p, torch.float32), t(w.top_k, torch.int32), t(w.rep, torch.float32),
                                 t(w.pres, torch.float32), t(w.freq, torch.float32), t(w.history, torch.int32))


# Surviving-set differences between the oracle and the reference's own torch-CPU
# pipeline (src/compute/sampler.py:32-37), counted over whole workloads:
# (rows compared, rows that differ, tokens that differ, of which explained by an
# fp32 probability tie at torch's boundary, of which by torch's normalisation).
TORCH_DIFFS = {
    "hetero_b64_bf16": (58, 1, 1, 0, 1),
    "penalties_b256_bf16": (64, 64, 197, 0, 197),
    "flat_topp_b1024_f32": (64, 10, 11, 2, 9),
    "topk_topp_rep_bf16": (1, 0, 0, 0, 0),
}
TORCH_ROWS = {"hetero_b64_bf16": None, "penalties_b256_bf16": list(range(64)),
              "flat_topp_b1024_f32": list(range(0, 1024, 16)), "topk_topp_rep_bf16": None}


@pytest.mark.parametrize("name", list(TORCH_DIFFS))
def test_topp_against_torch_pipeline_on_workloads(name):
    """Every set difference from torch's fp32 pipeline is explained by its fp32 arithmetic.

    torch sorts its fp32 probabilities (ties by id) and compares an fp64-accumulated
    cumsum with top_p.  Two effects move its boundary away from the exact rule:
      * normalisation: its softmax sums to sigma != 1 (1 + 5e-6 on the penalised
        rows), which scales every exclusive mass by sigma;
      * fp32 ties: distinct q can round to one fp32 probability, and torch then
        orders them by id instead of by q (the near-ties of the north star).
    Checks per row:
      1. the oracle set equals the float64 rule on exact probabilities, except
         tokens whose exclusive mass lies within 1e-6 of top_p (the contract
         weights' error);
      2. the torch set equals the float64 rule on sigma-scaled probabilities,
         except tokens in torch's boundary tie group (fp32 probability equal to
         the largest dropped one) or within 2 fp32 ulps of top_p;
      3. every token in which the oracle and torch differ either has an exact
         exclusive mass on the other side of top_p once scaled by sigma (within
         2 ulps), or lies in torch's boundary tie group.
    A wrong boundary rule, a wrong mass or a wrong order fails one of them.
    """
    w = W.make(name, rows=TORCH_ROWS[name])
    ref = contract.sample_workload(w, want_probs=True)
    st = _torch_state(w)
    rows = rows_diff = tokens_diff = n_tie = n_norm = 0
    for i in range(w.nrows):
        if bool(st.greedy[i]):
            assert ref.ids[i] == int(st.z[i].argmax())
            continue
        rows += 1
        q = (st.z[i].numpy() / w.temperature[i]).astype(np.float32)
        k = int(w.top_k[i])
        if 0 < k < w.V:
            kth = np.sort(q)[::-1][k - 1]
            q = np.where(q >= kth, q, -np.inf).astype(np.float32)
        tp = float(w.top_p[i])
        ulp = float(np.spacing(np.float32(tp)))
        pt = st.probs[i].numpy()
        sigma = float(st.probs[i].double().sum())
        torch_set = st.kept[i].numpy()
        dropped = pt[~torch_set & (pt > 0)]
        tie_p = dropped.max() if dropped.size else np.float32(-1)
        tie_group = (pt == tie_p) & (pt > 0)
        exact_set, exact_excl = _exact_topp(q, tp)
        got = ref.probs[i] > 0
        d1 = np.nonzero(got != exact_set)[0]
        assert np.all(np.abs(exact_excl[d1] - tp) <= 1e-6), (name, i, d1[:5])
        scaled_set, scaled_excl = _exact_topp(q, tp, scale=sigma)
        d2 = np.nonzero((torch_set != scaled_set) & ~tie_group)[0]
        assert np.all(np.abs(scaled_excl[d2] - tp) <= 2 * ulp), (name, i, d2[:5])
        d3 = np.nonzero(got != torch_set)[0]
        lo = np.minimum(exact_excl[d3], scaled_excl[d3]) - 2 * ulp
        hi = np.maximum(exact_excl[d3], scaled_excl[d3]) + 2 * ulp
        norm = (lo <= tp) & (tp <= hi)
        tie = ~norm & tie_group[d3]
        assert np.all(tie | norm), (name, i, d3[~(tie | norm)][:5])
        rows_diff += d3.size > 0
        tokens_diff += d3.size
        n_tie += int(tie.sum())
        n_norm += int(norm.sum())
        both = got & torch_set
        tol = 1e-5 if w.dtype == "f32" else 2e-3
        assert np.max(np.abs(ref.probs[i][both] - st.post[i].numpy()[both]), initial=0) < tol
    rec = (rows, rows_diff, tokens_diff, n_tie, n_norm)
    print(f"[torch-diff] {name}: rows, rows differing, tokens, fp32-tie tokens, normalisation tokens = {rec}")
    assert rec == TORCH_DIFFS[name]


def test_top_p_one_keeps_the_whole_row_where_torch_drops_its_tail():
    """top_p = 1.0 inside a top-p batch (the T=1 row of the greedy-spikes workload).

    torch's fp32 softmax sums above 1 on this row, so its exclusive masses pass
    1.0 near the end of the sorted row and it drops tail tokens that the exact
    rule keeps (exclusive mass <= 1 always).  The contract keeps the whole row;
    every token torch drops has a sigma-scaled exclusive mass above 1."""
    w = W.make("greedy_spikes_f32", rows=[1])
    ref = contract.sample_workload(w, want_probs=True)
    st = _torch_state(w)
    sigma = float(st.probs[0].double().sum())
    dropped = np.nonzero(~st.kept[0].numpy() & (st.probs[0].numpy() > 0))[0]
    assert ref.kept[0] == w.V
    q = (st.z[0].numpy() / w.temperature[0]).astype(np.float32)
    _, scaled_excl = _exact_topp(q, 1.0, scale=sigma)
    assert sigma > 1.0 and dropped.size > 0
    assert np.all(scaled_excl[dropped] > 1.0 - 2 * float(np.spacing(np.float32(1.0))))
    print(f"[torch-diff] top_p=1.0 row: sigma-1 = {sigma - 1:.3e}, torch drops {dropped.size} tail tokens")


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
        z, _, _, _ = contract.row_weights(x, "f32", 1.0, history=hist, rep=rp)
        proc = RepetitionPenaltyLogitsProcessor(penalty=rp)
        ref = proc(torch.from_numpy(hist[None, :].astype(np.int64)), torch.from_numpy(x[None, :].copy()))[0].numpy()
        np.testing.assert_array_equal(z, ref)


def test_presence_frequency_penalties_closed_form():
    rng = np.random.default_rng(9)
    V, H = 250, 200
    x = (rng.standard_normal(V) * 2).astype(np.float32)
    hist = np.concatenate([rng.integers(0, V, H), [-1, V, V + 5]]).astype(np.int32)  # out-of-range ids are padding
    rp, pres, freq = np.float32(1.1), np.float32(0.5), np.float32(0.3)
    z, q, _, _ = contract.row_weights(x, "f32", 0.8, history=hist, rep=float(rp), pres=float(pres),
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
