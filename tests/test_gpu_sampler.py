"""GPU parity of the HIP sampler against the CPU oracle: every id, surviving-set
size and post-filter probability must be identical.  Needs an MI355X."""
import numpy as np
import pytest
import torch

from oracle import contract
from qedge_amd import workloads as W
from qedge_amd.batch import SamplingBatch
from qedge_amd.sampler import BatchSampler, Workspace, argmax_into, sample_gpu, sample_into
from qedge_amd.sampling_params import SamplingParams
from tests.devrun import order_of, row_paths, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


def _dev_logits(x, dtype, device, stride=None):
    B, V = x.shape
    if dtype == "f32":
        full = np.zeros((B, stride or V), np.float32)
        full[:, :V] = x
        t = torch.from_numpy(full).to(device)
    else:
        full = np.zeros((B, stride or V), np.uint16)
        full[:, :V] = x
        t = torch.from_numpy(full.view(np.int16)).to(device).view(torch.bfloat16)
    return t[:, :V]


def _run(x, dtype, device, T, P=None, K=None, rep=None, pres=None, freq=None, hist=None, u=None,
         use_top_p=True, stride=None, probs=True, paths=None, min_p=None, order=False, no_wait=False, ws=None,
         all_greedy=False):
    B, V = x.shape
    lg = _dev_logits(x, dtype, device, stride)
    t = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dt)
    H = 0 if hist is None else hist.shape[1]
    ws = ws or Workspace(B, V, lg.dtype, H, device)
    ids = torch.empty(B, dtype=torch.int64, device=device)
    ro = t(order_of(T, K, V), torch.int32) if order else None
    pr = torch.empty((B, V), dtype=torch.float32, device=device) if probs else None
    kept = torch.empty(B, dtype=torch.int32, device=device) if probs else None
    sample_into(lg, ids, ws, temperatures=t(T, torch.float32), top_ps=t(P, torch.float32), top_ks=t(K, torch.int32),
                repetition_penalties=t(rep, torch.float32), presence_penalties=t(pres, torch.float32),
                frequency_penalties=t(freq, torch.float32), history=t(hist, torch.int32),
                uniforms=t(u, torch.float32), use_top_p=use_top_p, out_probs=pr, out_kept=kept,
                min_ps=t(min_p, torch.float32), row_order=ro, no_wait=no_wait, all_greedy=all_greedy)
    torch.cuda.synchronize()
    if paths is not None:
        paths.extend(row_paths(ws, B))
    return ids.cpu().numpy(), None if pr is None else pr.cpu().numpy(), None if kept is None else kept.cpu().numpy()


def _check(x, dtype, device, T, P=None, K=None, rep=None, pres=None, freq=None, hist=None, u=None, **kw):
    ids, probs, kept = _run(x, dtype, device, T, P, K, rep, pres, freq, hist, u, **kw)
    use_top_p = kw.get("use_top_p", True)
    Tref = np.zeros_like(T) if kw.get("all_greedy") else T
    ref = contract.sample(x, dtype, Tref, P if use_top_p else None, K, rep, pres, freq, hist, u,
                          want_probs=probs is not None, min_p=kw.get("min_p"))
    np.testing.assert_array_equal(ids, ref.ids)
    if probs is not None:
        np.testing.assert_array_equal(kept, ref.kept)
        np.testing.assert_array_equal(probs, ref.probs)
    return ids


# ---------------------------------------------------------------- the five workloads


@pytest.mark.parametrize("name", W.WORKLOADS)
def test_full_batch_ids(gpu, name):
    w = W.make(name)
    print(f"[full] {name} B={w.nrows}", flush=True)
    ids, _, _ = run_gpu(w, gpu, want_probs=False)
    ref = run_oracle(w, want_probs=False)
    np.testing.assert_array_equal(ids, ref.ids)


@pytest.mark.parametrize("name", W.WORKLOADS)
def test_steps_match_oracle_and_repeat(gpu, name):
    rows = {"hetero_b64_bf16": list(range(0, 64, 3)), "penalties_b256_bf16": [0, 77, 200],
            "flat_topp_b1024_f32": [5, 600]}.get(name)
    w = W.make(name, rows=rows)
    print(f"[steps] {name}", flush=True)
    for step in (1, 2):
        ids, probs, kept = run_gpu(w, gpu, step=step)
        ref = run_oracle(w, step=step)
        np.testing.assert_array_equal(ids, ref.ids)
        np.testing.assert_array_equal(kept, ref.kept)
        np.testing.assert_array_equal(probs, ref.probs)
        again, _, _ = run_gpu(w, gpu, step=step, want_probs=False)
        np.testing.assert_array_equal(again, ids)


# ---------------------------------------------------------------- edge cases


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("V", [777, 4096, 20011])
def test_small_and_ragged_vocabularies(gpu, dtype, V):
    rng = np.random.default_rng(V)
    B = 7
    x = (rng.standard_normal((B, V)) * rng.uniform(0.1, 3.0, (B, 1))).astype(np.float32)
    x[1] = np.round(x[1] * 2) / 2  # ties
    x[2, 5] = np.nan
    x[3, :10] = -np.inf
    xx = W.bf16_bits(x) if dtype == "bf16" else x
    T = np.array([0.0, 0.7, 1.0, 1.3, 0.5, 0.9, 2.0], np.float32)
    P = np.array([0.9, 0.5, 1.0, 0.99, 1e-4, 0.8, 0.95], np.float32)
    K = np.array([0, 5, 0, min(V - 1, 1500), 1, 40, 0], np.int32)
    u = rng.random(B).astype(np.float32)
    print(f"[edge] V={V} {dtype}", flush=True)
    _check(xx, dtype, gpu, T, P, K, u=u)


def test_padded_rows_and_no_top_p(gpu):
    rng = np.random.default_rng(3)
    B, V = 5, 30001
    x = rng.standard_normal((B, V)).astype(np.float32)
    T = np.full(B, 0.8, np.float32)
    P = np.full(B, 0.5, np.float32)
    u = rng.random(B).astype(np.float32)
    print("[edge] padded rows", flush=True)
    _check(x, "f32", gpu, T, P, u=u, stride=V + 13)
    _check(x, "f32", gpu, T, P, u=u, use_top_p=False)


def test_penalties_with_padding_ids(gpu):
    rng = np.random.default_rng(4)
    B, V, H = 6, 50000, 3000
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    hist = rng.integers(-5, V + 5, (B, H)).astype(np.int32)
    hist[0, :200] = 17  # one token many times
    T = np.array([0.0, 0.8, 1.0, 0.6, 1.2, 0.9], np.float32)
    P = np.array([1.0, 0.95, 0.7, 1.0, 0.9, 0.6], np.float32)
    K = np.array([0, 0, 30, 0, 500, 2000], np.int32)
    rep = rng.uniform(0.9, 1.4, B).astype(np.float32)
    pres = rng.uniform(0.0, 1.0, B).astype(np.float32)
    freq = rng.uniform(0.0, 0.5, B).astype(np.float32)
    u = rng.random(B).astype(np.float32)
    print("[edge] penalties", flush=True)
    _check(W.bf16_bits(x), "bf16", gpu, T, P, K, rep, pres, freq, hist, u)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_barrier_timeouts_take_the_exact_path(gpu, dtype):
    """With QS_FLAG_NO_WAIT every row barrier gives up at once (a host-forced
    time-out; every kernel still exits normally): the top-k-off rows are then
    resolved by the exact single-workgroup path, with the same results."""
    rng = np.random.default_rng(15)
    B, V = 6, 60000
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    xx = W.bf16_bits(x) if dtype == "bf16" else x
    T = np.array([1.0, 0.8, 0.0, 1.2, 0.6, 1.0], np.float32)
    P = np.array([0.9, 1.0, 1.0, 0.95, 0.7, 0.5], np.float32)
    K = np.array([0, 0, 0, 0, 40, 0], np.int32)
    hist = rng.integers(0, V, (B, 300)).astype(np.int32)
    rep = np.full(B, 1.2, np.float32)
    pres = np.full(B, 0.3, np.float32)
    freq = np.full(B, 0.2, np.float32)
    u = rng.random(B).astype(np.float32)
    print(f"[edge] barrier time-outs {dtype}", flush=True)
    paths = []
    _check(xx, dtype, gpu, T, P, K, rep, pres, freq, hist, u=u, no_wait=True, paths=paths)
    path, why = paths
    mass = [0, 1, 3, 5]
    assert np.all(path[mass] == 5) and np.all(why[mass] != 0), (path.tolist(), why.tolist())
    assert path[2] == 1 and path[4] == 2


def test_adversarial_layout_falls_back_exactly(gpu):
    """Sorted logits put the whole top-k in one chunk: the candidate path must give up and stay exact."""
    B, V = 2, 100000
    x = np.sort(np.random.default_rng(6).standard_normal((B, V)).astype(np.float32), axis=1)[:, ::-1].copy()
    T = np.ones(B, np.float32)
    P = np.array([0.99, 1.0], np.float32)
    K = np.array([1000, 700], np.int32)
    print("[edge] adversarial", flush=True)
    _check(x, "f32", gpu, T, P, K, u=np.array([0.3, 0.7], np.float32))


def test_argmax_entry_point(gpu):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((9, 70000)).astype(np.float32)
    x[2, [5, 600, 9000]] = 100.0
    x[4, 33] = np.nan
    lg = torch.from_numpy(x).to(gpu).to(torch.bfloat16)
    ws = Workspace(9, 70000, torch.bfloat16, 0, gpu)
    out = torch.empty(9, dtype=torch.int64, device=gpu)
    argmax_into(lg, out, ws)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), lg.float().cpu().argmax(dim=-1).numpy())


# ---------------------------------------------------------------- module API and graphs


def test_batch_sampler_module_and_runner(gpu):
    V = 248320
    w = W.make("hetero_b64_bf16", rows=list(range(0, 64, 5)))
    params = []
    for r in range(w.nrows):
        k = int(w.top_k[r])
        params.append(SamplingParams(temperature=float(w.temperature[r]), top_p=float(w.top_p[r]),
                                     top_k=None if k == 0 else k, seed=1000 + r))
    batch = SamplingBatch(w.nrows, V, gpu)
    batch.fill(params, step=3)
    lg = torch.from_numpy(np.ascontiguousarray(w.logits).view(np.int16)).to(gpu).view(torch.bfloat16)
    ids = sample_gpu(BatchSampler(), [lg[i:i + 1] for i in range(w.nrows)], batch)
    torch.cuda.synchronize()
    u = batch.uniforms[: w.nrows].cpu().numpy()
    ref = contract.sample(w.logits, "bf16", batch.temperatures[: w.nrows].cpu().numpy(),
                          batch.top_ps[: w.nrows].cpu().numpy(), batch.top_ks[: w.nrows].cpu().numpy(), uniforms=u)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref.ids)
    # all-greedy batch: the argmax path
    batch.fill([SamplingParams() for _ in range(w.nrows)])
    g = sample_gpu(BatchSampler(), lg, batch)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(g.cpu().numpy(), lg.float().cpu().argmax(dim=-1).numpy())


def test_graph_replays_match_eager(gpu):
    w = W.make("hetero_b64_bf16")
    lg = torch.from_numpy(np.ascontiguousarray(w.logits).view(np.int16)).to(gpu).view(torch.bfloat16)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device=gpu, dtype=dt)
    T, P, K = t(w.temperature, torch.float32), t(w.top_p, torch.float32), t(w.top_k, torch.int32)
    U = [t(w.uniforms(s), torch.float32) for s in range(3)]
    ws = Workspace(w.nrows, w.V, torch.bfloat16, 0, gpu)
    outs = [torch.empty(w.nrows, dtype=torch.int64, device=gpu) for _ in range(3)]

    def steps():
        for s in range(3):
            sample_into(lg, outs[s], ws, temperatures=T, top_ps=P, top_ks=K, uniforms=U[s], use_top_p=True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        steps()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = [o.cpu().numpy().copy() for o in outs]
    ref = [contract.sample_workload(w, step=s).ids for s in range(3)]
    for s in range(3):
        np.testing.assert_array_equal(eager[s], ref[s])
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        steps()
    for rep in range(4):
        for o in outs:
            o.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for s in range(3):
            np.testing.assert_array_equal(outs[s].cpu().numpy(), eager[s])
        steps()  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_special_values_in_top_keys(gpu, dtype):
    """NaN, -0 and +0 among the largest logits of top-k rows (the streaming
    pass ranks raw z bits there), an all-equal row, a row of -inf but three
    tokens, and more than 32 chunks per row (V = 300001)."""
    rng = np.random.default_rng(11)
    B, V = 8, 300001
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    top = np.argsort(-x[0])[:40]
    x[0, top[::3]] = np.nan                  # NaN scattered through the top-40 of row 0
    x[1] = np.minimum(x[1], 0.0)
    x[1, rng.integers(0, V, 500)] = -0.0     # many -0 next to +0 at the top of row 1
    x[1, rng.integers(0, V, 500)] = 0.0
    x[2] = 1.25                              # every token tied
    x[3] = -np.inf
    x[3, [7, V // 2, V - 1]] = [1.0, 1.0, 0.5]
    x[4, V - 5:] = 50.0                      # the top-k in the row's last (partial) chunk
    xx = W.bf16_bits(x) if dtype == "bf16" else x
    T = np.array([0.9, 1.0, 0.7, 1.0, 0.5, 1.1, 0.8, 0.0], np.float32)
    P = np.array([0.9, 0.8, 0.95, 1.0, 0.9, 0.7, 1.0, 1.0], np.float32)
    K = np.array([30, 200, 10, 2, 3, 0, 64, 0], np.int32)
    u = rng.random(B).astype(np.float32)
    print(f"[edge] special values {dtype}", flush=True)
    _check(xx, dtype, gpu, T, P, K, u=u)


@pytest.mark.parametrize("V", [8192 * 3 + 17, 8192 * 4, 248320])
def test_bf16_greedy_and_top_k_rows_two_chunks_per_workgroup(gpu, V):
    """bf16 greedy and top-k rows without penalties (16-bit keys, two chunks per
    workgroup): NaN as the greedy maximum (first NaN wins), -0 before +0 at the
    maximum of a non-positive row (the first zero wins), a row of -inf with
    two finite tokens, an all -inf row (index 0), the maximum in the last,
    partial or odd chunk (a workgroup serving one chunk), ties at the maximum,
    and top-k rows beside them with the same layouts."""
    rng = np.random.default_rng(V % 1009)
    B = 10
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    x[0, [V // 3, 5, V - 2]] = np.nan                     # first NaN: index 5
    x[1] = -np.abs(x[1]) - 0.5
    x[1, [11, 4000, V - 3]] = [-0.0, 0.0, -0.0]           # first zero: 11 (a -0)
    x[2] = -np.inf
    x[2, [V - 1, 9]] = [-3.0, -3.0]                       # tie among the only finite tokens
    x[3] = -np.inf                                        # every token -inf: index 0
    x[4, V - 1] = 40.0                                    # maximum in the last chunk
    x[5, [100, V - 100, V // 2]] = 30.0                   # three-way tie at the maximum
    x[6, V - 4:] = 25.0                                   # top-k inside the last chunk
    x[7, rng.integers(0, V, 300)] = 0.0
    x[7, rng.integers(0, V, 300)] = -0.0
    x[7] = np.minimum(x[7], 0.0)                          # top-k at the zeros
    xx = W.bf16_bits(x)
    T = np.array([0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.8, 1.0, 0.9, 0.7], np.float32)
    P = np.array([1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 0.9, 0.95, 0.8, 1.0], np.float32)
    K = np.array([0, 0, 0, 0, 0, 0, 3, 50, 700, 1], np.int32)
    u = rng.random(B).astype(np.float32)
    print(f"[edge] bf16 packed rows V={V}", flush=True)
    for order in (False, True):
        paths = []
        ids = _check(xx, "bf16", gpu, T, P, K, u=u, order=order, paths=paths)
        assert ids[0] == 5 and ids[1] == 11 and ids[2] == 9 and ids[3] == 0 and ids[4] == V - 1 and ids[5] == 100
        why = paths[1]
        # (row 7 may take the exact path: -0 and +0 are distinct 16-bit keys, so a
        # chunk threshold between them leaves a tie with the k-th value out)
        assert not np.any(why[[6, 8, 9]]), f"top-k rows fell back (reasons {why.tolist()})"


def test_bf16_batch_with_histories_mixing_penalised_and_plain_rows(gpu):
    """A bf16 batch with a history matrix where only some rows use penalties:
    the rows without them take the two-chunk path while every workgroup loads
    its chunk at once (histories present), the penalised rows the per-chunk
    path; greedy, top-k and top-k-off rows of both kinds."""
    rng = np.random.default_rng(97)
    B, V = 12, 248320
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    xx = W.bf16_bits(x)
    T = np.array([0.0, 0.8, 1.0, 0.7, 0.0, 0.9, 1.2, 0.6, 0.0, 0.5, 1.0, 0.8], np.float32)
    P = np.array([1.0, 0.9, 0.95, 0.8, 1.0, 0.7, 1.0, 0.9, 1.0, 0.85, 0.9, 1.0], np.float32)
    K = np.array([0, 40, 0, 500, 0, 7, 0, 90, 0, 1000, 0, 33], np.int32)
    rep = np.where(np.arange(B) % 2 == 0, 1.0, 1.15).astype(np.float32)   # even rows: no penalty
    pres = np.where(np.arange(B) % 2 == 0, 0.0, 0.4).astype(np.float32)
    freq = np.where(np.arange(B) % 2 == 0, 0.0, 0.2).astype(np.float32)
    hist = rng.integers(0, V, (B, 1024)).astype(np.int32)
    top = np.argsort(-x, axis=1)[:, :8]
    hist[:, :8] = top  # the penalties move the top tokens of the penalised rows
    u = rng.random(B).astype(np.float32)
    print("[edge] bf16 histories, penalised and plain rows", flush=True)
    for order in (False, True):
        _check(xx, "bf16", gpu, T, P, K, rep, pres, freq, hist, u=u, order=order)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_ties_at_the_one_wave_finishers(gpu, dtype):
    """Tie groups where the one-wave finishers draw their lines, every row on
    its fast path:
      0  k = 10 with 100 tokens at the k-th value: the sorted finisher keeps 64
         and hands the row to the general one (ties may go on past the 64);
      1  k = 20 with 40 tokens at the k-th value: the sorted finisher keeps all;
      2  top-k off, top-p 0.5 inside a group of 30 tied tokens (a short list);
      3  top-k off, top-p 0.7 across two tie groups near the top;
      4  k = 63 with 64 tied tokens at the top;
      5  k = 3 with 5 tied tokens (ties kept), top-p 0.9."""
    rng = np.random.default_rng(23)
    B, V = 6, 100000
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    ties = rng.choice(V, 100, replace=False)
    x[0, ties] = 9.0
    x[1, ties[:40]] = 9.0
    x[2, ties[:30]] = 12.0
    x[3, ties[:12]] = 12.0
    x[3, ties[12:20]] = 11.5
    x[4, ties[:64]] = 8.0
    x[5, ties[:5]] = 8.0
    xx = W.bf16_bits(x) if dtype == "bf16" else x
    T = np.array([1.0, 0.8, 1.0, 0.9, 1.0, 0.7], np.float32)
    P = np.array([0.9, 0.8, 0.5, 0.7, 0.95, 0.9], np.float32)
    K = np.array([10, 20, 0, 0, 63, 3], np.int32)
    u = rng.random(B).astype(np.float32)
    print(f"[edge] tie groups at the finishers {dtype}", flush=True)
    paths = []
    _check(xx, dtype, gpu, T, P, K, u=u, paths=paths)
    path, why = paths
    assert not np.any(why), f"rows fell back: {np.nonzero(why)[0].tolist()} (reasons {why.tolist()})"


@pytest.mark.parametrize("B,V,dtype", [(1, 248320, "bf16"), (2, 2048 * 7 + 100, "bf16"), (3, 600001, "bf16"),
                                       (12, 8192 * 5 + 300, "f32")])
def test_chunk_layouts_and_sparse_last_chunks(gpu, B, V, dtype):
    """Rows of 8192-logit chunks whose last chunk holds fewer logits than one
    wave's share (waves without tokens); every row must still be resolved on
    its fast path (no single-workgroup fallback)."""
    rng = np.random.default_rng(B * 1000 + V % 997)
    x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    x[0, V - 7] = 9.0  # a top token inside the last chunk
    xx = W.bf16_bits(x) if dtype == "bf16" else x
    kinds = [(0.8, 0.9, 20), (1.0, 0.95, 0), (0.0, 1.0, 0), (0.7, 1.0, 300), (1.2, 0.8, 5), (0.9, 0.9, 64)]
    T = np.array([kinds[r % len(kinds)][0] for r in range(B)], np.float32)
    P = np.array([kinds[r % len(kinds)][1] for r in range(B)], np.float32)
    K = np.array([kinds[r % len(kinds)][2] for r in range(B)], np.int32)
    hist = (rng.integers(0, V, (B, 512))).astype(np.int32)
    rep = np.full(B, 1.1, np.float32)
    pres = np.full(B, 0.2, np.float32)
    freq = np.full(B, 0.1, np.float32)
    u = rng.random(B).astype(np.float32)
    print(f"[edge] chunk layout B={B} V={V} {dtype}", flush=True)
    paths = []
    _check(xx, dtype, gpu, T, P, K, rep, pres, freq, hist, u=u, probs=False, paths=paths)
    why = paths[1]
    assert not np.any(why), f"rows {np.nonzero(why)[0].tolist()} fell back (reasons {why[why != 0].tolist()})"


@pytest.mark.parametrize("B,V,dtype", [(40, 8192 * 6 + 123, "bf16"), (64, 50000, "f32"), (8, 30011, "bf16"),
                                       (6, 20000, "f32")])
def test_many_top_k_off_rows(gpu, B, V, dtype):
    """Flat, peaked and no-top-p rows with top-k off, mixed with top-k and
    greedy rows, in the natural order and in the dispatch order."""
    rng = np.random.default_rng(B * 7919 + V)
    x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    xx = W.bf16_bits(x) if dtype == "bf16" else x
    kinds = [(1.0, 0.9, 0), (0.05, 0.95, 0), (1.3, 1.0, 0), (0.7, 0.8, 50), (0.0, 1.0, 0), (0.9, 0.6, 0)]
    T = np.array([kinds[r % len(kinds)][0] for r in range(B)], np.float32)
    P = np.array([kinds[r % len(kinds)][1] for r in range(B)], np.float32)
    K = np.array([kinds[r % len(kinds)][2] for r in range(B)], np.int32)
    u = rng.random(B).astype(np.float32)
    print(f"[edge] top-k-off rows B={B} V={V} {dtype}", flush=True)
    paths = []
    _check(xx, dtype, gpu, T, P, K, u=u, paths=paths)
    _check(xx, dtype, gpu, T, P, K, u=u, order=True)
    why = paths[1]
    assert not np.any(why), f"rows {np.nonzero(why)[0].tolist()} fell back (reasons {why[why != 0].tolist()})"


def _mixed_rows(B, V, seed):
    rng = np.random.default_rng(seed)
    x = (rng.gumbel(size=(B, V)) * rng.uniform(1.0, 4.0, size=(B, 1))).astype(np.float32)
    kinds = [(1.0, 0.9, 0), (0.3, 0.8, 300), (1.3, 1.0, 0), (0.7, 0.8, 50), (0.0, 1.0, 0), (0.9, 0.6, 0),
             (1.1, 0.95, 1000), (0.05, 0.95, 0)]
    T = np.array([kinds[r % len(kinds)][0] for r in range(B)], np.float32)
    P = np.array([kinds[r % len(kinds)][1] for r in range(B)], np.float32)
    K = np.array([kinds[r % len(kinds)][2] for r in range(B)], np.int32)
    return x, T, P, K, rng


@pytest.mark.parametrize("B,V,dtype", [(72, W.VOCAB, "bf16"), (100, W.VOCAB, "f32")])
def test_mixed_batches_above_64_rows(gpu, B, V, dtype):
    """Mixed kinds above 64 rows against the oracle, every row on its fast
    path at the full vocabulary, with the dispatch order."""
    x, T, P, K, rng = _mixed_rows(B, V, B * 31 + V)
    xx = W.bf16_bits(x) if dtype == "bf16" else x
    u = rng.random(B).astype(np.float32)
    print(f"[edge] mixed batch B={B} V={V} {dtype}", flush=True)
    paths = []
    _check(xx, dtype, gpu, T, P, K, u=u, paths=paths, order=True)
    why = paths[1]
    assert not np.any(why), f"rows {np.nonzero(why)[0].tolist()} fell back (reasons {why[why != 0].tolist()})"


def test_graph_replays_with_row_order(gpu):
    """Replays of a captured call (B = 72, dispatch order given) match the eager calls."""
    B, V = 72, 8192 * 12 + 77
    x, T, P, K, rng = _mixed_rows(B, V, 4242)
    lg = _dev_logits(W.bf16_bits(x), "bf16", gpu)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device=gpu, dtype=dt)
    Td, Pd, Kd = t(T, torch.float32), t(P, torch.float32), t(K, torch.int32)
    U = [t(rng.random(B).astype(np.float32), torch.float32) for _ in range(2)]
    ws = Workspace(B, V, torch.bfloat16, 0, gpu)
    ro = t(order_of(T, K, V), torch.int32)
    outs = [torch.empty(B, dtype=torch.int64, device=gpu) for _ in range(2)]

    def steps():
        for s in range(2):
            sample_into(lg, outs[s], ws, temperatures=Td, top_ps=Pd, top_ks=Kd, uniforms=U[s], use_top_p=True,
                        row_order=ro)

    print("[edge] graph replays with a row order", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        steps()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    eager = [o.cpu().numpy().copy() for o in outs]
    for s in range(2):
        ref = contract.sample(W.bf16_bits(x), "bf16", T, P, K, None, None, None, None, U[s].cpu().numpy(),
                              want_probs=False)
        np.testing.assert_array_equal(eager[s], ref.ids)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        steps()
    for rep in range(3):
        for o in outs:
            o.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for s in range(2):
            np.testing.assert_array_equal(outs[s].cpu().numpy(), eager[s])
        steps()  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_temperatures_outside_the_fast_division_range(gpu, dtype):
    """Rows whose T lies outside [2^-16, 2^16] take the IEEE division for every
    logit; rows inside it take the fast one for logits in [2^-80, 2^80) and the
    division for zeros, tiny and huge logits."""
    rng = np.random.default_rng(31)
    V = 8192 * 3 + 77
    x = (rng.standard_normal((6, V)) * 2).astype(np.float32)
    x[0, :50] = 0.0
    x[1, 10:20] = 1e-30  # below 2^-80
    x[2, 30:40] = 3e25   # above 2^80
    T = np.array([1.2e-5, 7e4, 0.7, 2.0 ** -16, 2.0 ** 16, 1e-4], np.float32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        x = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    P = np.array([0.9, 0.8, 0.95, 0.7, 1.0, 0.9], np.float32)
    K = np.array([0, 40, 0, 0, 0, 300], np.int32)
    _check(x, dtype, gpu, T, P, K, u=rng.random(6).astype(np.float32))
