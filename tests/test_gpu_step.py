"""GPU tests of the decode-step path around the sampler: the pending-token
slots, the on-device stop check and token history (qs_step_finish,
qs_history_append), greedy argmax inside a captured graph, histories staged
through SamplingBatch, min_p, and one workspace serving several batch sizes.
Every id is checked against the CPU oracle; the stop rule against its host
statement of src/control/scheduler.py:304-322.  Needs an MI355X."""
import numpy as np
import pytest
import torch

from oracle import contract
from qedge_amd.batch import SamplingBatch
from qedge_amd.sampler import BatchSampler, Workspace, argmax_into, sample_gpu, sample_into
from qedge_amd.sampling_params import SamplingParams
from qedge_amd.step import DecodeStep, step_finish_reference

pytestmark = pytest.mark.gpu


def _bf16(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def _f32(bits: np.ndarray) -> np.ndarray:
    """bf16 bits -> their fp32 values."""
    return (np.ascontiguousarray(bits).astype(np.uint32) << 16).view(np.float32)


def _dev_bf16(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(torch.bfloat16)


def _hist_matrix(hists, H):
    m = np.full((len(hists), H), -1, np.int32)
    for r, h in enumerate(hists):
        tail = h[-H:]
        m[r, :len(tail)] = tail
    return m


def test_decode_loop_in_graph_matches_host_rules(gpu):
    """Sampler + step bookkeeping captured once, replayed for 6 steps, against
    the oracle (ids, with the growing history) and the host stop rule."""
    B, V, H, STEPS, EOS = 6, 20011, 32, 6, 7
    rng = np.random.default_rng(11)
    T = np.array([0.0, 0.0, 0.0, 0.8, 0.9, 1.1], np.float32)
    P = np.array([1.0, 1.0, 1.0, 0.9, 0.95, 0.8], np.float32)
    K = np.array([0, 0, 0, 40, 0, 200], np.int32)
    rep = np.array([1.0, 1.2, 1.0, 1.3, 1.1, 1.0], np.float32)
    pres = np.array([0.0, 0.3, 0.0, 0.2, 0.0, 0.5], np.float32)
    freq = np.array([0.0, 0.1, 0.0, 0.5, 0.2, 0.0], np.float32)
    min_t = [0, 3, 0, 0, 0, 1]
    max_t = [8, 8, 8, 3, 0, 8]
    ign = [False, False, True, False, False, False]
    slots = [5, 0, 3, 1, 4, 2]
    hists = [list(rng.integers(0, V, size=int(n))) for n in (0, 5, 40, 12, 3, 31)]
    logits = []
    for s in range(STEPS):
        x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
        if s == 1:
            x[0, EOS] = 30.0  # row 0: greedy, EOS at its 2nd token -> finished
            x[1, EOS] = 30.0  # row 1: EOS before min_tokens -> not finished
            x[2, EOS] = 30.0  # row 2: ignore_eos
        logits.append(_bf16(x))
    U = [np.minimum(rng.random(B), 0.999999).astype(np.float32) for _ in range(STEPS)]

    def run(captured: bool):
        st = DecodeStep(B, gpu, n_pending=8, history=H, eos_id=EOS)
        for r in range(B):
            st.set_row(r, slot=slots[r], min_tokens=min_t[r], max_tokens=max_t[r], ignore_eos=ign[r],
                       history=hists[r])
        t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device=gpu, dtype=dt)
        lg = _dev_bf16(logits[0], gpu).clone()
        u = t(U[0], torch.float32)
        ids = torch.empty(B, dtype=torch.int64, device=gpu)
        ws = Workspace(B, V, torch.bfloat16, H, gpu)
        hv, hl = st.history_view(B)
        kw = dict(temperatures=t(T, torch.float32), top_ps=t(P, torch.float32), top_ks=t(K, torch.int32),
                  repetition_penalties=t(rep, torch.float32), presence_penalties=t(pres, torch.float32),
                  frequency_penalties=t(freq, torch.float32), history=hv, history_len=hl, uniforms=u,
                  use_top_p=True)

        def step():
            sample_into(lg, ids, ws, **kw)
            st.finish(ids, B)

        g = None
        if captured:
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step()
        out = []
        for s in range(STEPS):
            lg.copy_(_dev_bf16(logits[s], gpu))
            u.copy_(t(U[s], torch.float32))
            if captured:
                g.replay()
            else:
                step()
            host_ids, host_fin = st.read(ids, B)
            torch.cuda.synchronize()
            out.append(dict(ids=ids.cpu().numpy().copy(), host_ids=np.array(host_ids),
                            host_fin=np.array(host_fin), fin=st.finished[:B].cpu().numpy().astype(bool),
                            pending=st.pending.cpu().numpy().copy(), ngen=st.num_generated[:B].cpu().numpy().copy(),
                            hist=st.history[:B].cpu().numpy().copy(), hlen=st.history_len[:B].cpu().numpy().copy()))
        return out

    eager, graph = run(False), run(True)
    # host statement of the same loop
    ngen = [0] * B
    hl = [list(h) for h in hists]
    for s in range(STEPS):
        ref = contract.sample(logits[s], "bf16", T, P, K, rep, pres, freq, _hist_matrix(hl, H), U[s])
        ngen_new, fin = step_finish_reference(list(ref.ids), ngen, min_t, max_t, ign, EOS)
        for res in (eager[s], graph[s]):
            np.testing.assert_array_equal(res["ids"], ref.ids)
            np.testing.assert_array_equal(res["host_ids"], ref.ids)
            np.testing.assert_array_equal(res["fin"], np.array(fin))
            np.testing.assert_array_equal(res["host_fin"], np.array(fin))
            np.testing.assert_array_equal(res["ngen"], np.array(ngen_new))
            for r in range(B):
                assert res["pending"][slots[r]] == ref.ids[r]
        ngen = ngen_new
        for r in range(B):
            hl[r].append(int(ref.ids[r]))
        for res in (eager[s], graph[s]):
            for r in range(B):
                n = min(len(hl[r]), H)
                assert res["hlen"][r] == min(len(hists[r]), H) + s + 1  # the staged tail, then one per step
                assert sorted(res["hist"][r, :n].tolist()) == sorted(hl[r][-H:])
    # the planted stops
    assert eager[1]["fin"][0] and not eager[1]["fin"][1] and not eager[1]["fin"][2]
    assert eager[2]["fin"][3] and eager[0]["fin"][4]


def test_argmax_captured_in_a_graph(gpu):
    """The in-graph greedy path (src/compute/model_runner.py:349-354): argmax
    captured once and replayed on new logits, against torch's argmax."""
    B, V = 5, 248320
    rng = np.random.default_rng(5)
    lg = torch.empty((B, V), dtype=torch.bfloat16, device=gpu)
    ids = torch.empty(B, dtype=torch.int64, device=gpu)
    ws = Workspace(B, V, torch.bfloat16, 0, gpu)
    lg.copy_(_dev_bf16(_bf16(rng.standard_normal((B, V)).astype(np.float32)), gpu))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        argmax_into(lg, ids, ws)
    for rep in range(4):
        x = (rng.standard_normal((B, V)) * (1 + rep)).astype(np.float32)
        x[1, rng.integers(V)] = np.inf
        if rep == 2:
            x[3, 1000] = np.nan  # NaN is the maximum
        bits = _bf16(x)
        lg.copy_(_dev_bf16(bits, gpu))
        ids.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        want = lg.float().cpu().argmax(dim=-1).numpy()
        np.testing.assert_array_equal(ids.cpu().numpy(), want)
        ref = contract.sample(bits, "bf16", np.zeros(B, np.float32), uniforms=np.zeros(B, np.float32))
        np.testing.assert_array_equal(ids.cpu().numpy(), ref.ids)
        argmax_into(lg, ids, ws)  # eager work between replays
        torch.cuda.synchronize()


def test_histories_staged_through_sampling_batch(gpu):
    """Token histories go Sequence -> SamplingBatch.fill -> sample_gpu -> kernel
    (src/data/sequence.py:177-179, qedge_amd/batch.py) and match the oracle."""
    B, V, H = 7, 50000, 64
    rng = np.random.default_rng(21)
    x = _bf16((rng.standard_normal((B, V)) * 2.0).astype(np.float32))
    params, hists = [], []
    for r in range(B):
        params.append(SamplingParams(temperature=0.0 if r == 0 else 0.7 + 0.1 * r, top_p=0.9,
                                     top_k=None if r % 3 == 0 else 20 * r, repetition_penalty=1.0 + 0.1 * r,
                                     presence_penalty=0.1 * (r % 2), frequency_penalty=0.05 * r, seed=77 + r))
        hot = list(np.argsort(-_f32(x[r]))[:5])  # penalise likely tokens
        hists.append([int(t) for t in hot] * 3 + list(rng.integers(0, V, size=r * 9)))
    batch = SamplingBatch(B, V, gpu, max_history=H)
    batch.fill(params, histories=hists, step=4)
    ids = sample_gpu(BatchSampler(), _dev_bf16(x, gpu), batch)
    torch.cuda.synchronize()
    c = lambda t: t[:B].cpu().numpy()
    ref = contract.sample(x, "bf16", c(batch.temperatures), c(batch.top_ps), c(batch.top_ks),
                          c(batch.repetition_penalties), c(batch.presence_penalties), c(batch.frequency_penalties),
                          c(batch.history), c(batch.uniforms))
    np.testing.assert_array_equal(ids.cpu().numpy(), ref.ids)


def test_all_greedy_batch_with_penalties_is_penalised(gpu):
    """An all-greedy batch whose rows carry penalties takes the argmax of the
    penalised logits, the same id as in a mixed batch."""
    B, V, H = 4, 30011, 16
    rng = np.random.default_rng(8)
    x = _bf16(rng.standard_normal((B, V)).astype(np.float32))
    params = [SamplingParams(temperature=0.0, repetition_penalty=3.0, presence_penalty=2.0) for _ in range(B)]
    hists = [[int(np.argmax(_f32(x[r])))] for r in range(B)]
    batch = SamplingBatch(B, V, gpu, max_history=H)
    batch.fill(params, histories=hists)
    assert batch.all_greedy and batch.use_penalties
    ids = sample_gpu(BatchSampler(), _dev_bf16(x, gpu), batch).cpu().numpy()
    c = lambda t: t[:B].cpu().numpy()
    ref = contract.sample(x, "bf16", c(batch.temperatures), None, None, c(batch.repetition_penalties),
                          c(batch.presence_penalties), c(batch.frequency_penalties), c(batch.history),
                          np.zeros(B, np.float32))
    np.testing.assert_array_equal(ids, ref.ids)
    assert all(ids[r] != hists[r][0] for r in range(B))  # the penalised maximum lost


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_min_p_rows(gpu, dtype):
    """min_p on top-k rows and on top-k-off rows, with and without top-p."""
    B, V = 8, 248320
    rng = np.random.default_rng(3)
    xf = (rng.standard_normal((B, V)) * np.linspace(0.5, 3.0, B)[:, None]).astype(np.float32)
    x = xf if dtype == "f32" else _bf16(xf)
    T = np.array([0.7, 1.0, 0.5, 1.3, 0.9, 1.0, 0.8, 1.2], np.float32)
    P = np.array([0.9, 1.0, 0.95, 0.8, 1.0, 0.7, 0.99, 0.9], np.float32)
    K = np.array([0, 0, 50, 0, 1000, 0, 7, 300], np.int32)
    MP = np.array([0.05, 0.1, 0.2, 0.01, 0.3, 0.0, 0.5, 0.02], np.float32)
    U = rng.random(B).astype(np.float32)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device=gpu, dtype=dt)
    lg = t(x, torch.float32) if dtype == "f32" else _dev_bf16(x, gpu)
    ws = Workspace(B, V, lg.dtype, 0, gpu)
    ids = torch.empty(B, dtype=torch.int64, device=gpu)
    probs = torch.empty((B, V), dtype=torch.float32, device=gpu)
    kept = torch.empty(B, dtype=torch.int32, device=gpu)
    sample_into(lg, ids, ws, temperatures=t(T, torch.float32), top_ps=t(P, torch.float32), top_ks=t(K, torch.int32),
                min_ps=t(MP, torch.float32), uniforms=t(U, torch.float32), use_top_p=True, out_probs=probs,
                out_kept=kept)
    torch.cuda.synchronize()
    ref = contract.sample(x, dtype, T, P, K, uniforms=U, want_probs=True, min_p=MP)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref.ids)
    np.testing.assert_array_equal(kept.cpu().numpy(), ref.kept)
    np.testing.assert_array_equal(probs.cpu().numpy(), ref.probs)


def test_one_workspace_serves_every_batch_size_in_a_graph(gpu):
    """A workspace sized for 64 rows serves B = 64, 17 and 1 in one captured
    graph (the decode loop's varying batch), replayed with eager work between."""
    V = 248320
    rng = np.random.default_rng(9)
    ws = Workspace(64, V, torch.bfloat16, 0, gpu)
    cases = []
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device=gpu, dtype=dt)
    for B in (64, 17, 1):
        x = _bf16((rng.standard_normal((B, V)) * 2).astype(np.float32))
        T = rng.uniform(0.0, 1.4, B).astype(np.float32)
        T[rng.random(B) < 0.15] = 0.0
        P = rng.uniform(0.5, 1.0, B).astype(np.float32)
        K = rng.integers(0, 800, B).astype(np.int32)
        K[rng.random(B) < 0.2] = 0
        U = rng.random(B).astype(np.float32)
        cases.append(dict(x=x, T=T, P=P, K=K, U=U, lg=_dev_bf16(x, gpu), dT=t(T, torch.float32),
                          dP=t(P, torch.float32), dK=t(K, torch.int32), dU=t(U, torch.float32),
                          ids=torch.empty(B, dtype=torch.int64, device=gpu)))

    def steps():
        for c in cases:
            sample_into(c["lg"], c["ids"], ws, temperatures=c["dT"], top_ps=c["dP"], top_ks=c["dK"],
                        uniforms=c["dU"], use_top_p=True)

    refs = [contract.sample(c["x"], "bf16", c["T"], c["P"], c["K"], uniforms=c["U"]).ids for c in cases]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        steps()
    for rep in range(3):
        for c in cases:
            c["ids"].fill_(-3)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for c, ref in zip(cases, refs):
            np.testing.assert_array_equal(c["ids"].cpu().numpy(), ref)
        steps()
        torch.cuda.synchronize()
        for c, ref in zip(cases, refs):
            np.testing.assert_array_equal(c["ids"].cpu().numpy(), ref)
