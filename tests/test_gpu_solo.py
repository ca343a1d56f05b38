"""GPU parity of the one-workgroup-per-row path (QS_FLAG_SOLO) against the CPU
oracle: ids, surviving-set sizes and post-filter probabilities identical on the
workloads and on the cases that reach its rarer branches (top-k rows, greedy
rows, a bracket of one key too large to list, rows without weights, min_p,
ragged vocabularies).  Needs an MI355X."""
import numpy as np
import pytest
import torch

from oracle import contract
from qedge_amd import workloads as W
from qedge_amd.sampler import Workspace, sample_into
from tests.devrun import row_paths, to_device

pytestmark = pytest.mark.gpu


def _bf16(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _solo(logits, dtype, device, T, P=None, K=None, rep=None, pres=None, freq=None, hist=None, u=None,
          min_p=None, use_top_p=True, pad_to=None):
    B, V = logits.shape
    t = lambda a, dt: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dt)
    if pad_to is not None:
        # rows pad_to apart (16-byte aligned), the columns past V holding +inf,
        # which no call may read
        wide = np.full((B, pad_to), np.inf, np.float32) if dtype == "f32" else np.full((B, pad_to), 0x7F80, np.uint16)
        wide[:, :V] = logits
    src = logits if pad_to is None else wide
    lg = (t(src, torch.float32) if dtype == "f32"
          else torch.from_numpy(np.ascontiguousarray(src).view(np.int16)).to(device).view(torch.bfloat16))
    if pad_to is not None:
        lg = lg[:, :V]
    H = 0 if hist is None else hist.shape[1]
    ws = Workspace(B, V, lg.dtype, H, device)
    ids = torch.empty(B, dtype=torch.int64, device=device)
    probs = torch.empty((B, V), dtype=torch.float32, device=device)
    kept = torch.empty(B, dtype=torch.int32, device=device)
    sample_into(lg, ids, ws, temperatures=t(T, torch.float32), top_ps=t(P, torch.float32), top_ks=t(K, torch.int32),
                repetition_penalties=t(rep, torch.float32), presence_penalties=t(pres, torch.float32),
                frequency_penalties=t(freq, torch.float32), history=t(hist, torch.int32),
                uniforms=t(u, torch.float32), min_ps=t(min_p, torch.float32), use_top_p=use_top_p,
                out_probs=probs, out_kept=kept, solo=True)
    torch.cuda.synchronize()
    path, why = row_paths(ws, B)
    ref = contract.sample(logits, dtype, T, P if use_top_p else None, K, rep, pres, freq, hist, u, want_probs=True,
                          min_p=min_p)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref.ids)
    np.testing.assert_array_equal(kept.cpu().numpy(), ref.kept)
    np.testing.assert_array_equal(probs.cpu().numpy(), ref.probs)
    return path, why


@pytest.mark.parametrize("name", ["penalties_b256_bf16", "flat_topp_b1024_f32", "hetero_b64_bf16",
                                  "topk_topp_rep_bf16", "greedy_spikes_f32"])
def test_workloads_one_workgroup_per_row(gpu, name):
    rows = {"flat_topp_b1024_f32": list(range(0, 1024, 16)), "penalties_b256_bf16": list(range(0, 256, 4))}
    w = W.make(name, rows=rows.get(name))
    path, why = _solo(w.logits, w.dtype, gpu, w.temperature, w.top_p, w.top_k, w.rep, w.pres, w.freq, w.history,
                      w.uniforms(0))
    greedy = w.temperature <= 1e-5
    assert np.all(path[~greedy] == 6) and np.all(why == 0)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_rare_branches(gpu, dtype):
    V = 40961  # ragged: not a multiple of 8
    rng = np.random.default_rng(17)
    rows, T, P, K, MP = [], [], [], [], []
    x = rng.standard_normal(V).astype(np.float32)
    rows.append(np.full(V, 0.25, np.float32)); T.append(1.0); P.append(0.5); K.append(0); MP.append(0.0)  # one key
    rows.append(np.full(V, np.nan, np.float32)); T.append(0.8); P.append(0.9); K.append(0); MP.append(0.0)  # all NaN
    rows.append(x * 3); T.append(0.7); P.append(0.8); K.append(37); MP.append(0.0)       # top-k row
    rows.append(x * 2); T.append(0.9); P.append(1.0); K.append(2000); MP.append(0.0)     # top-k above 1024
    rows.append(x); T.append(0.0); P.append(1.0); K.append(0); MP.append(0.0)            # greedy
    rows.append(x * 4); T.append(1.2); P.append(0.95); K.append(0); MP.append(0.02)      # min_p
    y = (x * 0.05).astype(np.float32); y[rng.integers(V, size=50)] = np.inf
    rows.append(y); T.append(1.0); P.append(0.9); K.append(0); MP.append(0.0)            # +inf tokens
    z = np.round(x * 4) / 4; rows.append(z.astype(np.float32)); T.append(1.0); P.append(0.7); K.append(0); MP.append(0.0)
    v = (x * 0.5).astype(np.float32); v[rng.integers(V, size=300)] = -np.inf; v[rng.integers(V, size=300)] = np.nan
    rows.append(v); T.append(1.0); P.append(0.9); K.append(0); MP.append(0.0)           # -inf and NaN among finite
    n = np.full(V, -np.inf, np.float32); n[rng.integers(V, size=40)] = np.nan
    rows.append(n); T.append(1.0); P.append(0.5); K.append(0); MP.append(0.0)           # maximum -inf
    X = np.stack(rows)
    if dtype == "bf16":
        X = _bf16(X)
    B = X.shape[0]
    U = rng.random(B).astype(np.float32)
    _solo(X, dtype, gpu, np.array(T, np.float32), np.array(P, np.float32), np.array(K, np.int32), u=U,
          min_p=np.array(MP, np.float32))
    # without top-p
    _solo(X, dtype, gpu, np.array(T, np.float32), None, np.array(K, np.int32), u=U, use_top_p=False)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("V", [40961, 3 * 8192 + 5, 16387])
def test_strided_rows_with_a_vector_across_v(gpu, dtype, V):
    """Rows 16-byte aligned with V not a multiple of the vector: the vector
    holding id V - 1 is read by elements, nothing past V is read."""
    rng = np.random.default_rng(V)
    B = 6
    X = (rng.standard_normal((B, V)) * np.array([[0.05], [1.0], [3.0], [2.0], [1.0], [0.5]])).astype(np.float32)
    X[1, V - 1] = 9.0  # the last id is the largest of row 1
    if dtype == "bf16":
        X = _bf16(X)
    T = np.array([1.0, 0.8, 1.0, 0.0, 1.3, 1.0], np.float32)
    P = np.array([0.95, 0.9, 0.5, 1.0, 0.99, 1.0], np.float32)
    K = np.array([0, 0, 0, 0, 50, 0], np.int32)
    MP = np.array([0.0, 0.0, 0.0, 0.0, 0.0, 0.01], np.float32)
    pad = (V + 15) // 16 * 16 + 16
    _solo(X, dtype, gpu, T, P, K, u=rng.random(B).astype(np.float32), min_p=MP, pad_to=pad)


def test_penalties_and_long_histories(gpu):
    B, V, H = 6, 70000, 6000  # histories longer than the ids kept in LDS
    rng = np.random.default_rng(23)
    X = _bf16((rng.standard_normal((B, V)) * 2).astype(np.float32))
    hist = rng.integers(-5, V + 5, size=(B, H)).astype(np.int32)  # with padding ids outside [0, V)
    hist[:, :300] = rng.integers(0, 50, size=(B, 300))  # a few ids counted many times
    T = np.array([0.8, 1.0, 0.0, 1.3, 0.6, 0.9], np.float32)
    P = np.array([0.95, 0.9, 1.0, 0.99, 0.5, 1.0], np.float32)
    rep = np.array([1.1, 1.3, 1.2, 1.0, 1.05, 2.0], np.float32)
    pres = np.array([0.5, 0.0, 0.3, 0.2, 0.0, 1.0], np.float32)
    freq = np.array([0.3, 0.1, 0.0, 0.05, 0.5, 0.0], np.float32)
    _solo(X, "bf16", gpu, T, P, None, rep, pres, freq, hist, rng.random(B).astype(np.float32))


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_long_rows(gpu, dtype):
    """V = 600001: 74 chunks, 592 segments per row."""
    V = 600001
    rng = np.random.default_rng(41)
    X = (rng.standard_normal((3, V)) * np.array([[0.05], [1.5], [3.0]])).astype(np.float32)
    if dtype == "bf16":
        X = _bf16(X)
    T = np.array([1.0, 0.7, 1.1], np.float32)
    P = np.array([0.95, 0.9, 0.6], np.float32)
    _solo(X, dtype, gpu, T, P, u=rng.random(3).astype(np.float32))
