"""The oracle and the workload generator reproduce the committed golden vectors
(tests/golden/oracle_vectors.npz, written by tests/golden/make_golden.py)."""
import os

import numpy as np
import pytest

from oracle import contract
from qedge_amd import workloads as W
from tests.golden.make_golden import WORKLOAD_ROWS, digest, mixed_problem, solve

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "oracle_vectors.npz"))


@pytest.mark.parametrize("tag,seed,B,V,dtype", [("mix_f32", 11, 12, 777, "f32"), ("mix_bf16", 12, 12, 1500, "bf16")])
def test_mixed_problems(tag, seed, B, V, dtype):
    prob = mixed_problem(seed, B, V, dtype)
    for k, v in prob.items():
        np.testing.assert_array_equal(v, GOLD[f"{tag}/{k}"])
    res = solve(prob, dtype)
    np.testing.assert_array_equal(res.ids, GOLD[f"{tag}/ids"])
    np.testing.assert_array_equal(res.kept, GOLD[f"{tag}/kept"])
    np.testing.assert_array_equal(res.probs, GOLD[f"{tag}/probs"])


@pytest.mark.parametrize("name", list(WORKLOAD_ROWS))
def test_workload_rows(name):
    w = W.make(name, rows=WORKLOAD_ROWS[name])
    np.testing.assert_array_equal(np.array([digest(r) for r in w.logits], np.uint64), GOLD[f"{name}/logits_digest"])
    res = contract.sample_workload(w, want_probs=True)
    np.testing.assert_array_equal(res.ids, GOLD[f"{name}/ids"])
    np.testing.assert_array_equal(res.kept, GOLD[f"{name}/kept"])
    np.testing.assert_array_equal(res.kend, GOLD[f"{name}/topk_end"])
    assert [format(x, "x") for x in res.W] == list(GOLD[f"{name}/W_hex"])
    np.testing.assert_allclose(res.probs.astype(np.float64).sum(axis=1), GOLD[f"{name}/probs_sum"], rtol=0, atol=0)
