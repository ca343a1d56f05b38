"""GPU parity: HIP sampler vs the CPU oracle on the five workloads (exact ids)."""
import numpy as np
import pytest

from qedge_amd import workloads as W
from tests.devrun import run_gpu, run_oracle

SUBSETS = {
    "greedy_spikes_f32": None,
    "topk_topp_rep_bf16": None,
    "hetero_b64_bf16": list(range(0, 64, 4)) + [W.make("hetero_b64_bf16", rows=[0]).notes["topk_off_rows"][0]],
    "penalties_b256_bf16": [0, 1, 2, 3, 100, 255],
    "flat_topp_b1024_f32": [0, 1, 513, 1023],
}


@pytest.mark.gpu
@pytest.mark.parametrize("name", W.WORKLOADS)
def test_workload_parity(gpu, name):
    w = W.make(name, rows=SUBSETS[name])
    print(f"[parity] {name} rows={w.rows}", flush=True)
    ids, probs, kept = run_gpu(w, gpu)
    ref = run_oracle(w)
    np.testing.assert_array_equal(ids, ref.ids)
    np.testing.assert_array_equal(kept, ref.kept)
    np.testing.assert_array_equal(probs, ref.probs)
