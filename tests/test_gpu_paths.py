"""GPU: every row of the five workloads is resolved on its fast path.

The single-workgroup path is exact but slow; a row that lands there on these
inputs (a region or bracket overflow, an incomplete candidate set) is a
performance bug even though its token is right.  The ids are checked against
the oracle as well, on the first rows.
"""
import numpy as np
import pytest

from qedge_amd import workloads as W
from qedge_amd.sampler import Workspace
from tests.devrun import row_paths, run_gpu, run_oracle, to_device


@pytest.mark.gpu
@pytest.mark.parametrize("name", W.WORKLOADS)
def test_no_single_workgroup_rows(gpu, name):
    w = W.make(name)
    d = to_device(w, gpu)
    B, V = d["logits"].shape
    H = 0 if d["history"] is None else d["history"].shape[1]
    ws = Workspace(B, V, d["logits"].dtype, H, gpu)
    print(f"[paths] {name} B={B}", flush=True)
    ids, _, _ = run_gpu(w, gpu, want_probs=False, ws=ws)
    path, why = row_paths(ws, B)
    bad = np.nonzero(why)[0]
    assert bad.size == 0, f"rows {bad[:8].tolist()} fell back (reasons {why[bad[:8]].tolist()})"
    sub = list(range(min(B, 8)))  # the oracle on a few rows: the full batches take it minutes
    np.testing.assert_array_equal(ids[sub], run_oracle(W.make(name, rows=sub), want_probs=False).ids)
