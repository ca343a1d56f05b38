"""The 16-bit keys of bf16 logits that the kernels compare two per register
(qs_device.hpp hkey2 / key_of_h, qs_kernels.hpp bf16_of_h), checked on the host
over every bf16 bit pattern in both halves of a register: order as the values
(NaN below -inf, -0 just below +0), the NaN/-inf boundary the thresholds rely
on, key_of_h equal to the value's order key, bf16_of_h inverting hkey2, and the
greedy offset putting every NaN above +inf.  The functions are compiled from
the kernel headers themselves (host side of hipcc)."""
import os
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    return None


def test_h_keys_over_every_bf16_pattern():
    cc = _hipcc()
    if cc is None:
        pytest.skip("hipcc not found")
    out = os.path.join(tempfile.mkdtemp(), "hkey_check")
    subprocess.run([cc, "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), "-I",
                    os.path.join(ROOT, "qedge_amd", "csrc"), "-o", out, os.path.join(HERE, "cdiv", "hkey_check.cpp")],
                   check=True, capture_output=True)
    r = subprocess.run([out], check=True, capture_output=True, text=True)
    assert int(r.stdout.split()[0]) == 0
