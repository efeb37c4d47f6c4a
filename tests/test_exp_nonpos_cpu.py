"""The GPU softmax exponential for non-positive arguments (tl_device.h
tl_expf_nonpos: no clamps, 2^k by ldexp) equals the exponential the oracle
and the other kernels use (tl_expf, branch-free as tl_expf_sel) on every
float in [-90, -0]: the same operation sequence in C (fmaf), compared bit for
bit, the range below the cut-off at -80 included."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_exp_for_nonpositive_arguments_equals_clamped_exp(tmp_path):
    exe = tmp_path / "exp_nonpos_check"
    src = os.path.join(HERE, "exp_nonpos_check.c")
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-fopenmp", "-o", str(exe), src, "-lm"]
    if subprocess.run(cmd, capture_output=True).returncode != 0:   # no OpenMP: one thread
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), src, "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout
    assert "floats in [-90, -0]: 1119092737, mismatches 0" in out.stdout
