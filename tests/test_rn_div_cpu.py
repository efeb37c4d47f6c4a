"""The GPU quantizers' division by a row-uniform scale (a correctly rounded
reciprocal and two FMA residual corrections, tl_device.h rn_div_fast) equals
correctly rounded division: the same operation sequence in C (fmaf) against
float64 division rounded to float32, on random and near-midpoint quotients."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")
def test_residual_corrected_division_is_correctly_rounded(tmp_path):
    exe = tmp_path / "rn_div_check"
    subprocess.run(["gcc", "-O2", "-mfma", "-o", str(exe), os.path.join(HERE, "rn_div_check.c"), "-lm"], check=True)
    out = subprocess.run([str(exe), "2000000"], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout
    assert "float mismatches 0, rint mismatches 0" in out.stdout
