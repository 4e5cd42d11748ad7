"""The rounding identity the quantisation kernels rely on (qmm.hip qmm_quant).

Acts::new rounds half away from zero (qmm.rs:1194-1201, f32::round).  The
kernels compute it as trunc(t + copysign(0.5 - 2^-25, t)) -- one add and one
truncation -- which is exact only because of how f32 addition rounds near the
halves; this test compiles tests/cpp/round_away_check.c and checks the form
against roundf bit for bit over all 2^32 bit patterns (finite ones), about 20
seconds on one core.
"""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_trunc_form_equals_roundf_on_every_float(tmp_path):
    exe = tmp_path / "round_away_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(HERE, "cpp", "round_away_check.c"), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout
    assert " 0 differ" in res.stdout
