"""The e4m3 activation quantisation (quant_group16 in layerbatch_amd/csrc/common.hpp) replaces
the per-value division x / s by a reciprocal and two fused multiply-adds. quant_division_check.c
checks that the sequence rounds exactly as the division on a large sample (binary32, libm fmaf,
no contraction). CPU only."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_matches_division(tmp_path):
    exe = str(tmp_path / "quant_division_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe,
                    os.path.join(HERE, "quant_division_check.c"), "-lm"], check=True)
    r = subprocess.run([exe, "200000"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 mismatches" in r.stdout
