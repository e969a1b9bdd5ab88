"""The quantize kernel divides the group range by 15 without a division
instruction (div15 in marlin-mlx_amd/csrc/mq4_quantize.hip: one Markstein
step with the constant RN(1/15)).  tests/cpp/div15_check.c restates that
sequence in C (float arithmetic and fmaf, correctly rounded on the host) and
compares it with IEEE x / 15 bit for bit: here over every 97th non-negative
float, every subnormal and every float in [2^-30, 2^-20]; run with stride 1
it covers all 2^31 non-negative floats (about 45 s), also without a
mismatch."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div15_matches_ieee_division(tmp_path):
    exe = tmp_path / "div15_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(HERE, "cpp", "div15_check.c"), "-lm"], check=True)
    r = subprocess.run([str(exe), "97"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches: 0" in r.stdout
