"""The router's softmax forms p / den as div_by_recip(p, den, RN(1/den))
(system-lab_amd/csrc/smoe_common.h): one correctly rounded reciprocal per
token, then a product and two fmas per expert, instead of an IEEE division per
expert.  Markstein's theorem makes that exact for normal quotients; the kernel
sends p < 2^-100 to the IEEE division.  This test checks the identity
bit for bit on the CPU over every significand of the dividend at the
exponents the kernel sees (p in (2^-100, 1]) against divisors in [1, 2048),
so a wrong sign, a missing fma or an unrounded reciprocal shows up as
mismatches."""
import os
import shutil
import subprocess
import tempfile

import pytest

SRC = os.path.join(os.path.dirname(__file__), "csrc", "div_by_recip_check.c")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div_by_recip_is_ieee_division():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "chk")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, SRC, "-lm"], check=True)
        out = subprocess.run([exe, "24", "0", "-1", "-37", "-99"], check=True,
                             capture_output=True, text=True, timeout=300).stdout.split()
    total, bad = int(out[0]), int(out[1])
    assert total == 24 * 4 * (1 << 23)
    assert bad == 0
