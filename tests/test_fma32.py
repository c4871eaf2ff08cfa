"""oracle.fma32 (the float64 emulation of the GPU's single-rounding fp32
fma that the exp routine uses) against C's fmaf, which is correctly rounded,
bit for bit.  Triples: random values over a wide exponent range; cancelling
ones (c close to -a*b, where the exact residual decides); and exact ties
(a*b a float32 rounding midpoint) with c = 0 and with c a tiny nudge either
way, which only the round-to-odd step gets right."""
import os
import shutil
import subprocess
import sys
import tempfile

import numpy as np
import pytest

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from oracle import smoe_oracle as O  # noqa: E402

SRC = os.path.join(os.path.dirname(__file__), "csrc", "fmaf_check.c")


def _triples(n=400_000, seed=7):
    rng = np.random.default_rng(seed)
    f = lambda k: (rng.standard_normal(k) * np.exp2(rng.integers(-40, 40, k))).astype(np.float32)
    a, b, c = f(n), f(n), f(n)
    # cancellation: c = -RN(a*b) + a few ulps
    a2, b2 = f(n), f(n)
    pr = (a2.astype(np.float64) * b2).astype(np.float32)
    c2 = (-pr + np.spacing(pr) * rng.integers(-3, 4, n).astype(np.float32)).astype(np.float32)
    # exact ties: (1 + i*2^-12)(1 + j*2^-12) has bits below float32's last
    m = 20_000
    i = rng.integers(1, 1 << 11, m) * 2 + 1
    j = rng.integers(1, 1 << 11, m) * 2 + 1
    a3 = (1.0 + i * 2.0 ** -12).astype(np.float32)
    b3 = (1.0 + j * 2.0 ** -12).astype(np.float32)
    tiny = np.exp2(rng.integers(-70, -40, m)).astype(np.float32)
    c3 = np.concatenate([np.zeros(m, np.float32), tiny, -tiny])
    a3, b3 = np.tile(a3, 3), np.tile(b3, 3)
    return (np.concatenate([a, a2, a3]), np.concatenate([b, b2, b3]),
            np.concatenate([c, c2, c3]))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_fma32_equals_fmaf():
    a, b, c = _triples()
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "fmaf_check")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, SRC, "-lm"], check=True)
        inp = np.stack([a, b, c], 1).astype(np.float32).tobytes()
        out = subprocess.run([exe], input=inp, capture_output=True, check=True, timeout=120).stdout
    ref = np.frombuffer(out, np.float32)
    with np.errstate(all="ignore"):
        got = O.fma32(a, b, c)
    fin = np.isfinite(ref)
    assert fin.mean() > 0.99
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
