"""The packed grouped GEMMs (system-lab_amd/csrc/smoe_gemm_packed.hip and
smoe_gemm_e8m0.hip) mix activation DMAs issued as inline asm, which the
compiler does not count, with weight loads into registers whose waits the
compiler places itself.  Both retire through one in-order counter, so the
compiler's waits can only wait longer than needed; this compiles each
kernel source with the library's flags and
checks, counting every memory instruction as the hardware does, that no
register of a weight load is read, copied or overwritten before a wait that
covers it (tests/asm_inflight.py).  The scanner is first held to snippets
with and without a hazard."""
import os
import shutil
import subprocess
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import asm_inflight  # noqa: E402

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

GOOD = """\
\tglobal_load_dwordx4 v[30:33], v199, s[0:1]
\tglobal_load_lds_dwordx4 v2, s[4:5]
\tv_mfma_f32_16x16x128_f8f6f4 v[40:43], v[2:9], v[10:17], 0
\ts_waitcnt vmcnt(1)
\tv_mov_b32_e32 v50, v30
"""
READ_EARLY = """\
\tglobal_load_dwordx4 v[30:33], v199, s[0:1]
\tglobal_load_lds_dwordx4 v2, s[4:5]
\ts_waitcnt vmcnt(2)
\tv_mov_b64_e32 v[2:3], v[30:31]
"""
REUSED = """\
\tglobal_load_dwordx4 v[30:33], v199, s[0:1]
\tv_or_b32_e32 v30, 0x20400, v19
\ts_waitcnt vmcnt(0)
"""
LOOP = """\
.LBB0_1:
\tv_mov_b32_e32 v60, v30
\tglobal_load_dwordx4 v[30:33], v199, s[0:1]
\ts_cbranch_scc1 .LBB0_1
\ts_waitcnt vmcnt(0)
"""


def test_scanner_flags_hazards_and_passes_clean_code():
    assert asm_inflight.check(GOOD) == []
    assert [h[0] for h in asm_inflight.check(READ_EARLY)] == [4]
    assert [h[0] for h in asm_inflight.check(REUSED)] == [2]
    # a load at a loop's end read at its top, before any wait
    assert [h[0] for h in asm_inflight.check(LOOP)] == [2]


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not found")
@pytest.mark.parametrize("name", ["smoe_gemm_packed", "smoe_gemm_e8m0"])
def test_packed_gemm_has_no_inflight_register_access(tmp_path, name):
    """Both packed-weight GEMM sources, every kernel instantiation in them."""
    sys.path.insert(0, os.path.join(ROOT, "system-lab_amd"))
    from smoe import build
    src = os.path.join(ROOT, "system-lab_amd", "csrc", name + ".hip")
    out = tmp_path / "packed.s"
    flags = [f for f in build.HIP_FLAGS if not f.startswith("-W")]
    subprocess.run([HIPCC, *flags, "--cuda-device-only", "-S", src, "-o", str(out)], check=True,
                   capture_output=True, timeout=600)
    text = out.read_text()
    assert text.count("global_load_dwordx4") >= 8  # the register loads are there
    assert asm_inflight.check(text) == []
