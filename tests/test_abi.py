"""The C-ABI library loads, exports every entry point include/smoe.h
declares, and rejects bad arguments on the host (no GPU needed: every case
here returns before any HIP call)."""
import ctypes
import os
import re

import pytest

from smoe import _C

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "smoe.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(smoe_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    names = declared()
    assert len(names) >= 12
    assert sorted(_C.SIGNATURES) == names


def test_library_exports_every_declared_symbol():
    lib = _C.lib()
    for n in declared():
        assert hasattr(lib, n), n
    assert lib.smoe_version().decode().startswith("smoe")


def test_strerror_covers_codes():
    lib = _C.lib()
    for code in range(0, -9, -1):
        assert lib.smoe_strerror(code)
    assert b"unknown" in lib.smoe_strerror(-99)


FAKE = 0x100000  # aligned, never dereferenced: validation fails first
MIS = FAKE + 4


@pytest.mark.parametrize("args,code", [
    ((None, FAKE, 4, 256, 2, FAKE, FAKE, None), -1),      # x NULL
    ((FAKE, FAKE, 4, 200, 2, FAKE, FAKE, None), -3),      # H % 128
    ((FAKE, FAKE, 0, 256, 2, FAKE, FAKE, None), -2),      # T == 0
    ((FAKE, FAKE, 4, 256, 0, FAKE, FAKE, None), -7),      # K == 0
    ((MIS, FAKE, 4, 256, 2, FAKE, FAKE, None), -6),       # misaligned x
])
def test_permute_quant_rejects(args, code):
    assert _C.lib().smoe_permute_quant(*args) == code


def test_route_sort_rejects():
    lib = _C.lib()
    need = lib.smoe_route_sort_workspace_size(16, 2, 8)
    assert need > 0
    ok = (FAKE, 16, 2, 8, FAKE, FAKE, FAKE, FAKE)
    assert lib.smoe_route_sort(*ok, FAKE, need - 1, None) == -5
    assert lib.smoe_route_sort(*ok, None, need, None) == -5
    assert lib.smoe_route_sort(FAKE, 16, 9, 8, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None) == -7
    assert lib.smoe_route_sort(FAKE, 16, 2, 0, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None) == -4
    assert lib.smoe_route_sort(FAKE, 16, 2, 2000, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None) == -4
    assert lib.smoe_route_sort(None, 16, 2, 8, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None) == -1


def test_route_topk_sort_rejects():
    lib = _C.lib()
    need = lib.smoe_route_sort_workspace_size(16, 2, 8)
    f = lib.smoe_route_topk_sort
    ok = (FAKE, None, 16, 8, 2, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE)
    assert f(*ok, FAKE, need - 1, None) == -5
    assert f(*ok, None, need, None) == -5
    assert f(*ok, MIS, need, None) == -6
    assert f(None, None, 16, 8, 2, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need, None) == -1
    assert f(FAKE, None, 16, 8, 9, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need, None) == -7
    assert f(FAKE, None, 16, 2000, 2, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need, None) == -4
    assert f(FAKE, None, 0, 8, 2, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, need, None) == -2


def test_gemm_swiglu_combine_router_reject():
    lib = _C.lib()
    g = lib.smoe_grouped_gemm_fp8
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 100, 256, 100, FAKE, None, 0, None) == -3
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 100, 256, 256, FAKE, None, 0, None) == -4
    assert g(FAKE, FAKE, FAKE, FAKE, None, 4, 100, 256, 256, FAKE, None, 0, None) == -1
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 0, 256, 256, FAKE, None, 0, None) == -2
    assert lib.smoe_swiglu_quant(FAKE, 10, 100, FAKE, FAKE, None) == -3
    assert lib.smoe_swiglu_quant(FAKE, 10, 128, None, FAKE, None) == -1
    assert lib.smoe_unpermute_combine(FAKE, FAKE, FAKE, 4, 2, 130, FAKE, None) == -3
    assert lib.smoe_unpermute_combine(FAKE, FAKE, FAKE, 4, 33, 128, FAKE, None) == -7
    assert lib.smoe_router_topk(FAKE, None, 4, 8, 9, FAKE, FAKE, None) == -7
    assert lib.smoe_router_topk(FAKE, None, 4, 1025, 2, FAKE, FAKE, None) == -4
    assert lib.smoe_quantize_weight_blockwise(FAKE, 2, 128, 100, FAKE, FAKE, None) == -3
    assert lib.smoe_grouped_gemm_fp8_workspace_size(4, 100, 256, 256) == 0


def test_ops_refuse_cpu_tensors():
    import torch
    from smoe import ops
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.router_topk(torch.zeros(4, 8), 2)


def test_remaining_entry_points_reject():
    """Every other entry point returns its documented code on the host for
    malformed arguments (the checks run before any HIP call)."""
    lib = _C.lib()
    # fused fc1 + SwiGLU: I % 128, experts, 2*I*Kdim >= 2^31, hs NULL, misaligned c1
    f = lib.smoe_grouped_gemm_fp8_swiglu
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 100, 192, 256, FAKE, FAKE, None, None) == -3
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 100, 256, 256, FAKE, FAKE, None, None) == -4
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 100, 131072, 8192, FAKE, FAKE, None, None) == -2
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 100, 256, 256, FAKE, None, None, None) == -1
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 100, 256, 256, FAKE, FAKE, MIS, None) == -6
    # dispatch: H % 128, T == 0, sort workspace missing
    d = lib.smoe_dispatch_quant
    assert d(FAKE, FAKE, 16, 200, 2, 8, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None) == -3
    assert d(FAKE, FAKE, 0, 256, 2, 8, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1 << 20, None) == -2
    assert d(FAKE, FAKE, 16, 256, 2, 8, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, None) == -5
    # column quantiser: C % 128, experts, ld too small, gather_div, offsets NULL
    q = lib.smoe_quant_cols_128x1
    ld = lib.smoe_quant_cols_ld(1000, 4)
    assert ld >= 1000 and ld % 128 == 0
    assert q(FAKE, None, 1, 1000, 100, FAKE, 4, ld, FAKE, FAKE, FAKE, 0, None) == -3
    assert q(FAKE, None, 1, 1000, 128, FAKE, 0, ld, FAKE, FAKE, FAKE, 0, None) == -4
    assert q(FAKE, None, 1, 1000, 128, FAKE, 4, ld - 128, FAKE, FAKE, FAKE, 0, None) == -2
    assert q(FAKE, FAKE, 0, 1000, 128, FAKE, 4, ld, FAKE, FAKE, FAKE, 0, None) == -2
    assert q(FAKE, None, 1, 1000, 128, None, 4, ld, FAKE, FAKE, FAKE, 0, None) == -1
    # wgrad: N % 128, experts, ld <= 0, pad NULL
    w = lib.smoe_grouped_gemm_fp8_wgrad
    assert w(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 100, 256, 1024, FAKE, None) == -3
    assert w(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 256, 256, 1024, FAKE, None) == -4
    assert w(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 256, 256, 0, FAKE, None) == -2
    assert w(FAKE, FAKE, FAKE, FAKE, None, 4, 256, 256, 1024, FAKE, None) == -1
    # SwiGLU backward, combine backward, transpose, row quantiser
    assert lib.smoe_swiglu_bwd(FAKE, FAKE, 10, 100, FAKE, None) == -3
    assert lib.smoe_swiglu_bwd(FAKE, FAKE, 0, 128, FAKE, None) == -2
    cb = lib.smoe_unpermute_combine_bwd
    assert cb(FAKE, FAKE, FAKE, FAKE, 4, 2, 130, FAKE, FAKE, None) == -3
    assert cb(FAKE, FAKE, FAKE, FAKE, 4, 33, 128, FAKE, FAKE, None) == -7
    assert cb(FAKE, FAKE, FAKE, None, 4, 2, 128, FAKE, FAKE, None) == -1
    t = lib.smoe_transpose_blockwise_fp8
    assert t(FAKE, FAKE, 2, 100, 128, FAKE, FAKE, None) == -3
    assert t(FAKE, FAKE, 0, 128, 128, FAKE, FAKE, None) == -4
    assert t(FAKE, None, 2, 128, 128, FAKE, FAKE, None) == -1
    assert lib.smoe_quant_rows_1x128(FAKE, 10, 100, FAKE, FAKE, None) == -3
    assert lib.smoe_quant_rows_1x128(FAKE, 0, 128, FAKE, FAKE, None) == -2
    # one-read row + column quantiser: C % 128, experts, ld too small, xs NULL
    rc = lib.smoe_quant_rows_cols
    assert rc(FAKE, 1000, 100, FAKE, 4, ld, FAKE, FAKE, FAKE, FAKE, FAKE, 0, None) == -3
    assert rc(FAKE, 1000, 128, FAKE, 0, ld, FAKE, FAKE, FAKE, FAKE, FAKE, 0, None) == -4
    assert rc(FAKE, 1000, 128, FAKE, 4, ld - 128, FAKE, FAKE, FAKE, FAKE, FAKE, 0, None) == -2
    assert rc(FAKE, 1000, 128, FAKE, 4, ld, FAKE, None, FAKE, FAKE, FAKE, 0, None) == -1
    sb = lib.smoe_swiglu_bwd_quant
    assert sb(FAKE, FAKE, 1000, 100, FAKE, 4, ld, FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, None) == -3
    assert sb(FAKE, FAKE, 1000, 128, FAKE, 0, ld, FAKE, FAKE, FAKE, FAKE, FAKE, None, 0, None) == -4
    assert sb(FAKE, FAKE, 1000, 128, FAKE, 4, ld, FAKE, FAKE, FAKE, FAKE, FAKE, MIS, 0, None) == -6
    # fused combine backward + quantiser: H % 128, top-k, experts, ld too small, row_map NULL
    cq = lib.smoe_unpermute_combine_bwd_quant
    ld2 = lib.smoe_quant_cols_ld(1000, 4)
    args = lambda T=500, K=2, H=128, E=4, ld=ld2, rm=FAKE: (
        FAKE, FAKE, FAKE, rm, FAKE, T, K, H, FAKE, E, ld, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 0, None)
    assert cq(*args(H=130)) == -3
    assert cq(*args(K=33)) == -7
    assert cq(*args(E=0)) == -4
    assert cq(*args(ld=ld2 - 128)) == -2
    assert cq(*args(rm=None)) == -1
    # dyTq and dyTs both NULL skip the column pass; only one of them NULL is an error
    one_null = list(args()); one_null[13] = None
    assert cq(*one_null) == -1
    # its column pass alone: the same checks, the column bit only
    cc = lib.smoe_combine_bwd_quant_cols
    cargs = lambda T=500, K=2, H=128, E=4, ld=ld2, rm=FAKE, mode=0: (
        FAKE, rm, FAKE, T, K, H, FAKE, E, ld, FAKE, FAKE, FAKE, mode, None)
    assert cc(*cargs(H=130)) == -3
    assert cc(*cargs(K=33)) == -7
    assert cc(*cargs(E=0)) == -4
    assert cc(*cargs(ld=ld2 - 128)) == -2
    assert cc(*cargs(rm=None)) == -1
    assert cc(*cargs(mode=2)) == -8 and cc(*cargs(mode=-1)) == -8
    # a column-scale rule other than SMOE_COLSCALE_FP32 / _POW2
    assert q(FAKE, None, 1, 1000, 128, FAKE, 4, ld, FAKE, FAKE, FAKE, 2, None) == -8
    assert rc(FAKE, 1000, 128, FAKE, 4, ld, FAKE, FAKE, FAKE, FAKE, FAKE, -1, None) == -8
    # SwiGLU with the bf16 h output: misaligned h; the quantiser self-test
    assert lib.smoe_swiglu_quant_h(FAKE, 10, 128, FAKE, FAKE, MIS, None) == -6
    assert lib.smoe_selftest_quant(None, None) == -1
    assert lib.smoe_selftest_quant(MIS, None) == -6
    assert lib.smoe_selftest_recip(None, None) == -1
    assert lib.smoe_selftest_recip(MIS, None) == -6


def test_wgrad_ex_and_packed_bounds_reject():
    """The wgrad output-mode entry rejects a mode outside SMOE_WGRAD_* (with
    the optional SMOE_WGRAD_E8M0 bit) and the plain wgrad's bad shapes; the packed GEMM's K limit (the weight-scale
    column of a tile lives in LDS: K <= 65536) is the same in the C check
    and in ops.packed_gemm_ok, so SimpleMoE never packs a weight the packed
    entry point would refuse."""
    from smoe import ops
    lib = _C.lib()
    w = lib.smoe_grouped_gemm_fp8_wgrad_ex
    assert w(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 256, 256, 1024, FAKE, 8, None) == -8
    assert w(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 256, 256, 1024, FAKE, -1, None) == -8
    assert w(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 100, 256, 1024, FAKE, 1, None) == -3
    assert w(FAKE, FAKE, FAKE, FAKE, None, 4, 256, 256, 1024, FAKE, 3, None) == -1
    p = lib.smoe_grouped_gemm_fp8_packed
    K = 65536 + 512
    assert not ops.packed_gemm_ok(128, K)
    assert p(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 128, K, FAKE, None) == -2
    assert ops.packed_gemm_ok(128, 65536)
    assert not ops.packed_gemm_ok(128, 0) and not ops.packed_gemm_ok(128, 1536 + 128)


def test_scale_mode_entries_reject():
    """The _ex quantisers take SMOE_SCALE_AMAX (0) or SMOE_SCALE_POW2 (1) and
    nothing else; the column quantiser takes only the column bit, the fused
    row-and-column quantisers also the row bit (2); the E8M0 GEMM takes K a
    multiple of 128 from 512 to 65536 (ops.packed_e8m0_ok says the same),
    its fused SwiGLU form also I a multiple of 128.
    All rejected before any launch."""
    from smoe import ops
    assert ops.packed_e8m0_ok(128, 640) and ops.packed_e8m0_ok(128, 65536)
    assert not ops.packed_e8m0_ok(128, 384) and not ops.packed_e8m0_ok(128, 576)
    assert not ops.packed_e8m0_ok(120, 1024) and not ops.packed_e8m0_ok(128, 65536 + 128)
    lib = _C.lib()
    for mode in (2, -1):
        assert lib.smoe_permute_quant_ex(FAKE, FAKE, 4, 256, 2, FAKE, FAKE, mode, None) == -8
        assert lib.smoe_quant_rows_1x128_ex(FAKE, 4, 256, FAKE, FAKE, mode, None) == -8
        assert lib.smoe_swiglu_quant_ex(FAKE, 4, 256, FAKE, FAKE, None, mode, None) == -8
        assert lib.smoe_quantize_weight_blockwise_ex(FAKE, 2, 256, 256, FAKE, FAKE, mode, None) == -8
    # the other checks still come first for a valid mode
    assert lib.smoe_permute_quant_ex(None, FAKE, 4, 256, 2, FAKE, FAKE, 1, None) == -1
    assert lib.smoe_quant_rows_1x128_ex(FAKE, 4, 200, FAKE, FAKE, 1, None) == -3
    assert lib.smoe_swiglu_quant_ex(FAKE, 4, 256, FAKE, FAKE, MIS + 8, 1, None) == -6
    assert lib.smoe_quantize_weight_blockwise_ex(FAKE, 0, 256, 256, FAKE, FAKE, 1, None) == -4
    ld = lib.smoe_quant_cols_ld(256, 2)
    assert lib.smoe_quant_cols_128x1(FAKE, None, 1, 256, 256, FAKE, 2, ld, FAKE, FAKE, FAKE, 2,
                                     None) == -8
    assert lib.smoe_quant_rows_cols(FAKE, 256, 256, FAKE, 2, ld, FAKE, FAKE, FAKE, FAKE, FAKE, 4,
                                    None) == -8
    assert lib.smoe_quant_rows_cols(None, 256, 256, FAKE, 2, ld, FAKE, FAKE, FAKE, FAKE, FAKE, 3,
                                    None) == -1
    assert lib.smoe_swiglu_bwd_quant(FAKE, FAKE, 256, 128, FAKE, 2, ld, FAKE, FAKE, FAKE, FAKE,
                                     FAKE, None, 7, None) == -8
    assert lib.smoe_unpermute_combine_bwd_quant(FAKE, FAKE, FAKE, FAKE, FAKE, 128, 2, 256, FAKE,
                                                2, ld, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, -2,
                                                None) == -8
    g = lib.smoe_grouped_gemm_fp8_packed_e8m0
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 128, 576, FAKE, None) == -3   # K % 128
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 128, 384, FAKE, None) == -2   # K < 512
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 120, 1024, FAKE, None) == -3  # N % 16
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 128, 65536 + 512, FAKE, None) == -2
    # the fused SwiGLU form: I % 128, its K range, hs NULL, misaligned c1
    f = lib.smoe_grouped_gemm_fp8_packed_e8m0_swiglu
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 192, 1024, FAKE, FAKE, None, None) == -3
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 0, 1024, FAKE, FAKE, None, None) == -2
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 256, 384, FAKE, FAKE, None, None) == -2
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 256, 576, FAKE, FAKE, None, None) == -3
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 256, 640, FAKE, None, None, None) == -1
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 256, 256, 640, FAKE, FAKE, MIS, None) == -6
    assert f(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 256, 256, 640, FAKE, FAKE, None, None) == -4
    assert g(FAKE, FAKE, FAKE, FAKE, FAKE, 0, 256, 128, 1024, FAKE, None) == -4
    assert g(FAKE, None, FAKE, FAKE, FAKE, 2, 256, 128, 1024, FAKE, None) == -1
    assert g(FAKE, FAKE + 2, FAKE, FAKE, FAKE, 2, 256, 128, 1024, FAKE, None) == -6
