"""Malformed arguments are refused on the host by the ops layer
(system-lab_amd/smoe/ops.py): each case below raises ValueError (TypeError
for a wrong dtype) before any kernel is launched, so a wrong shape, dtype or length can never become an
out-of-bounds device access.  One case per op that hands raw pointers to the
library, including every caller-supplied ``out=``."""
import pytest
import torch

from smoe import ops

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
BAD = (ValueError, TypeError)


def _z(shape, dtype, dev):
    return torch.zeros(shape, dtype=dtype, device=dev)


def test_unpermute_combine_out(dev):
    T, K, H = 4, 2, 128
    y = _z((T * K, H), torch.bfloat16, dev)
    inv = torch.arange(T * K, dtype=torch.int32, device=dev)
    w = _z((T, K), torch.float32, dev)
    with pytest.raises(BAD):
        ops.unpermute_combine(y, inv, w, out=_z((T, H + 128), torch.bfloat16, dev))
    with pytest.raises(BAD):
        ops.unpermute_combine(y, inv, w, out=_z((T, H), torch.float32, dev))
    with pytest.raises(BAD):
        ops.unpermute_combine(y, inv[:-1], w)


def test_grouped_gemm_out_and_scales(dev):
    R, K, N, E = 8, 128, 256, 2
    xq, xs = _z((R, K), FP8, dev), _z((R, 1), torch.float32, dev)
    wq, ws = _z((E, N, K), FP8, dev), _z((E, 2, 1), torch.float32, dev)
    off = torch.tensor([0, 4, 8], dtype=torch.int32, device=dev)
    with pytest.raises(BAD):
        ops.grouped_gemm_fp8(xq, xs, wq, ws, off, out=_z((R, N - 128), torch.bfloat16, dev))
    with pytest.raises(BAD):
        ops.grouped_gemm_fp8(xq, xs, wq, _z((E, 1, 1), torch.float32, dev), off)
    with pytest.raises(BAD):
        ops.grouped_gemm_fp8(xq, xs, wq, ws, off[:-1])


def test_wgrad_scales_and_out(dev):
    E, N, K = 2, 128, 256
    off = torch.tensor([0, 100, 300], dtype=torch.int32, device=dev)
    a = _z((300, N), torch.bfloat16, dev)
    b = _z((300, K), torch.bfloat16, dev)
    aq, as_, pad, ld = ops.quant_cols(a, off)
    bq, bs_, _, _ = ops.quant_cols(b, off)
    with pytest.raises(BAD):
        ops.grouped_gemm_fp8_wgrad(aq, as_[:, :-1], bq, bs_, pad, ld)
    with pytest.raises(BAD):
        ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld, out=_z((E, N, K - 128), torch.float32, dev))
    with pytest.raises(BAD):
        ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld - 128)


def test_quant_cols_gather_bound(dev):
    off = torch.tensor([0, 8], dtype=torch.int32, device=dev)
    x = _z((3, 128), torch.bfloat16, dev)           # 3 rows
    gather = torch.arange(8, dtype=torch.int32, device=dev)
    with pytest.raises(BAD):                  # gather // 2 reaches row 3
        ops.quant_cols(x, off, gather, gather_div=2)
    with pytest.raises(BAD):
        ops.quant_cols(x, off, gather, gather_div=0)


def test_transpose_blockwise_scale_grid(dev):
    wq = _z((1, 256, 128), FP8, dev)
    with pytest.raises(BAD):
        ops.transpose_blockwise(wq, _z((1, 1, 1), torch.float32, dev))


def test_combine_bwd_shapes(dev):
    T, K, H = 4, 2, 128
    w = _z((T, K), torch.float32, dev)
    inv = torch.arange(T * K, dtype=torch.int32, device=dev)
    with pytest.raises(BAD):
        ops.unpermute_combine_bwd(_z((T + 1, H), torch.bfloat16, dev), _z((T * K, H), torch.bfloat16, dev),
                                  inv, w)
    with pytest.raises(BAD):
        ops.unpermute_combine_bwd(_z((T, H), torch.bfloat16, dev), _z((T * K - 1, H), torch.bfloat16, dev),
                                  inv, w)


def test_router_shapes(dev):
    T, E, K = 4, 8, 2
    lg = _z((T, E), torch.float32, dev)
    with pytest.raises(BAD):
        ops.router_topk(lg, K, _z((E - 1,), torch.float32, dev))
    with pytest.raises(BAD):
        ops.router_topk_bwd(lg, _z((T, K + 1), torch.int32, dev), _z((T, K), torch.float32, dev))
    with pytest.raises(BAD):
        ops.permute_quant_rows(_z((T, 128), torch.bfloat16, dev),
                               _z((T * K - 1,), torch.int32, dev), K)
