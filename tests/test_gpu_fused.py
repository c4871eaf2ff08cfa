"""GPU parity of the fused fc1 GEMM + SwiGLU + 1x128 requant epilogue.

The fused entry point (smoe_grouped_gemm_fp8_swiglu) must produce the same
bytes as the two-kernel path it replaces: smoe_grouped_gemm_fp8 -> bf16 c1 ->
smoe_swiglu_quant.  Both halves of that path are pinned against the oracle
elsewhere (the GEMM to the float64 oracle within the GEMM tolerance, the
SwiGLU requant bit-exactly), so bit-equality with it is the bar here: hq and
hs byte for byte, and the optional c1 output byte for byte."""
import sys

import numpy as np
import pytest
import torch

from oracle import smoe_oracle as O
import smoe
from smoe import ops, workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def _bytes(t):
    return t.detach().contiguous().view(torch.uint8)


def _operands(dev, rng, R, I, Kd, E):
    x = rng.standard_normal((R, Kd)).astype(np.float32)
    if R > 2:
        x[1] = 0.0    # an all-zero row: c1 = 0, h = 0, group scale 1
        x[2] *= 300.  # a large row: silu saturates to g, large h
    xq, xs = O.quant_1x128(x)
    w = (torch.randn((E, 2 * I, Kd), generator=torch.Generator().manual_seed(R + I)) * 0.05)
    wq, ws = ops.quantize_weight_blockwise(w.to(torch.bfloat16).to(dev))
    return (torch.from_numpy(xq).view(torch.float8_e4m3fn).to(dev), torch.from_numpy(xs).to(dev),
            wq, ws)


def _check_same(dev, xq, xs, wq, ws, off):
    c1 = ops.grouped_gemm_fp8(xq, xs, wq, ws, off)
    rq, rs = ops.swiglu_quant(c1)
    hq, hs = ops.grouped_gemm_fp8_swiglu(xq, xs, wq, ws, off)
    hq2, hs2, c1f = ops.grouped_gemm_fp8_swiglu(xq, xs, wq, ws, off, save_c1=True)
    torch.cuda.synchronize()
    lo, hi = int(off[0]), int(off[-1])
    for q, s in ((hq, hs), (hq2, hs2)):
        assert torch.equal(_bytes(q[lo:hi]), _bytes(rq[lo:hi])), "hq bytes differ"
        assert torch.equal(s[lo:hi].view(torch.int32), rs[lo:hi].view(torch.int32)), "hs differ"
    assert torch.equal(c1f[lo:hi].view(torch.int16), c1[lo:hi].view(torch.int16)), "c1 differs"


@pytest.mark.parametrize("counts,I,Kd", [([5, 0, 300, 1, 0, 129, 128, 17], 256, 512),
                                         ([0, 0, 1000], 512, 1024),
                                         ([1], 128, 128),
                                         ([700, 3], 768, 256),
                                         ([4096, 0, 0, 3], 1024, 2048)])
def test_fused_swiglu_matches_two_kernel_path(dev, counts, I, Kd):
    say("fused swiglu", counts, I, Kd)
    rng = np.random.default_rng(sum(counts) + I)
    E, R = len(counts), sum(counts)
    xq, xs, wq, ws = _operands(dev, rng, R, I, Kd, E)
    off = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)).to(dev)
    _check_same(dev, xq, xs, wq, ws, off)


def test_fused_swiglu_row_window(dev):
    """offsets need not start at row 0: rows outside [offsets[0], offsets[E])
    are left as they were."""
    say("fused swiglu window")
    rng = np.random.default_rng(5)
    xq, xs, wq, ws = _operands(dev, rng, 600, 256, 256, 3)
    off = torch.tensor([40, 300, 300, 555], dtype=torch.int32, device=dev)
    _check_same(dev, xq, xs, wq, ws, off)


def test_fused_swiglu_dsv3_full_shape(dev):
    """Benchmark config 4's fc1 (R=65536, 32 Zipf-loaded experts with
    zero-token ones, I=2048, K=7168) at full size: the fused epilogue's
    bytes against the two-kernel path over every row, and directly against
    the float64 oracle on 10 sampled rows of every non-empty expert (first
    and last included): c1 within the GEMM bar, hq/hs bit-exact to the
    oracle's SwiGLU requantisation of those c1 rows."""
    say("fused swiglu dsv3 full")
    c = W.CONFIGS["dsv3"]
    off = W.offsets_from_counts(W.zipf_counts()).to(dev)
    x = W.tokens(c.T, c.H, device=dev)
    xq, xs = ops.permute_quant_rows(x, torch.arange(c.T, dtype=torch.int32, device=dev), 1)
    del x
    wq, ws = ops.quantize_weight_blockwise(W.weights(c.E, 2 * c.I, c.H, device=dev, seed=3))
    _check_same(dev, xq, xs, wq, ws, off)
    hq, hs, c1 = ops.grouped_gemm_fp8_swiglu(xq, xs, wq, ws, off, save_c1=True)
    off_np = off.cpu().numpy()
    rng = np.random.default_rng(12)
    rows = []
    for e in range(c.E):
        lo, hi = int(off_np[e]), int(off_np[e + 1])
        if hi > lo:
            rows += [lo, hi - 1] + list(rng.integers(lo, hi, 8))
    rows = np.unique(np.array(rows))
    ex = np.searchsorted(off_np, rows, side="right") - 1
    soff = np.concatenate([[0], np.cumsum(np.bincount(ex, minlength=c.E))]).astype(np.int32)
    ridx = torch.from_numpy(rows).to(dev)
    ref = O.grouped_gemm_fp8(_bytes(xq[ridx]).cpu().numpy(), xs[ridx].cpu().numpy(),
                             _bytes(wq).cpu().numpy(), ws.cpu().numpy(), soff)
    c1_s = c1[ridx].view(torch.int16).cpu().numpy().view(np.uint16)
    ref = O.bf16_to_f32(O.f32_to_bf16(ref.astype(np.float32))).astype(np.float64)
    got = O.bf16_to_f32(c1_s).astype(np.float64)
    d = np.abs(got - ref)
    assert d.max() <= 1e-2 * np.abs(ref).max() and d.mean() <= 1e-3 * np.abs(ref).mean()
    oq, os_ = O.swiglu_quant(c1_s)
    assert np.array_equal(_bytes(hq[ridx]).cpu().numpy(), oq), "fused SwiGLU bytes vs oracle"
    assert np.array_equal(hs[ridx].cpu().numpy().view(np.uint32), os_.view(np.uint32))
    del wq, ws, hq, hs, c1
    torch.cuda.empty_cache()


def test_fused_swiglu_rejects_bad_shapes(dev):
    """I = 200 (not a multiple of 16) is refused; I = 192 (a multiple of 16,
    not of 128) is computed as the GEMM followed by the SwiGLU kernel, the
    bytes the fused op promises."""
    say("fused swiglu bad shapes")
    xq = torch.zeros((4, 128), dtype=torch.float8_e4m3fn, device=dev)
    xs = torch.ones((4, 1), device=dev)
    off = torch.tensor([0, 4], dtype=torch.int32, device=dev)
    wq = torch.zeros((1, 400, 128), dtype=torch.float8_e4m3fn, device=dev)  # I = 200
    ws = torch.ones((1, 4, 1), device=dev)
    with pytest.raises(ValueError):
        ops.grouped_gemm_fp8_swiglu(xq, xs, wq, ws, off)
    aq, as_ = ops.quant_rows(W.tokens(4, 128, device=dev))
    wq, ws = ops.quantize_weight_blockwise(W.weights(1, 384, 128, device=dev))  # I = 192
    hq, hs = ops.grouped_gemm_fp8_swiglu(aq, as_, wq, ws, off)
    rq, rs = ops.swiglu_quant(ops.grouped_gemm_fp8(aq, as_, wq, ws, off))
    assert hq.shape == (4, 256)
    assert torch.equal(hq.view(torch.uint8), rq.view(torch.uint8)) and torch.equal(hs, rs)


def test_simple_moe_inference_path_equals_training_path(dev):
    """SimpleMoE.forward without intermediates runs the fused fc1 epilogue;
    with intermediates it runs GEMM + SwiGLU separately.  Outputs must be
    bit-identical (config 1 shape)."""
    say("SimpleMoE fused vs unfused")
    c = W.CONFIGS["tiny"]
    m = smoe.SimpleMoE(c.H, c.I, c.E, c.K, device=dev)
    with torch.no_grad():
        m.w1.copy_(W.weights(c.E, 2 * c.I, c.H).to(dev))
        m.w2.copy_(W.weights(c.E, c.H, c.I, seed=13).to(dev))
    x, lg = W.tokens(c.T, c.H).to(dev), W.logits(c.T, c.E).to(dev)
    out_f = m(x, lg)
    out_u, _ = m(x, lg, return_intermediates=True)
    torch.cuda.synchronize()
    assert torch.equal(out_f.view(torch.int16), out_u.view(torch.int16))
