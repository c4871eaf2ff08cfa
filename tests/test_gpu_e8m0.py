"""GPU parity of the opt-in E8M0 weight-gradient recipe: power-of-two 128x1
column scales (the least power of two >= amax/448) from the four column
quantisers, and the wgrad GEMM's ``e8m0`` mode that hands those scales to
the hardware-scaled MFMA as E8M0 exponents.

Bars: quantiser bytes and scales bit-exact to the oracle (and the fused
quantisers byte-equal to the separate passes, as for the amax/448 scales);
the row (1x128) half of the fused quantisers unchanged by the column recipe;
the e8m0 wgrad within max 1e-2 / mean 1e-3 of the float64 oracle on the same
operands, its output modes bit-identical to the separate addition / rounding
of its own fp32 gradient; SimpleMoE(wgrad_recipe="e8m0") against the
oracle's backward with the same recipe: dW1 stagewise (from the oracle's
dc1) at max 1e-2 / mean 1e-3, end to end at max 4e-2 (twice the amax/448
recipe's 2e-2, since a power-of-two quantisation step is up to twice as
large), mean 1e-3."""
import sys

import numpy as np
import pytest
import torch

from oracle import smoe_oracle as O
import smoe
from smoe import _C, ops, workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def bf(u, dev):
    return torch.from_numpy(np.ascontiguousarray(u).view(np.int16)).view(torch.bfloat16).to(dev)


def close(got, ref, what, mx_tol=1e-2, mn_tol=1e-3):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    mx = d.max() / max(np.abs(ref).max(), 1e-30)
    mn = d.mean() / max(np.abs(ref).mean(), 1e-30)
    assert mx <= mx_tol and mn <= mn_tol, f"{what}: max_rel={mx:.3e} mean_rel={mn:.3e}"


def _offsets(counts):
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


def _wide_range(R, C, seed):
    """bf16 values spread over 2^-60 .. 2^40 per row, zero rows/columns and
    an all-denormal column, so scales hit the clamp and every exponent."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((R, C)) * np.exp2(rng.integers(-60, 40, (R, 1)))).astype(np.float32)
    x[:, 0] = 0.0
    x[:, 1] = rng.choice([1e-39, -3e-40, 0.0], R)
    if R > 3:
        x[3, :] = 0.0
    return O.f32_to_bf16(x)


def _check_cols(q, s, pad, x_f32, off):
    rq, rs, rpad = O.quant_cols_128x1(x_f32, off, pow2=True)
    Rp = int(rpad[-1])
    assert np.array_equal(pad.cpu().numpy(), rpad)
    assert np.array_equal(u8(q)[:, :Rp], rq), "pow2 column bytes"
    got = s.cpu().numpy()[:, :Rp // 128]
    assert np.array_equal(got.view(np.uint32), rs.view(np.uint32)), "pow2 column scales"
    assert (np.frexp(got)[0] == 0.5).all(), "scales are powers of two"


@pytest.mark.parametrize("counts,C,wide", [([130, 0, 5, 256, 1], 256, False),
                                           ([1000, 24, 0, 2000], 768, True),
                                           ([129], 2880, True)])
def test_quant_cols_pow2_bit_exact(dev, counts, C, wide):
    say("quant_cols pow2", counts, C, wide)
    off = _offsets(counts)
    R = int(off[-1])
    xb = _wide_range(R, C, R + C) if wide else u16(W.tokens(R, C, seed=R + C))
    q, s, pad, ld = ops.quant_cols(bf(xb, dev), torch.from_numpy(off).to(dev), col_scale="pow2")
    _check_cols(q, s, pad, O.bf16_to_f32(xb), off)


@pytest.mark.parametrize("counts,C", [([300, 0, 77, 512], 768), ([200, 57], 2880)])
def test_quant_rows_cols_pow2(dev, counts, C):
    """Rows keep the amax/448 scale (they feed the dgrad GEMM); columns are
    the oracle's power-of-two groups."""
    say("quant_rows_cols pow2", counts, C)
    off = _offsets(counts)
    R = int(off[-1])
    xb = _wide_range(R, C, 3 * R + C)
    q, s, qT, sT, pad, ld = ops.quant_rows_cols(bf(xb, dev), torch.from_numpy(off).to(dev),
                                                col_scale="pow2")
    rq, rs = O.quant_1x128(O.bf16_to_f32(xb))
    assert np.array_equal(u8(q), rq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    _check_cols(qT, sT, pad, O.bf16_to_f32(xb), off)


@pytest.mark.parametrize("counts,I", [([300, 0, 77, 512], 768), ([5, 129], 2880)])
def test_swiglu_bwd_quant_pow2(dev, counts, I):
    say("swiglu_bwd_quant pow2", counts, I)
    off = _offsets(counts)
    R = int(off[-1])
    rng = np.random.default_rng(R + I)
    c1 = O.f32_to_bf16((rng.standard_normal((R, 2 * I)) * 3).astype(np.float32))
    dh = O.f32_to_bf16(rng.standard_normal((R, I)).astype(np.float32))
    off_t = torch.from_numpy(off).to(dev)
    got = ops.swiglu_bwd_quant(bf(c1, dev), bf(dh, dev), off_t, col_scale="pow2")
    dc1 = O.swiglu_bwd(c1, dh)
    rq, rs = O.quant_1x128(O.bf16_to_f32(dc1))
    assert np.array_equal(u8(got[0]), rq)
    assert np.array_equal(got[1].cpu().numpy().view(np.uint32), rs.view(np.uint32))
    _check_cols(got[2], got[3], got[4], O.bf16_to_f32(dc1), off)


@pytest.mark.parametrize("T,K,H,E", [(300, 3, 768, 5), (513, 1, 2880, 4)])
def test_combine_bwd_quant_pow2(dev, T, K, H, E):
    say("combine_bwd_quant pow2", T, K, H, E)
    rng = np.random.default_rng(T * K + H)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    row_map, inv_map, _, off = O.route_sort(idx, E)
    dout, y = W.tokens(T, H, seed=21), W.tokens(T * K, H, seed=22)
    w = torch.from_numpy(rng.random((T, K)).astype(np.float32) * 2 - 0.5)
    rm, im, off_t = (torch.from_numpy(a).to(dev) for a in (row_map, inv_map, off))
    got = ops.unpermute_combine_bwd_quant(dout.to(dev), y.to(dev), im, rm, w.to(dev), off_t,
                                          col_scale="pow2")
    ody, odw = O.combine_bwd(u16(dout), u16(y), inv_map, w.numpy(), K)
    rq, rs = O.quant_1x128(O.bf16_to_f32(ody))
    assert np.array_equal(u8(got[0]), rq) and np.array_equal(got[1].cpu().numpy(), rs)
    _check_cols(got[2], got[3], got[4], O.bf16_to_f32(ody), off)
    close(got[6].cpu().numpy(), odw, "dw")


@pytest.mark.parametrize("counts,N,K", [([300, 0, 129, 1, 0, 500], 384, 640),
                                        ([4096, 0, 3, 1000], 768, 2048),
                                        ([257, 64], 2880, 2880)])
def test_wgrad_e8m0_vs_oracle(dev, counts, N, K):
    """The hardware-scaled wgrad on power-of-two operands against the float64
    oracle, against the fp32-scale kernel on the same operands (which differs
    only in where the exact power-of-two scaling is applied), and its
    accumulate / bf16 modes against separate arithmetic on its fp32 output."""
    E, R = len(counts), sum(counts)
    say("wgrad e8m0", counts, N, K)
    off = W.offsets_from_counts(torch.tensor(counts), dev)
    a, b = W.tokens(R, N, device=dev, seed=R), W.tokens(R, K, device=dev, seed=R + 1)
    aq, as_, pad, ld = ops.quant_cols(a, off, col_scale="pow2")
    bq, bs_, _, _ = ops.quant_cols(b, off, col_scale="pow2")
    got = ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld, e8m0=True)
    plain = ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld)
    ref = O.grouped_gemm_fp8_wgrad(u8(aq), as_.cpu().numpy(), u8(bq), bs_.cpu().numpy(),
                                   pad.cpu().numpy(), E)
    close(got.cpu().numpy(), ref, "dW e8m0 vs oracle")
    close(got.cpu().numpy(), plain.cpu().numpy(), "dW e8m0 vs fp32-scale kernel", 1e-4, 1e-5)
    for e, c in enumerate(counts):
        if c == 0:
            assert torch.equal(got[e], torch.zeros_like(got[e]))
    base = torch.randn((E, N, K), generator=torch.Generator(device=dev).manual_seed(7), device=dev)
    acc = base.clone()
    ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld, out=acc, accumulate=True, e8m0=True)
    assert torch.equal(acc.view(torch.int32), (base + got).view(torch.int32))
    b16 = ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld, dtype=torch.bfloat16, e8m0=True)
    assert torch.equal(b16.view(torch.int16), got.to(torch.bfloat16).view(torch.int16))
    base16 = base.to(torch.bfloat16)
    acc16 = base16.clone()
    ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld, out=acc16, accumulate=True, e8m0=True)
    assert torch.equal(acc16.view(torch.int16), (base16.float() + got).to(torch.bfloat16).view(torch.int16))


@pytest.mark.parametrize("T,H,I,E,K", [(256, 256, 256, 8, 2), (1024, 2048, 768, 128, 8),
                                       (256, 2880, 2880, 8, 4)])
def test_layer_backward_e8m0_recipe(dev, T, H, I, E, K):
    """SimpleMoE(wgrad_recipe="e8m0").backward_from against the oracle's
    backward with power-of-two wgrad operands: dx and dtopk_w do not depend on
    the recipe, so they keep the default recipe's bars; dW1/dW2 are checked
    against the oracle with C10 scales."""
    say("layer backward e8m0", T, H, I, E, K)
    m = smoe.SimpleMoE(H, I, E, K, device=dev, wgrad_recipe="e8m0")
    with torch.no_grad():
        m.w1.copy_(W.weights(E, 2 * I, H, seed=3).to(dev))
        m.w2.copy_(W.weights(E, H, I, seed=13).to(dev))
    x, lg = W.tokens(T, H, seed=0), W.logits(T, E, seed=1)
    out, st = m(x.to(dev), lg.to(dev), return_intermediates=True)
    dout = W.tokens(T, H, seed=4)
    w1q, w1s, w2q, w2s = m.fp8_weights()
    fwd = {k: (u16(v) if v.dtype == torch.bfloat16 else v.cpu().numpy())
           for k, v in st.items() if k in ("topk_w", "row_map", "inv_map", "offsets", "c1", "y")}
    r = O.moe_backward(fwd, u16(x), u8(w1q), w1s.cpu().numpy(), u8(w2q), w2s.cpu().numpy(),
                       u16(dout), K, pow2=True)
    g = m.backward_from(st, dout.to(dev))
    f = lambda a: O.bf16_to_f32(a).astype(np.float64)
    close(g["dw2"].cpu().numpy(), r["dW2"], "dW2")
    # a requantisation flip in dc1 moves one fp8 step, and a power-of-two
    # step is up to twice the amax/448 one: end to end dW1 gets twice the
    # default recipe's max bound; fed the oracle's dc1 it holds 1e-2
    close(g["dw1"].cpu().numpy(), r["dW1"], "dW1", mx_tol=4e-2)
    off = st["offsets"]
    cq, cs, pad, ld = ops.quant_cols(bf(r["dc1"], dev), off, col_scale="pow2")
    xq, xs, _, _ = ops.quant_cols(x.to(dev), off, gather=st["row_map"], gather_div=K,
                                  col_scale="pow2")
    close(ops.grouped_gemm_fp8_wgrad(cq, cs, xq, xs, pad, ld, e8m0=True).cpu().numpy(),
          r["dW1"], "dW1 stagewise")
    close(f(u16(g["dx"])), f(r["dx"]), "dx", mx_tol=2e-2)
    close(g["dtopk_w"].cpu().numpy(), r["dw"], "dtopk_w")
    # the default recipe on the same model gives the same dx bit for bit
    m.wgrad_recipe = "fp32"
    g0 = m.backward_from(st, dout.to(dev))
    assert torch.equal(g0["dx"].view(torch.int16), g["dx"].view(torch.int16))
    assert torch.equal(g0["dtopk_w"], g["dtopk_w"])


def test_wgrad_recipe_rejects_unknown(dev):
    with pytest.raises(ValueError):
        smoe.SimpleMoE(256, 256, 4, 2, device=dev, wgrad_recipe="mxfp8")
    x = torch.zeros((4, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.quant_cols(x, torch.tensor([0, 4], dtype=torch.int32, device=dev), col_scale="e8m0")


# ---------------------------------------------------------------------------
# The whole recipe with power-of-two scales: row and weight quantisers, the
# E8M0 grouped GEMM and SimpleMoE(recipe="e8m0").
# ---------------------------------------------------------------------------

def _ulps_bf16(a, b):
    """|a - b| in bf16 units in the last place, elementwise (same-sign
    values: the bit patterns as ordered integers)."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    key = lambda i: torch.where(i < 0, -32768 - i, i)
    return (key(ia) - key(ib)).abs()


@pytest.mark.parametrize("T,H,K,E", [(300, 768, 3, 5), (129, 2880, 2, 4), (64, 7168, 8, 16)])
def test_row_quantisers_pow2_bit_exact(dev, T, H, K, E):
    """permute_quant_rows, quant_rows, swiglu_quant (with h) and the weight
    quantiser with scale="pow2": bytes and scales equal the oracle's C10."""
    say("row quantisers pow2", T, H, K, E)
    rng = np.random.default_rng(T + H)
    xb = _wide_range(T, H, T * H)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    _, inv_map, _, _ = O.route_sort(idx, E)
    xq, xs = ops.permute_quant_rows(bf(xb, dev), torch.from_numpy(inv_map).to(dev), K, scale="pow2")
    rq, rs = O.permute_quant(xb, inv_map, K, pow2=True)
    assert np.array_equal(u8(xq), rq) and np.array_equal(xs.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    q, s = ops.quant_rows(bf(xb, dev), scale="pow2")
    rq, rs = O.quant_1x128(O.bf16_to_f32(xb), pow2=True)
    assert np.array_equal(u8(q), rq) and np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    c1 = O.f32_to_bf16((rng.standard_normal((T, 2 * H)) * 3).astype(np.float32))
    hq, hs, h = ops.swiglu_quant(bf(c1, dev), save_h=True, scale="pow2")
    rq, rs = O.swiglu_quant(c1, pow2=True)
    assert np.array_equal(u8(hq), rq) and np.array_equal(hs.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    h0 = ops.swiglu_quant(bf(c1, dev), save_h=True)[2]
    assert torch.equal(h.view(torch.int16), h0.view(torch.int16))  # h does not depend on the rule
    w = _wide_range(E * 2 * 144, H, E + H).reshape(E, 2 * 144, H)
    wq, ws = ops.quantize_weight_blockwise(bf(w, dev), scale="pow2")
    rwq, rws = O.quantize_weight_blockwise(w, pow2=True)
    assert np.array_equal(u8(wq), rwq) and np.array_equal(ws.cpu().numpy().view(np.uint32), rws.view(np.uint32))


@pytest.mark.parametrize("counts,C", [([300, 0, 77, 512], 768), ([200, 57], 2880)])
def test_fused_row_scales_pow2(dev, counts, C):
    """The row half of the fused quantisers with row_scale="pow2" (columns
    with either rule): rows equal the oracle's C10 1x128 groups, columns are
    unchanged by the row rule."""
    say("fused row scales pow2", counts, C)
    off = _offsets(counts)
    R = int(off[-1])
    xb = _wide_range(R, C, R + 5 * C)
    off_t = torch.from_numpy(off).to(dev)
    rq, rs = O.quant_1x128(O.bf16_to_f32(xb), pow2=True)
    for cs in ("fp32", "pow2"):
        got = ops.quant_rows_cols(bf(xb, dev), off_t, col_scale=cs, row_scale="pow2")
        ref = ops.quant_rows_cols(bf(xb, dev), off_t, col_scale=cs)
        assert np.array_equal(u8(got[0]), rq)
        assert np.array_equal(got[1].cpu().numpy().view(np.uint32), rs.view(np.uint32))
        Rp = int(ref[4][-1])
        assert torch.equal(got[2].view(torch.uint8)[:, :Rp], ref[2].view(torch.uint8)[:, :Rp])
    rng = np.random.default_rng(R)
    I = C // 2 if (C // 2) % 16 == 0 else C
    c1 = O.f32_to_bf16((rng.standard_normal((R, 2 * I)) * 3).astype(np.float32))
    dh = O.f32_to_bf16(rng.standard_normal((R, I)).astype(np.float32))
    got = ops.swiglu_bwd_quant(bf(c1, dev), bf(dh, dev), off_t, col_scale="pow2", row_scale="pow2")
    dq, ds = O.quant_1x128(O.bf16_to_f32(O.swiglu_bwd(c1, dh)), pow2=True)
    assert np.array_equal(u8(got[0]), dq) and np.array_equal(got[1].cpu().numpy().view(np.uint32), ds.view(np.uint32))


@pytest.mark.parametrize("T,K,H,E", [(300, 3, 768, 5), (513, 1, 2880, 4), (256, 8, 2048, 64)])
def test_combine_bwd_quant_row_pow2(dev, T, K, H, E):
    say("combine_bwd_quant row pow2", T, K, H, E)
    rng = np.random.default_rng(T * K + H + 1)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    row_map, inv_map, _, off = O.route_sort(idx, E)
    dout, y = W.tokens(T, H, seed=23), W.tokens(T * K, H, seed=24)
    w = torch.from_numpy(rng.random((T, K)).astype(np.float32) * 2 - 0.5)
    rm, im, off_t = (torch.from_numpy(a).to(dev) for a in (row_map, inv_map, off))
    got = ops.unpermute_combine_bwd_quant(dout.to(dev), y.to(dev), im, rm, w.to(dev), off_t,
                                          col_scale="pow2", row_scale="pow2")
    ody, _ = O.combine_bwd(u16(dout), u16(y), inv_map, w.numpy(), K)
    rq, rs = O.quant_1x128(O.bf16_to_f32(ody), pow2=True)
    assert np.array_equal(u8(got[0]), rq) and np.array_equal(got[1].cpu().numpy(), rs)
    _check_cols(got[2], got[3], got[4], O.bf16_to_f32(ody), off)


def _pow2_gemm_operands(dev, counts, N, Kd, seed):
    R = sum(counts)
    off = W.offsets_from_counts(torch.tensor(counts), dev)
    x = W.tokens(R, Kd, device=dev, seed=seed)
    if R > 2:
        x[1] = 0  # an all-zero row: scale 1
    xq, xs = ops.quant_rows(x, scale="pow2")
    wq, ws = ops.quantize_weight_blockwise(W.weights(len(counts), N, Kd, device=dev, seed=seed + 1),
                                           scale="pow2")
    return off, xq, xs, wq, ws


def _check_e8m0_gemm(dev, off, xq, xs, wq, ws, rows=None):
    """E8M0 kernel against the packed kernel on the same operands (the
    plain kernel where K is not a multiple of 512), within one bf16 ulp and
    nearly all equal, and against the float64 oracle on the given rows (all
    rows by default) at the GEMM bar."""
    wp = ops.pack_weight_fp8(wq)
    got = ops.grouped_gemm_fp8(xq, xs, wp, ws, off, e8m0=True)
    ref = ops.grouped_gemm_fp8(xq, xs, wp if ops.packed_gemm_ok(*wq.shape[1:]) else wq, ws, off)
    torch.cuda.synchronize()
    lo, hi = int(off[0]), int(off[-1])
    d = _ulps_bf16(got[lo:hi], ref[lo:hi])
    assert int(d.max()) <= 1 and float((d > 0).float().mean()) < 1e-3, \
        f"e8m0 vs packed: max {int(d.max())} ulp, {float((d > 0).float().mean()):.2e} differ"
    off_np = off.cpu().numpy()
    E = off_np.size - 1
    if rows is None:
        rows = np.arange(lo, hi)
    ex = np.searchsorted(off_np, rows, side="right") - 1
    soff = np.concatenate([[0], np.cumsum(np.bincount(ex, minlength=E))]).astype(np.int32)
    ridx = torch.from_numpy(rows).to(dev)
    r = O.grouped_gemm_fp8(u8(xq[ridx]), xs[ridx].cpu().numpy(), u8(wq), ws.cpu().numpy(), soff)
    r = O.bf16_to_f32(O.f32_to_bf16(r.astype(np.float32))).astype(np.float64)
    close(O.bf16_to_f32(u16(got[ridx])), r, "e8m0 GEMM vs oracle")
    return got


@pytest.mark.parametrize("counts,N,Kd", [([5, 0, 300, 1, 0, 129, 128, 17], 256, 512),
                                         ([0, 0, 1000], 512, 1024),
                                         ([700, 3], 784, 512),
                                         ([4096, 0, 0, 3], 2048, 2048),
                                         ([1], 16, 65536),
                                         # K blocks not a multiple of 4: the last
                                         # scale chunk's window ends at K
                                         ([300, 7], 256, 640),
                                         ([513, 0, 64], 512, 768),
                                         ([257], 256, 896),
                                         ([129, 400], 384, 1152),
                                         ([1000, 5], 512, 1280),
                                         ([600, 77], 2880, 2944)])
def test_e8m0_gemm(dev, counts, N, Kd):
    say("e8m0 gemm", counts, N, Kd)
    off, xq, xs, wq, ws = _pow2_gemm_operands(dev, counts, N, Kd, sum(counts) + N)
    _check_e8m0_gemm(dev, off, xq, xs, wq, ws)


def test_e8m0_gemm_row_window(dev):
    """offsets need not start at row 0: rows outside [offsets[0], offsets[E])
    are left as they were."""
    say("e8m0 gemm row window")
    _, xq, xs, wq, ws = _pow2_gemm_operands(dev, [600], 512, 512, 7)
    off = torch.tensor([40, 300, 300, 555], dtype=torch.int32, device=dev)
    wq, ws = wq.repeat(3, 1, 1).contiguous(), ws.repeat(3, 1, 1).contiguous()
    out = torch.full((600, 512), 3.0, dtype=torch.bfloat16, device=dev)
    ops.grouped_gemm_fp8(xq, xs, ops.pack_weight_fp8(wq), ws, off, out=out, e8m0=True)
    assert bool((out[:40] == 3.0).all()) and bool((out[555:] == 3.0).all())
    _check_e8m0_gemm(dev, off, xq, xs, wq, ws, rows=np.arange(40, 555, 7))


def test_e8m0_gemm_dsv3_full_shape(dev):
    """Benchmark config 4's fc1 and fc2 (R=65536, 32 Zipf-loaded experts with
    zero-token ones, H=7168, I=2048) at full size with power-of-two scales:
    every row against the packed kernel, 8 sampled rows of every non-empty
    expert (first and last included) against the float64 oracle; fc1's
    fused SwiGLU form against the GEMM and the SwiGLU quantiser, every row."""
    say("e8m0 gemm dsv3 full")
    c = W.CONFIGS["dsv3"]
    off = W.offsets_from_counts(W.zipf_counts()).to(dev)
    off_np = off.cpu().numpy()
    rng = np.random.default_rng(4)
    rows = []
    for e in range(c.E):
        lo, hi = int(off_np[e]), int(off_np[e + 1])
        if hi > lo:
            rows += [lo, hi - 1] + list(rng.integers(lo, hi, 6))
    rows = np.unique(np.array(rows))
    for N, Kd, seed in ((2 * c.I, c.H, 3), (c.H, c.I, 13)):
        xq, xs = ops.quant_rows(W.tokens(c.T, Kd, device=dev, seed=seed), scale="pow2")
        wq, ws = ops.quantize_weight_blockwise(W.weights(c.E, N, Kd, device=dev, seed=seed),
                                               scale="pow2")
        _check_e8m0_gemm(dev, off, xq, xs, wq, ws, rows=rows)
        if N == 2 * c.I:
            _check_e8m0_swiglu(dev, off, xq, xs, wq, ws)
        del xq, xs, wq, ws
        torch.cuda.empty_cache()


def _check_e8m0_swiglu(dev, off, xq, xs, w1q, w1s):
    """The fused entry (smoe_grouped_gemm_fp8_packed_e8m0_swiglu) against the
    E8M0 GEMM followed by the SwiGLU quantiser on the rows in
    [offsets[0], offsets[E]): hq, hs and c1 bit-exact; hs powers of two.
    Then hq, hs against the oracle's SwiGLU quantiser of the GPU's c1,
    bit-exact."""
    w1p = ops.pack_weight_fp8(w1q)
    hq, hs, c1 = ops.grouped_gemm_fp8_swiglu(xq, xs, w1p, w1s, off, save_c1=True, scale="pow2")
    qhq, qhs = ops.grouped_gemm_fp8_swiglu(xq, xs, w1p, w1s, off, scale="pow2")
    rc1 = ops.grouped_gemm_fp8(xq, xs, w1p, w1s, off, e8m0=True)
    rhq, rhs = ops.swiglu_quant(rc1, scale="pow2")
    torch.cuda.synchronize()
    lo, hi = int(off[0]), int(off[-1])
    assert torch.equal(c1[lo:hi].view(torch.int16), rc1[lo:hi].view(torch.int16))
    for q, sc in ((hq, hs), (qhq, qhs)):
        assert torch.equal(q[lo:hi].view(torch.uint8), rhq[lo:hi].view(torch.uint8))
        assert torch.equal(sc[lo:hi], rhs[lo:hi])
    assert bool((torch.frexp(hs[lo:hi])[0] == 0.5).all())
    oq, os_ = O.swiglu_quant(u16(c1[lo:hi]), pow2=True)
    assert np.array_equal(u8(hq[lo:hi]), oq) and np.array_equal(hs[lo:hi].cpu().numpy(), os_)
    return c1


@pytest.mark.parametrize("counts,I,Kd", [([200, 0, 333], 256, 1024), ([513, 64], 768, 2048),
                                         ([300, 0, 77], 128, 512), ([1000], 1408, 1024),
                                         ([257, 3], 384, 640), ([129, 0, 400], 256, 2944)])
def test_e8m0_swiglu_fused(dev, counts, I, Kd):
    say("e8m0 swiglu fused", counts, I, Kd)
    off, xq, xs, w1q, w1s = _pow2_gemm_operands(dev, counts, 2 * I, Kd, sum(counts) + I)
    _check_e8m0_swiglu(dev, off, xq, xs, w1q, w1s)


def test_e8m0_swiglu_fused_row_window(dev):
    """Rows outside [offsets[0], offsets[E]) of hq, hs and c1 are not written."""
    say("e8m0 swiglu fused row window")
    _, xq, xs, w1q, w1s = _pow2_gemm_operands(dev, [600], 512, 512, 9)
    off = torch.tensor([40, 300, 300, 555], dtype=torch.int32, device=dev)
    w1q, w1s = w1q.repeat(3, 1, 1).contiguous(), w1s.repeat(3, 1, 1).contiguous()
    hq = torch.full((600, 256), 7, dtype=torch.uint8, device=dev)
    hs = torch.full((600, 2), 3.0, dtype=torch.float32, device=dev)
    c1 = torch.full((600, 512), 3.0, dtype=torch.bfloat16, device=dev)
    w1p = ops.pack_weight_fp8(w1q)
    _C.call("smoe_grouped_gemm_fp8_packed_e8m0_swiglu", xq.data_ptr(), xs.data_ptr(),
            w1p.data.data_ptr(), w1s.data_ptr(), off.data_ptr(), 3, 600, 256, 512, hq.data_ptr(),
            hs.data_ptr(), c1.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for lo, hi in ((0, 40), (555, 600)):
        assert bool((hq[lo:hi] == 7).all()) and bool((hs[lo:hi] == 3.0).all())
        assert bool((c1[lo:hi] == 3.0).all())
    _check_e8m0_swiglu(dev, off, xq, xs, w1q, w1s)


def _close_bf16(got, ref, what, mx=1e-2, mn=1e-3):
    close(O.bf16_to_f32(u16(got)).astype(np.float64), O.bf16_to_f32(ref).astype(np.float64), what,
          mx, mn)


@pytest.mark.parametrize("T,H,I,E,K", [(256, 256, 256, 8, 2), (1024, 2048, 768, 128, 8),
                                       (256, 2880, 2880, 8, 4), (512, 1024, 512, 16, 4),
                                       (512, 640, 768, 8, 2)])
def test_layer_e8m0_recipe(dev, T, H, I, E, K):
    """SimpleMoE(recipe="e8m0") against the oracle with C10 everywhere.
    Forward stage by stage, each GPU stage fed the GPU's previous output:
    fp8 bytes and scales bit-exact, GEMM outputs within the GEMM bar, the
    combine exact.  Backward end to end against moe_backward(pow2=True,
    row_pow2=True) at the E8M0 bars of the wgrad-only recipe (dW1 max 4e-2)."""
    say("layer e8m0 recipe", T, H, I, E, K)
    m = smoe.SimpleMoE(H, I, E, K, device=dev, recipe="e8m0")
    with torch.no_grad():
        m.w1.copy_(W.weights(E, 2 * I, H, seed=3).to(dev))
        m.w2.copy_(W.weights(E, H, I, seed=13).to(dev))
    x, lg = W.tokens(T, H, seed=0), W.logits(T, E, seed=1)
    out, st = m(x.to(dev), lg.to(dev), return_intermediates=True)
    w1q, w1s, w2q, w2s = m.fp8_weights()
    for s_ in (w1s, w2s):
        assert bool((torch.frexp(s_)[0] == 0.5).all())
    rwq, rws = O.quantize_weight_blockwise(u16(m.w1.detach().to(torch.bfloat16)), pow2=True)
    assert np.array_equal(u8(w1q), rwq) and np.array_equal(w1s.cpu().numpy(), rws)
    off_np = st["offsets"].cpu().numpy()
    rq, rs = O.permute_quant(u16(x), st["inv_map"].cpu().numpy(), K, pow2=True)
    assert np.array_equal(u8(st["xq"]), rq) and np.array_equal(st["xs"].cpu().numpy(), rs)
    c1 = O.grouped_gemm_fp8(rq, rs, u8(w1q), w1s.cpu().numpy(), off_np)
    _close_bf16(st["c1"], O.f32_to_bf16(c1.astype(np.float32)), "c1")
    hq, hs = O.swiglu_quant(u16(st["c1"]), pow2=True)
    assert np.array_equal(u8(st["hq"]), hq) and np.array_equal(st["hs"].cpu().numpy(), hs)
    y = O.grouped_gemm_fp8(hq, hs, u8(w2q), w2s.cpu().numpy(), off_np)
    _close_bf16(st["y"], O.f32_to_bf16(y.astype(np.float32)), "y")
    ro = O.unpermute_combine(u16(st["y"]), st["inv_map"].cpu().numpy(), st["topk_w"].cpu().numpy(), K)
    assert np.array_equal(u16(out), ro)
    # the inference path (SwiGLU fused into the fc1 epilogue) gives the same output
    with torch.no_grad():
        out_inf = m(x.to(dev), lg.to(dev))
    assert torch.equal(out_inf.view(torch.int16), out.view(torch.int16))
    dout = W.tokens(T, H, seed=4)
    fwd = {k: (u16(v) if v.dtype == torch.bfloat16 else v.cpu().numpy())
           for k, v in st.items() if k in ("topk_w", "row_map", "inv_map", "offsets", "c1", "y")}
    r = O.moe_backward(fwd, u16(x), u8(w1q), w1s.cpu().numpy(), u8(w2q), w2s.cpu().numpy(),
                       u16(dout), K, pow2=True, row_pow2=True)
    g = m.backward_from(st, dout.to(dev))
    dyq, dys = O.quant_1x128(O.bf16_to_f32(r["dy"]), pow2=True)
    assert np.array_equal(u8(g["dyq"]), dyq) and np.array_equal(g["dys"].cpu().numpy(), dys)
    f = lambda a: O.bf16_to_f32(a).astype(np.float64)
    close(f(u16(g["dh"])), f(r["dh"]), "dh")
    close(g["dw2"].cpu().numpy(), r["dW2"], "dW2")
    close(g["dw1"].cpu().numpy(), r["dW1"], "dW1", mx_tol=4e-2)
    close(f(u16(g["dx"])), f(r["dx"]), "dx", mx_tol=2e-2)
    close(g["dtopk_w"].cpu().numpy(), r["dw"], "dtopk_w")


def test_recipe_rejects_unknown(dev):
    with pytest.raises(ValueError):
        smoe.SimpleMoE(256, 256, 4, 2, device=dev, recipe="mxfp8")
    x = torch.zeros((4, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.quant_rows(x, scale="e8m0")
