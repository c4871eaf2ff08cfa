"""Packed-weight grouped GEMM (smoe_pack_weight_fp8,
smoe_grouped_gemm_fp8_packed[_swiglu]): the packed layout byte by byte, and
the packed kernels held bit-identical to the plain ones (which the oracle
pins: tests/test_gpu_parity.py) over ragged, empty and skewed experts, tile
edges and the config-4 shape.  The operands are quantised N(0,1) activations
and N(0,0.02) weights, for which each K block's products sum without rounding
in the MFMA, so the kernels' different K orders cannot show; for operands
spanning the whole e4m3 range they can, in the last bf16 bit
(tests/test_gpu_large.py holds both kernels to the oracle there)."""
import numpy as np
import pytest
import torch

import smoe
from smoe import _C, ops
from smoe import workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[packed]", *a, flush=True)


def _operands(dev, counts, N, K, extra_rows=0, seed=0):
    off = W.offsets_from_counts(counts, dev)
    R = int(sum(counts)) + extra_rows
    xq, xs = ops.permute_quant_rows(W.tokens(R, K, device=dev, seed=30 + seed),
                                    torch.arange(R, dtype=torch.int32, device=dev), 1)
    wq, ws = ops.quantize_weight_blockwise(W.weights(len(counts), N, K, device=dev, seed=40 + seed))
    return off, xq, xs, wq, ws


def test_pack_layout(dev):
    """wp[e][nb][kb][h][l] = wq[e, 16nb + l%16, 128kb + 64h + 16(l/16) .. +16]."""
    say("layout")
    E, N, K = 2, 256, 512
    g = torch.Generator(device=dev).manual_seed(9)
    wq = torch.randint(0, 256, (E, N, K), dtype=torch.uint8, device=dev, generator=g)
    wp = ops.pack_weight_fp8(wq).data.cpu().numpy().reshape(E, N // 16, K // 128, 2, 64, 16)
    w = wq.cpu().numpy()
    nb, kb, h, ln = np.meshgrid(np.arange(N // 16), np.arange(K // 128), np.arange(2),
                                np.arange(64), indexing="ij")
    rows = nb * 16 + ln % 16
    cols = kb * 128 + h * 64 + (ln // 16) * 16
    for e in range(E):
        exp = np.stack([w[e][rows, cols + b] for b in range(16)], axis=-1)
        assert np.array_equal(wp[e], exp)


@pytest.mark.parametrize("counts,N,K,extra", [
    ([300, 0, 513, 1], 512, 512, 0),
    ([256, 256, 256], 384, 1024, 37),       # N % 256 == 128, rows past offsets[E]
    ([1000], 256, 2048, 0),
    ([0, 700, 0, 5, 1300, 0, 256, 1], 1024, 4096, 11),
    ([17, 600], 2048, 7168, 0),
    ([100, 200], 128, 512, 5),              # N = 128: one half-filled column tile
])
def test_packed_gemm_bit_identical(dev, counts, N, K, extra):
    say("gemm", counts, N, K, extra)
    off, xq, xs, wq, ws = _operands(dev, counts, N, K, extra)
    R = xq.shape[0]
    ref = torch.full((R, N), 7.0, dtype=torch.bfloat16, device=dev)   # rows past offsets[E] keep 7
    got = ref.clone()
    ops.grouped_gemm_fp8(xq, xs, wq, ws, off, out=ref)
    ops.grouped_gemm_fp8(xq, xs, ops.pack_weight_fp8(wq), ws, off, out=got)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    if extra:
        assert (got[-extra:].float() == 7.0).all()


def test_packed_gemm_many_small_and_empty_experts(dev):
    """256 experts of 0-40 rows (each such expert's one m-tile is mostly
    masked rows) plus one of 300, and a call whose experts are all empty
    (nothing is written)."""
    say("many small experts")
    rng = np.random.default_rng(5)
    counts = [int(c) for c in rng.integers(0, 41, 256)]
    counts[7] = 0
    counts[100] = 300
    off, xq, xs, wq, ws = _operands(dev, counts, 256, 512, 9, seed=6)
    R = xq.shape[0]
    ref = torch.full((R, 256), 3.0, dtype=torch.bfloat16, device=dev)
    got = ref.clone()
    ops.grouped_gemm_fp8(xq, xs, wq, ws, off, out=ref)
    ops.grouped_gemm_fp8(xq, xs, ops.pack_weight_fp8(wq), ws, off, out=got)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert (got[-9:].float() == 3.0).all()
    zero = torch.zeros_like(off)
    got.fill_(5.0)
    ops.grouped_gemm_fp8(xq, xs, ops.pack_weight_fp8(wq), ws, zero, out=got)
    torch.cuda.synchronize()
    assert (got.float() == 5.0).all()


@pytest.mark.parametrize("counts,I,K", [([200, 0, 333], 256, 1024), ([513, 64], 768, 2048),
                                        ([300, 0, 77], 128, 512), ([1000], 1408, 1024)])
def test_packed_swiglu_bit_identical(dev, counts, I, K):
    say("swiglu", counts, I, K)
    off, xq, xs, w1q, w1s = _operands(dev, counts, 2 * I, K, seed=3)
    w1p = ops.pack_weight_fp8(w1q)
    hq, hs, c1 = ops.grouped_gemm_fp8_swiglu(xq, xs, w1q, w1s, off, save_c1=True)
    phq, phs, pc1 = ops.grouped_gemm_fp8_swiglu(xq, xs, w1p, w1s, off, save_c1=True)
    assert torch.equal(phq.view(torch.uint8), hq.view(torch.uint8))
    assert torch.equal(phs, hs)
    assert torch.equal(pc1.view(torch.int16), c1.view(torch.int16))
    qhq, qhs = ops.grouped_gemm_fp8_swiglu(xq, xs, w1p, w1s, off)
    assert torch.equal(qhq.view(torch.uint8), hq.view(torch.uint8)) and torch.equal(qhs, hs)


def test_packed_config4_full(dev):
    """The config-4 GEMMs (R=65536 rows over 32 Zipf-loaded experts, fc1
    N=4096 K=7168 with and without the SwiGLU epilogue, fc2 N=7168 K=2048)."""
    say("config 4")
    c = W.CONFIGS["dsv3"]
    off = W.offsets_from_counts(W.zipf_counts(), dev)
    R = c.T
    inv = torch.arange(R, dtype=torch.int32, device=dev)
    xq, xs = ops.permute_quant_rows(W.tokens(R, c.H, device=dev), inv, 1)
    w1q, w1s = ops.quantize_weight_blockwise(W.weights(c.E, 2 * c.I, c.H, device=dev))
    w1p = ops.pack_weight_fp8(w1q)
    a = ops.grouped_gemm_fp8(xq, xs, w1q, w1s, off)
    b = ops.grouped_gemm_fp8(xq, xs, w1p, w1s, off)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    hq, hs = ops.grouped_gemm_fp8_swiglu(xq, xs, w1q, w1s, off)
    phq, phs = ops.grouped_gemm_fp8_swiglu(xq, xs, w1p, w1s, off)
    assert torch.equal(phq.view(torch.uint8), hq.view(torch.uint8)) and torch.equal(phs, hs)
    del a, b, xq, xs, w1q, w1p
    w2q, w2s = ops.quantize_weight_blockwise(W.weights(c.E, c.H, c.I, device=dev, seed=13))
    a = ops.grouped_gemm_fp8(hq, hs, w2q, w2s, off)
    b = ops.grouped_gemm_fp8(hq, hs, ops.pack_weight_fp8(w2q), w2s, off)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def _np_u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _np_u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def _oracle_rows(O, aq, as_, wq, ws, rows, offs):
    """float64 oracle GEMM restricted to the given sorted rows."""
    aq_np, as_np = _np_u8(aq[rows]), as_[rows].cpu().numpy()
    wq_np, ws_np = _np_u8(wq), ws.cpu().numpy()
    rows_np = rows.cpu().numpy()
    owner = np.searchsorted(offs, rows_np, side="right") - 1
    ref = np.zeros((len(rows_np), wq.shape[1]), np.float64)
    for e in np.unique(owner):
        sel = owner == e
        ref[sel] = O.dequant_rows(aq_np[sel], as_np[sel]) @ O.dequant_weight(wq_np[e], ws_np[e]).T
    return ref


def test_packed_config4_oracle_samples(dev):
    """The packed kernel SimpleMoE runs at config 4, held to the float64 oracle
    directly (not only through the plain kernel): rows of every non-empty
    expert of fc1 (N=4096, K=7168) and fc2 (N=7168, K=2048), within the GEMM
    tolerance (max 1e-2, mean 1e-3 of the bf16-rounded oracle); and the fused
    SwiGLU epilogue's hq / hs on those rows byte-identical to the oracle's
    swiglu_quant of the kernel's own c1 (the same input), with c1 within the
    GEMM tolerance."""
    from oracle import smoe_oracle as O

    def gemm_close(got, ref, what):
        ref = O.bf16_to_f32(O.f32_to_bf16(np.asarray(ref, np.float32))).astype(np.float64)
        d = np.abs(got - ref)
        mx, mn = d.max() / np.abs(ref).max(), d.mean() / np.abs(ref).mean()
        assert mx <= 1e-2 and mn <= 1e-3, f"{what}: max_rel={mx:.3e} mean_rel={mn:.3e}"

    say("config 4 vs oracle")
    c = W.CONFIGS["dsv3"]
    counts = W.zipf_counts()
    off = W.offsets_from_counts(counts, dev)
    offs = off.cpu().numpy()
    R = c.T
    inv = torch.arange(R, dtype=torch.int32, device=dev)
    rows = torch.from_numpy(np.concatenate(
        [np.unique(np.linspace(offs[e], offs[e + 1] - 1, 5).astype(np.int64))
         for e in range(c.E) if counts[e] > 0])).to(dev)
    xq, xs = ops.permute_quant_rows(W.tokens(R, c.H, device=dev), inv, 1)
    w1q, w1s = ops.quantize_weight_blockwise(W.weights(c.E, 2 * c.I, c.H, device=dev))
    w1p = ops.pack_weight_fp8(w1q)
    c1 = ops.grouped_gemm_fp8(xq, xs, w1p, w1s, off)
    ref1 = _oracle_rows(O, xq, xs, w1q, w1s, rows, offs)
    gemm_close(O.bf16_to_f32(_np_u16(c1[rows])).astype(np.float64), ref1, "packed fc1")
    hq, hs, c1f = ops.grouped_gemm_fp8_swiglu(xq, xs, w1p, w1s, off, save_c1=True)
    assert torch.equal(c1f[rows].view(torch.int16), c1[rows].view(torch.int16))
    rq, rs = O.swiglu_quant(_np_u16(c1f[rows]))
    assert np.array_equal(_np_u8(hq[rows]), rq) and np.array_equal(hs[rows].cpu().numpy(), rs)
    del xq, xs, w1q, w1p, c1, c1f
    torch.cuda.empty_cache()
    w2q, w2s = ops.quantize_weight_blockwise(W.weights(c.E, c.H, c.I, device=dev, seed=13))
    y = ops.grouped_gemm_fp8(hq, hs, ops.pack_weight_fp8(w2q), w2s, off)
    ref2 = _oracle_rows(O, hq, hs, w2q, w2s, rows, offs)
    gemm_close(O.bf16_to_f32(_np_u16(y[rows])).astype(np.float64), ref2, "packed fc2")


def test_packed_validation(dev):
    say("validation")
    off, xq, xs, wq, ws = _operands(dev, [100, 50], 256, 384)
    with pytest.raises(ValueError):
        ops.pack_weight_fp8(wq)                       # K = 384: below 512, no packed kernel
    off, xq, xs, wq, ws = _operands(dev, [100, 50], 256, 640)
    # K = 640 packs for the E8M0 kernel only; the packed kernel refuses it
    assert not ops.packed_gemm_ok(256, 640) and ops.packed_gemm_ok(256, 512)
    assert ops.packed_e8m0_ok(256, 640)
    with pytest.raises(ValueError):
        ops.grouped_gemm_fp8(xq, xs, ops.pack_weight_fp8(wq), ws, off)
    st = torch.cuda.current_stream().cuda_stream
    c = torch.empty((150, 256), dtype=torch.bfloat16, device=dev)
    rc = _C.lib().smoe_grouped_gemm_fp8_packed(xq.data_ptr(), xs.data_ptr(), wq.data_ptr(),
                                               ws.data_ptr(), off.data_ptr(), 2, 150, 256, 640,
                                               c.data_ptr(), st)
    assert rc == -3                                   # SMOE_EINVAL_ALIGN128
    off, xq, xs, wq, ws = _operands(dev, [100, 50], 256, 512)
    wp = ops.pack_weight_fp8(wq)
    xq2, xs2 = ops.permute_quant_rows(W.tokens(150, 1024, device=dev),
                                      torch.arange(150, dtype=torch.int32, device=dev), 1)
    with pytest.raises(ValueError):
        ops.grouped_gemm_fp8(xq2, xs2, wp, ws, off)   # K mismatch


def test_simple_moe_uses_packed_weights(dev):
    """SimpleMoE packs a GEMM's weights exactly when the packed kernel covers
    them, and its forward matches the plain kernels' composition."""
    say("SimpleMoE packed")
    H, I, E, K, T = 512, 256, 4, 2, 300
    m = smoe.SimpleMoE(H, I, E, K, device=dev)
    m.reset_parameters(torch.Generator(device=dev).manual_seed(2))
    w1g, _, w2g, _ = m.gemm_weights()
    assert isinstance(w1g, ops.PackedWeight)          # K = H = 512
    assert not isinstance(w2g, ops.PackedWeight)      # K = I = 256
    w1t, _, w2t, _ = m.gemm_weights_t()
    assert isinstance(w1t, ops.PackedWeight)          # dgrad fc1: K = 2I = 512
    assert isinstance(w2t, ops.PackedWeight)          # dgrad fc2: K = H = 512
    x = W.tokens(T, H).to(dev)
    lg = W.logits(T, E).to(dev)
    with torch.no_grad():
        out = m(x, lg)
    w1q, w1s, w2q, w2s = m.fp8_weights()
    idx, w, rm, im, cnt, off = ops.route_topk_sort(lg, K)
    xq, xs = ops.permute_quant_rows(x, im, K)
    hq, hs = ops.grouped_gemm_fp8_swiglu(xq, xs, w1q, w1s, off)
    ref = ops.unpermute_combine(ops.grouped_gemm_fp8(hq, hs, w2q, w2s, off), im, w)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
