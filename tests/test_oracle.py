"""Pins for the CPU oracle (no GPU).  Each check is independent of the
oracle's own formula: a library routine, a closed form, brute force, or the
reference's worked example."""
import os

import numpy as np
import pytest
import torch

from oracle import smoe_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ------------------------------------------------------------------ e4m3
def _torch_e4m3(v):
    return torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encode_all_bf16_patterns_match_torch():
    # every finite bf16 value with |v| <= 448 (torch's cast is RNE; it does
    # not saturate, so only in-range values are compared)
    u = np.arange(1 << 16, dtype=np.uint32)
    v = (u << 16).view(np.float32)
    v = v[np.isfinite(v) & (np.abs(v) <= 448)]
    assert np.array_equal(O.e4m3_encode(v), _torch_e4m3(v))


def test_e4m3_encode_rounding_midpoints_match_torch():
    # midpoints between consecutive e4m3 magnitudes, and one fp32 ulp either side
    mags = np.sort(np.unique(np.abs(O.e4m3_decode(np.arange(0x7F, dtype=np.uint8)))))
    mid = ((mags[:-1].astype(np.float64) + mags[1:]) / 2).astype(np.float32)
    probe = np.concatenate([mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9)), mags])
    probe = np.concatenate([probe, -probe])
    assert np.array_equal(O.e4m3_encode(probe), _torch_e4m3(probe))


def test_e4m3_encode_dense_fp32_sweep_matches_torch():
    # every 61st fp32 pattern in [0, 448] (an exhaustive sweep of all 1.1e9
    # patterns also matches; it takes about a minute so the suite samples)
    hi = int(np.float32(448).view(np.uint32))
    u = np.arange(0, hi + 1, 61, dtype=np.uint32)
    v = u.view(np.float32)
    assert np.array_equal(O.e4m3_encode(v), _torch_e4m3(v))
    assert np.array_equal(O.e4m3_encode(-v), _torch_e4m3(-v))


def test_e4m3_decode_matches_torch():
    q = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(q).view(torch.float8_e4m3fn).float().numpy()
    got = O.e4m3_decode(q)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok], ref[ok])
    assert O.e4m3_decode(np.array([0x7E], np.uint8))[0] == 448.0


def test_quant_rule_saturates():
    s = np.float32(1.0)
    assert O.quant_rule(np.float32(1000.0), s) == 0x7E
    assert O.quant_rule(np.float32(-1000.0), s) == 0xFE
    assert O.quant_rule(np.float32(449.0), s) == 0x7E


# ---------------------------------------------------------------- bf16
def test_bf16_roundtrip_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(100000) * 10).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), ref)
    assert np.array_equal(O.bf16_to_f32(ref), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ------------------------------------------------------------------ exp
def test_expf32_within_2ulp_of_float64():
    x = np.linspace(-87, 88, 400001).astype(np.float32)
    got = O.expf32(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) / ulp).max() <= 2.0


def test_expf32_special_values():
    v = O.expf32(np.array([0.0, -0.0, 100.0, -100.0, 1.0], np.float32))
    assert v[0] == 1.0 and v[1] == 1.0
    assert np.isinf(v[2]) and v[3] == 0.0
    assert abs(v[4] - np.e) < 1e-6


# --------------------------------------------------------------- router
def test_softmax_close_to_float64_and_tree_order():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal((50, 256)).astype(np.float32)
    p = O.softmax_f32(lg)
    l64 = lg.astype(np.float64)
    ref = np.exp(l64 - l64.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    assert np.abs(p - ref).max() < 1e-6
    # the reduction tree for E <= 64 with one element per lane: brute force
    vals = rng.random((3, 64)).astype(np.float32)
    lanes = [list(r) for r in vals]
    for off in (32, 16, 8, 4, 2, 1):
        lanes = [[np.float32(r[i] + r[i ^ off]) for i in range(64)] for r in lanes]
    assert np.array_equal(O._wave_tree_sum(vals), np.array([r[0] for r in lanes], np.float32))


def test_router_topk_brute_force_with_ties():
    rng = np.random.default_rng(2)
    T, E, K = 40, 16, 4
    lg = rng.integers(-2, 3, (T, E)).astype(np.float32)  # many exact ties
    bias = rng.integers(-1, 2, E).astype(np.float32) * 0.0625
    idx, w = O.router_topk(lg, K, bias)
    p = O.softmax_f32(lg)
    for t in range(T):
        sc = [(float(np.float32(p[t, e] + bias[e])), e) for e in range(E)]
        want = [e for _, e in sorted(sc, key=lambda z: (-z[0], z[1]))[:K]]
        assert list(idx[t]) == want
        picked = p[t, want].astype(np.float64)
        assert np.allclose(w[t], picked / picked.sum(), rtol=1e-6)
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)


# ----------------------------------------------------------------- sort
def test_router_topk_bwd_matches_float64_autograd():
    """The router backward formula against torch float64 autograd through
    softmax -> gather of the picks -> renormalisation, with a selection bias
    (which only changes the picks) and K up to E."""
    rng = np.random.default_rng(5)
    for T, E, K, use_bias in ((64, 8, 2, False), (32, 64, 6, True), (16, 256, 8, True), (8, 5, 5, False)):
        lg = rng.standard_normal((T, E)).astype(np.float32)
        b = rng.standard_normal(E).astype(np.float32) * 0.5 if use_bias else None
        idx, _ = O.router_topk(lg, K, b)
        g = rng.standard_normal((T, K))
        l64 = torch.tensor(lg, dtype=torch.float64, requires_grad=True)
        p = torch.softmax(l64, dim=1)
        pk = torch.gather(p, 1, torch.from_numpy(idx.astype(np.int64)))
        w = pk / pk.sum(dim=1, keepdim=True)
        (w * torch.from_numpy(g)).sum().backward()
        got = O.router_topk_bwd(lg, idx, g)
        ref = l64.grad.numpy()
        assert np.abs(got - ref).max() <= 1e-12 * max(1.0, np.abs(ref).max())
        # each row's logit gradient sums to zero (softmax shift invariance)
        assert np.abs(got.sum(axis=1)).max() < 1e-12


def test_route_sort_reference_worked_example():
    g = np.load(os.path.join(GOLDEN, "worked_example.npz"))
    row_map, inv_map, counts, offsets = O.route_sort(g["topk_idx"], 8)
    assert counts.tolist() == g["counts"].tolist() == [5, 4, 5, 4, 3, 4, 4, 3]
    assert offsets.tolist() == [0, 5, 9, 14, 18, 21, 25, 29, 32]
    # E0 holds t0 t2 t4 t9 t14 in token order (dataflow.md:103)
    assert (row_map[:5] // 2).tolist() == [0, 2, 4, 9, 14]
    # E2: t3 t4 t8 t13 t15
    assert (row_map[9:14] // 2).tolist() == [3, 4, 8, 13, 15]


def test_route_sort_brute_force_and_invariants():
    rng = np.random.default_rng(3)
    T, K, E = 300, 4, 37
    idx = rng.integers(0, E, (T, K)).astype(np.int32)
    idx[:, 1] = 5  # a hot expert
    row_map, inv_map, counts, offsets = O.route_sort(idx, E)
    brute = [p for e in range(E) for p in range(T * K) if idx.reshape(-1)[p] == e]
    assert row_map.tolist() == brute
    assert np.array_equal(inv_map[row_map], np.arange(T * K))
    assert offsets[-1] == T * K and np.array_equal(np.diff(offsets), counts)


# ---------------------------------------------------------------- quant
def test_quant_1x128_closed_forms():
    x = np.zeros((4, 256), np.float32)
    x[0, 3] = -7.5                       # one-hot: -> -448, others 0
    x[1, :128] = 0.25                    # constant group -> all 448
    x[2, 128:] = np.linspace(-1, 1, 128)  # amax 1 -> s = 1/448
    q, s = O.quant_1x128(x)
    assert s[0, 0] == np.float32(7.5) / np.float32(448) and q[0, 3] == 0xFE
    assert (q[0, np.arange(256) != 3] == 0).all() and s[0, 1] == 1.0
    assert (q[1, :128] == 0x7E).all() and s[1, 0] == np.float32(0.25 / 448)
    assert (q[3] == 0).all() and (s[3] == 1.0).all()  # amax == 0 -> s = 1, q = 0
    assert q[2, 255] == 0x7E and q[2, 128] == 0xFE
    # dequantised error within half an e4m3 ulp of the scaled value
    rng = np.random.default_rng(4)
    y = rng.standard_normal((64, 512)).astype(np.float32)
    q, s = O.quant_1x128(y)
    deq = O.dequant_rows(q, s)
    rel = np.abs(deq - y) / np.repeat(s, 128, axis=1)
    scaled = np.abs(y) / np.repeat(s, 128, axis=1)
    half_ulp = np.where(scaled < 2 ** -6, 2.0 ** -10, 2.0 ** (np.floor(np.log2(np.maximum(scaled, 1e-30))) - 4))
    assert (rel <= half_ulp * (1 + 1e-5)).all()


def test_weight_quant_blocks_equal_flattened_groups():
    g = np.load(os.path.join(GOLDEN, "weight_quant.npz"))
    wq, ws = O.quantize_weight_blockwise(g["w"])
    assert np.array_equal(wq, g["wq"]) and np.array_equal(ws, g["ws"])
    # a 128x128 block is one group: its amax sets one scale for all 16384 values
    w = O.bf16_to_f32(g["w"])
    blk = w[1, 0:128, 128:256].reshape(1, -1)
    amax = np.abs(blk).max()
    s = np.float32(amax) / np.float32(448)
    assert ws[1, 0, 1] == s
    assert np.array_equal(wq[1, 0:128, 128:256].reshape(-1), O.quant_rule(blk.reshape(-1), s))


# ----------------------------------------------------------------- GEMM
def _rand_fp8(rng, shape):
    q = rng.integers(0, 256, shape).astype(np.uint8)
    q[(q & 0x7F) == 0x7F] = 0x3C  # no NaN codes
    return q


def test_quant_1x128_short_last_group():
    """C9 at GPT-OSS's H = 2880 (22.5 groups): the 22 full groups equal the
    aligned prefix quantised alone; the short group's scale is the amax of
    its 64 valid values / 448 (float32 division) and its bytes are torch's
    e4m3 cast of clamp(x / s); the 64 padding bytes are 0."""
    rng = np.random.default_rng(2880)
    M, H = 9, 2880
    x = (rng.standard_normal((M, H)) * np.exp(rng.standard_normal((M, 1)))).astype(np.float32)
    x[3, 2816:] = 0.0            # an all-zero short group: s = 1
    x[4, 2870] = 1000.0          # an outlier in the short group
    q, s = O.quant_1x128(x)
    assert q.shape == (M, 2944) and s.shape == (M, 23)
    q0, s0 = O.quant_1x128(x[:, :2816])
    assert np.array_equal(q[:, :2816], q0) and np.array_equal(s[:, :22], s0)
    amax = np.abs(x[:, 2816:]).max(axis=1)
    want_s = np.where(amax == 0, np.float32(1), (amax / np.float32(448)).astype(np.float32))
    assert np.array_equal(s[:, 22], want_s.astype(np.float32))
    assert s[3, 22] == 1.0
    v = np.clip(x[:, 2816:] / s[:, 22:23], -448, 448).astype(np.float32)
    assert np.array_equal(q[:, 2816:2880], _torch_e4m3(v))
    assert not q[:, 2880:].any()


def test_weight_quant_short_blocks_and_transpose():
    """C9 for 128x128 weight blocks at N = K = 2880: blocks inside the
    aligned part equal the aligned restatement, a short block's scale is the
    amax of its valid elements / 448, padding columns are 0; the transposed
    weights dequantise to the transpose of the dequantised weights."""
    rng = np.random.default_rng(2881)
    E, N, K = 2, 2880, 2880
    w = O.f32_to_bf16((rng.standard_normal((E, N, K)) * 0.02).astype(np.float32))
    q, s = O.quantize_weight_blockwise(w)
    assert q.shape == (E, N, 2944) and s.shape == (E, 23, 23)
    qa, sa = O.quantize_weight_blockwise(np.ascontiguousarray(w[:, :2816, :2816]))
    assert np.array_equal(q[:, :2816, :2816], qa) and np.array_equal(s[:, :22, :22], sa)
    wf = O.bf16_to_f32(w)
    for (r0, r1, c0, c1) in ((2816, 2880, 0, 128), (0, 128, 2816, 2880), (2816, 2880, 2816, 2880)):
        amax = np.abs(wf[0, r0:r1, c0:c1]).max()
        assert s[0, r0 // 128, c0 // 128] == np.float32(amax) / np.float32(448)
    assert not q[:, :, 2880:].any()
    qt, st = O.transpose_blockwise(q, s, k=K)
    assert qt.shape == (E, K, 2944) and st.shape == (E, 23, 23)
    for e in range(E):
        assert np.array_equal(O.dequant_weight(qt[e], st[e])[:, :N], O.dequant_weight(q[e], s[e])[:, :K].T)
    assert not qt[:, :, 2880:].any()


def test_group_scale_pow2_closed_forms():
    """C10: powers of two stay, anything above one moves up to the next
    power of two, zero gives 1, tiny amax clamps to 2^-127; dividing by the
    scale is exact, so the bytes are torch's e4m3 cast of x * 2^-e with no
    clamp needed (|x / s| <= 448)."""
    amax = np.array([0.0, 448.0, 448.0 * 2 ** -20, np.nextafter(np.float32(448), np.float32(1e9)),
                     3.0, 1e-40, 2.0 ** -130 * 448], np.float32)
    s = O.group_scale_pow2(amax)
    assert list(s[:3]) == [1.0, 1.0, 2.0 ** -20]
    assert s[3] == 2.0 and s[4] == 2.0 ** -7 and s[5] == 2.0 ** -127 and s[6] == 2.0 ** -127
    assert all(np.frexp(v)[0] == 0.5 for v in s)
    rng = np.random.default_rng(10)
    x = (rng.standard_normal((64, 384)) * np.exp2(rng.integers(-20, 20, (64, 1)))).astype(np.float32)
    q, sc = O.quant_1x128(x, pow2=True)
    y = x.reshape(64, 3, 128) / sc[:, :, None]
    assert np.abs(y).max() <= 448
    assert np.array_equal(q, _torch_e4m3(y.reshape(64, 384)))
    # against the C3 scale: never below it, less than twice it
    _, s3 = O.quant_1x128(x)
    assert (sc >= s3).all() and (sc < 2 * s3).all()


def test_pow2_weight_and_swiglu_quantisers():
    """C10 on weight blocks and on SwiGLU's h: every scale a power of two in
    [s_C3, 2 s_C3), the bytes torch's e4m3 cast of x * 2^-e (exact, no clamp
    needed), and a short last block (C9) still the zero-padded block."""
    rng = np.random.default_rng(12)
    w = O.f32_to_bf16((rng.standard_normal((2, 200, 272)) * np.exp2(rng.integers(-9, 9, (2, 1, 1))))
                      .astype(np.float32))
    q, s = O.quantize_weight_blockwise(w, pow2=True)
    _, s3 = O.quantize_weight_blockwise(w)
    assert (np.frexp(s)[0] == 0.5).all() and (s >= s3).all() and (s < 2 * s3).all()
    wf = np.pad(O.bf16_to_f32(w), ((0, 0), (0, 56), (0, 112)))
    y = wf.reshape(2, 2, 128, 3, 128) / s[:, :, None, :, None]
    assert np.abs(y).max() <= 448
    assert np.array_equal(q, _torch_e4m3(y.reshape(2, 256, 384))[:, :200])
    c1 = O.f32_to_bf16((rng.standard_normal((33, 2 * 144)) * 4).astype(np.float32))
    hq, hs = O.swiglu_quant(c1, pow2=True)
    cf = O.bf16_to_f32(c1)
    h = (O.silu_f32(cf[:, :144]) * cf[:, 144:]).astype(np.float32)
    rq, rs = O.quant_1x128(h, pow2=True)
    assert np.array_equal(hq, rq) and np.array_equal(hs, rs)
    assert (np.frexp(hs)[0] == 0.5).all()


def test_pow2_wgrad_operands_as_accurate_as_c3():
    """The opt-in E8M0 recipe loses no accuracy: a weight gradient from
    power-of-two 128x1 operands is as close to the exact product of the bf16
    inputs as one from amax/448 operands (mean relative error within 10% of
    each other)."""
    rng = np.random.default_rng(11)
    R, N, K = 1024, 256, 384
    a = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((R, N)).astype(np.float32)))
    b = O.bf16_to_f32(O.f32_to_bf16((rng.standard_normal((R, K)) * 1e-3).astype(np.float32)))
    off = np.array([0, 300, 1024], np.int32)
    exact = np.stack([a[0:300].astype(np.float64).T @ b[0:300], a[300:].astype(np.float64).T @ b[300:]])
    err = {}
    for p2 in (False, True):
        aq, as_, pad = O.quant_cols_128x1(a, off, pow2=p2)
        bq, bs_, _ = O.quant_cols_128x1(b, off, pow2=p2)
        got = O.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, 2)
        err[p2] = np.abs(got - exact).mean() / np.abs(exact).mean()
    assert err[True] < 0.05 and abs(err[True] - err[False]) <= 0.1 * err[False], err


def test_grouped_gemm_brute_force_blocks():
    rng = np.random.default_rng(5)
    E, N, Kd = 3, 256, 384
    counts = [5, 0, 9]
    off = np.array([0, 5, 5, 14], np.int32)
    R = 14
    a, b = _rand_fp8(rng, (R, Kd)), _rand_fp8(rng, (E, N, Kd))
    a_s = rng.random((R, Kd // 128)).astype(np.float32)
    b_s = rng.random((E, N // 128, Kd // 128)).astype(np.float32)
    got = O.grouped_gemm_fp8(a, a_s, b, b_s, off)
    av, bv = O.e4m3_decode(a).astype(np.float64), O.e4m3_decode(b).astype(np.float64)
    for r in range(R):
        e = int(np.searchsorted(off, r, side="right") - 1)
        for n in (0, 17, 128, 255):
            ref = 0.0
            for kb in range(Kd // 128):
                part = float(np.dot(av[r, kb * 128:(kb + 1) * 128], bv[e, n, kb * 128:(kb + 1) * 128]))
                ref += float(a_s[r, kb]) * float(b_s[e, n // 128, kb]) * part
            assert abs(got[r, n] - ref) <= 1e-9 * max(1.0, abs(ref))
    assert counts[1] == 0  # expert 1 owns no rows and nothing breaks


def test_grouped_gemm_one_hot_and_single_block():
    E, N, Kd = 2, 128, 256
    a = np.zeros((4, Kd), np.uint8)
    a[0, 5] = 0x38      # 1.0 at k=5 (block 0)
    a[1, 200] = 0x40    # 2.0 at k=200 (block 1)
    a_s = np.array([[1, 1], [1, 3], [2, 2], [1, 1]], np.float32)
    b = np.zeros((E, N, Kd), np.uint8)
    b[0, :, 5] = 0x38
    b[1, 7, 200] = 0x48  # 4.0
    b_s = np.ones((E, 1, 2), np.float32)
    b_s[1, 0, 1] = 0.5
    off = np.array([0, 1, 4], np.int32)
    out = O.grouped_gemm_fp8(a, a_s, b, b_s, off)
    assert (out[0] == 1.0).all()                    # row 0 -> expert 0, one-hot
    assert out[1, 7] == 2.0 * 4.0 * 3.0 * 0.5       # scales of block 1 only
    assert np.count_nonzero(out[1]) == 1 and not out[2:].any()


# --------------------------------------------------------------- SwiGLU
def test_silu_and_swiglu():
    g = np.array([0.0, 30.0, -30.0, 1.0, -1.0], np.float32)
    s = O.silu_f32(g)
    assert s[0] == 0 and s[1] == 30.0 and abs(s[2]) < 1e-11
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    assert np.allclose(s, ref, rtol=1e-6)
    rng = np.random.default_rng(6)
    c1 = O.f32_to_bf16(rng.standard_normal((8, 512)).astype(np.float32) * 3)
    hq, hs = O.swiglu_quant(c1)
    c = O.bf16_to_f32(c1).astype(np.float64)
    h = c[:, :256] / (1 + np.exp(-c[:, :256])) * c[:, 256:]
    deq = O.dequant_rows(hq, hs)
    assert np.abs(deq - h).max() <= np.abs(h).max() * 2 ** -4


# -------------------------------------------------------------- combine
def test_combine_identity_and_scalar_loop():
    rng = np.random.default_rng(7)
    T, K, H = 6, 3, 128
    y = O.f32_to_bf16(rng.standard_normal((T * K, H)).astype(np.float32))
    inv = rng.permutation(T * K).astype(np.int32)
    w = rng.random((T, K)).astype(np.float32)
    out = O.unpermute_combine(y, inv, w, K)
    yf = O.bf16_to_f32(y)
    for t in range(T):
        for h in (0, 64, 127):
            acc = np.float32(0)
            for k in range(K):
                acc = np.float32(acc + np.float32(w[t, k] * yf[inv[t * K + k], h]))
            assert out[t, h] == O.f32_to_bf16(np.array([acc], np.float32))[0]
    # K=1, w=1: exact inverse permutation
    one = O.unpermute_combine(y, inv, np.ones((T * K, 1), np.float32), 1)
    assert np.array_equal(one, y[inv])


# ----------------------------------------------------------- whole layer
def test_oracle_tiny_fixture_regression():
    g = np.load(os.path.join(GOLDEN, "oracle_tiny.npz"))
    res = O.moe_forward(g["x"], g["logits"], g["w1q"], g["w1s"], g["w2q"], g["w2s"], int(g["K"]))
    for k, v in res.items():
        assert np.array_equal(v, g[k]), k
    # end-to-end against a float64 dense MoE on the dequantised weights
    E = g["w1q"].shape[0]
    x = O.bf16_to_f32(g["x"]).astype(np.float64)
    ref = np.zeros_like(x)
    for t in range(x.shape[0]):
        for k in range(int(g["K"])):
            e = g["topk_idx"][t, k]
            w1 = O.dequant_weight(g["w1q"][e], g["w1s"][e])
            w2 = O.dequant_weight(g["w2q"][e], g["w2s"][e])
            c = w1 @ x[t]
            I = c.size // 2
            h = c[:I] / (1 + np.exp(-c[:I])) * c[I:]
            ref[t] += g["topk_w"][t, k] * (w2 @ h)
    out = O.bf16_to_f32(g["out"]).astype(np.float64)
    # fp8 activations on both GEMM inputs: a few percent of the output scale
    assert np.abs(out - ref).max() <= 0.1 * np.abs(ref).max()
    assert np.abs(out - ref).mean() <= 0.05 * np.abs(ref).mean()
    assert E == 4


# ------------------------------------------------------------- backward
def test_transpose_blockwise_commutes_with_dequant():
    rng = np.random.default_rng(8)
    w = O.f32_to_bf16((rng.standard_normal((2, 256, 384)) * 0.02).astype(np.float32))
    wq, ws = O.quantize_weight_blockwise(w)
    tq, ts = O.transpose_blockwise(wq, ws)
    for e in range(2):
        assert np.array_equal(O.dequant_weight(tq[e], ts[e]), O.dequant_weight(wq[e], ws[e]).T)
    # requantising the transposed dequantised block gives the same bytes
    rq, rs = O.quantize_weight_blockwise(O.f32_to_bf16(O.bf16_to_f32(w).transpose(0, 2, 1).copy()))
    assert np.array_equal(rq, tq) and np.array_equal(rs, ts)


def test_quant_cols_matches_padded_transpose_and_closed_form():
    rng = np.random.default_rng(9)
    counts = [130, 0, 5, 256, 1]
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    R, C = off[-1], 256
    x = rng.standard_normal((R, C)).astype(np.float32)
    q, s, pad = O.quant_cols_128x1(x, off)
    assert pad.tolist() == [0, 256, 256, 384, 640, 768]
    # independent construction: per expert, per column, python slicing
    for e, cnt in enumerate(counts):
        for g0 in range(0, cnt, 128):
            rows = x[off[e] + g0: off[e] + min(cnt, g0 + 128)]
            for col in (0, 77, 255):
                seg = rows[:, col]
                amax = np.float32(np.abs(seg).max())
                sc = np.float32(1.0) if amax == 0 else amax / np.float32(448)
                pos = pad[e] + g0
                assert s[col, pos // 128] == sc
                assert np.array_equal(q[col, pos:pos + seg.size], O.quant_rule(seg, sc))
                assert not q[col, pos + seg.size:pos + 128].any()  # zero padding


def test_wgrad_brute_force():
    rng = np.random.default_rng(10)
    counts = [3, 0, 200]
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    R = off[-1]
    dy = rng.standard_normal((R, 128)).astype(np.float32)
    h = rng.standard_normal((R, 256)).astype(np.float32)
    aq, as_, pad = O.quant_cols_128x1(dy, off)
    bq, bs_, _ = O.quant_cols_128x1(h, off)
    dW = O.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, 3)
    assert not dW[1].any()
    A = O.e4m3_decode(aq).astype(np.float64)
    B = O.e4m3_decode(bq).astype(np.float64)
    for e in (0, 2):
        for n, k in ((0, 0), (5, 200), (127, 31)):
            ref = 0.0
            for r in range(pad[e], pad[e + 1]):
                ref += A[n, r] * float(as_[n, r // 128]) * B[k, r] * float(bs_[k, r // 128])
            assert abs(dW[e, n, k] - ref) <= 1e-9 * max(1, abs(ref))
    # and it approximates the unquantised product
    ref = dy[off[2]:].astype(np.float64).T @ h[off[2]:].astype(np.float64)
    assert np.abs(dW[2] - ref).max() <= 0.1 * np.abs(ref).max()


def test_swiglu_bwd_matches_float64_derivative():
    rng = np.random.default_rng(11)
    c1 = O.f32_to_bf16((rng.standard_normal((16, 512)) * 3).astype(np.float32))
    dh = O.f32_to_bf16(rng.standard_normal((16, 256)).astype(np.float32))
    dc = O.bf16_to_f32(O.swiglu_bwd(c1, dh)).astype(np.float64)
    c = O.bf16_to_f32(c1).astype(np.float64)
    d = O.bf16_to_f32(dh).astype(np.float64)
    g, u = c[:, :256], c[:, 256:]
    s = 1 / (1 + np.exp(-g))
    ref = np.concatenate([d * u * s * (1 + g * (1 - s)), d * g * s], axis=1)
    assert np.abs(dc - ref).max() <= 2 ** -7 * np.abs(ref).max()
    # finite differences on the gate
    eps = 1e-6
    f = lambda gg: gg / (1 + np.exp(-gg)) * u
    num = (f(g + eps) - f(g - eps)) / (2 * eps) * d
    assert np.abs(ref[:, :256] - num).max() <= 1e-6 * np.abs(num).max() + 1e-9


def test_combine_bwd_against_float64_autograd_and_identities():
    """combine_bwd pinned on its own: dw and the unrounded dy are the
    gradients float64 autograd takes through the combine's definition
    out[t] = sum_k w[t,k] * y[inv_map[t*K+k]] (the forward C7 restates,
    pinned by test_combine_identity_and_scalar_loop); dy is that gradient
    rounded once to bf16; dw is linear in dout; and the adjoint identity
    <combine(y, w), dout> = sum(w * dw) holds in float64."""
    rng = np.random.default_rng(71)
    T, K, H = 37, 3, 256
    R = T * K
    inv = rng.permutation(R).astype(np.int32)
    y = O.f32_to_bf16(rng.standard_normal((R, H)).astype(np.float32))
    d1 = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    d2 = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    w = rng.random((T, K)).astype(np.float32)
    dy, dw = O.combine_bwd(d1, y, inv, w, K)
    yt = torch.from_numpy(O.bf16_to_f32(y).astype(np.float64)).requires_grad_(True)
    wt = torch.from_numpy(w.astype(np.float64)).requires_grad_(True)
    out = (wt[:, :, None] * yt[torch.from_numpy(inv.astype(np.int64)).view(T, K)]).sum(1)
    dt = torch.from_numpy(O.bf16_to_f32(d1).astype(np.float64))
    (out * dt).sum().backward()
    assert np.allclose(dw, wt.grad.numpy(), rtol=1e-12, atol=1e-12)
    # dy: the autograd gradient (exact in fp32: one product of a bf16 and an
    # fp32 value) rounded once to bf16
    g32 = yt.grad.numpy().astype(np.float32)
    assert np.array_equal(dy, O.f32_to_bf16(g32))
    # linearity in dout
    _, dw2 = O.combine_bwd(d2, y, inv, w, K)
    d12 = O.f32_to_bf16((O.bf16_to_f32(d1) + 2 * O.bf16_to_f32(d2)).astype(np.float32))
    _, dw12 = O.combine_bwd(d12, y, inv, w, K)
    ref12 = np.einsum("th,tkh->tk", O.bf16_to_f32(d12).astype(np.float64),
                      O.bf16_to_f32(y).astype(np.float64)[inv.reshape(T, K)])
    assert np.allclose(dw12, ref12, rtol=1e-12, atol=1e-10)
    exact12 = O.bf16_to_f32(d12) == O.bf16_to_f32(d1) + 2 * O.bf16_to_f32(d2)
    if exact12.all():
        assert np.allclose(dw12, dw + 2 * dw2, rtol=1e-10, atol=1e-10)
    # adjoint identity, with out in float64 from the definition
    lhs = float((out.detach() * dt).sum())
    assert abs(lhs - float((w.astype(np.float64) * dw).sum())) <= 1e-9 * max(1.0, abs(lhs))


def test_combine_bwd_k1_unit_weight_is_inverse_scatter():
    """K = 1, w = 1: dy is dout scattered through inv_map, byte for byte, and
    dw[t] = <dout[t], y[inv_map[t]]> exactly in float64 (bf16 products are
    exact there)."""
    rng = np.random.default_rng(72)
    T, H = 301, 384
    inv = rng.permutation(T).astype(np.int32)
    y = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    d = O.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    dy, dw = O.combine_bwd(d, y, inv, np.ones((T, 1), np.float32), 1)
    want = np.zeros_like(dy)
    want[inv] = d
    assert np.array_equal(dy, want)
    prod = O.bf16_to_f32(d).astype(np.float64) * O.bf16_to_f32(y).astype(np.float64)[inv]
    assert np.array_equal(dw[:, 0], prod.sum(1))


def test_moe_backward_against_float64_autograd():
    """The whole backward against torch autograd in float64 on the
    dequantised weights with the same routing: quantisation noise only."""
    g = np.load(os.path.join(GOLDEN, "oracle_tiny.npz"))
    K = int(g["K"])
    rng = np.random.default_rng(12)
    dout = O.f32_to_bf16(rng.standard_normal(g["out"].shape).astype(np.float32))
    fwd = {k: g[k] for k in ("topk_idx", "topk_w", "row_map", "inv_map", "offsets", "c1", "y")}
    b = O.moe_backward(fwd, g["x"], g["w1q"], g["w1s"], g["w2q"], g["w2s"], dout, K)
    E = g["w1q"].shape[0]
    W1 = torch.tensor(np.stack([O.dequant_weight(g["w1q"][e], g["w1s"][e]) for e in range(E)]), requires_grad=True)
    W2 = torch.tensor(np.stack([O.dequant_weight(g["w2q"][e], g["w2s"][e]) for e in range(E)]), requires_grad=True)
    x = torch.tensor(O.bf16_to_f32(g["x"]).astype(np.float64), requires_grad=True)
    wts = torch.tensor(g["topk_w"].astype(np.float64), requires_grad=True)
    T = x.shape[0]
    out = torch.zeros_like(x)
    outs = []
    for t in range(T):
        acc = 0
        for k in range(K):
            e = int(g["topk_idx"][t, k])
            c = W1[e] @ x[t]
            I = c.shape[0] // 2
            h = torch.nn.functional.silu(c[:I]) * c[I:]
            acc = acc + wts[t, k] * (W2[e] @ h)
        outs.append(acc)
    out = torch.stack(outs)
    loss = (out * torch.tensor(O.bf16_to_f32(dout).astype(np.float64))).sum()
    loss.backward()
    rel = lambda a, r: np.abs(a - r).max() / np.abs(r).max()
    assert rel(O.bf16_to_f32(b["dx"]).astype(np.float64), x.grad.numpy()) < 0.1
    assert rel(b["dW1"], W1.grad.numpy()) < 0.1
    assert rel(b["dW2"], W2.grad.numpy()) < 0.1
    assert rel(b["dw"], wts.grad.numpy()) < 0.08


def test_cpu_torch_dispatch_matches_oracle():
    """The multi-threaded PyTorch-CPU dispatch that bench.py times as its CPU
    baseline computes exactly the oracle's sort, maps and fp8 bytes/scales."""
    from oracle import cpu_torch
    rng = np.random.default_rng(11)
    for T, H, E, K in ((512, 1024, 64, 8), (97, 384, 5, 3), (1, 128, 1, 1)):
        x = (rng.standard_normal((T, H)) * np.exp2(rng.integers(-8, 8, (T, H)))).astype(np.float32)
        x[0, :128] = 0.0
        if T > 2:
            x[1, 5] = 3.0e38
            x[2, :] = 1e-40
        xb = O.f32_to_bf16(x)
        idx = rng.integers(0, E, (T, K)).astype(np.int32)
        xt = torch.from_numpy(xb.view(np.int16)).view(torch.bfloat16)
        xq, xs, rm, im, cnt, off = cpu_torch.dispatch_quant(xt, torch.from_numpy(idx), E)
        r_rm, r_im, r_cnt, r_off = O.route_sort(idx, E)
        rq, rs = O.permute_quant(xb, r_im, K)
        assert np.array_equal(rm.numpy(), r_rm) and np.array_equal(im.numpy(), r_im)
        assert np.array_equal(cnt.numpy(), r_cnt) and np.array_equal(off.numpy(), r_off)
        assert np.array_equal(xq.numpy(), rq)
        assert np.array_equal(xs.numpy().view(np.uint32), rs.view(np.uint32))


def test_cpu_torch_gemm_matches_oracle():
    """The PyTorch-CPU grouped GEMM that bench.py times as the GEMM's CPU
    baseline agrees with the float64 oracle within the GEMM tolerance
    (max 1e-2, mean 1e-3 of the reference magnitude), zero-token experts
    included."""
    from oracle import cpu_torch
    rng = np.random.default_rng(12)
    counts = [5, 0, 130, 1, 0, 64]
    E, N, Kd = len(counts), 256, 384
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    R = int(off[-1])
    xq, xs = O.quant_1x128(rng.standard_normal((R, Kd)).astype(np.float32))
    w = O.f32_to_bf16((rng.standard_normal((E, N, Kd)) * 0.05).astype(np.float32))
    wq, wsc = O.quantize_weight_blockwise(w)
    ref = O.grouped_gemm_fp8(xq, xs, wq, wsc, off)
    got = cpu_torch.grouped_gemm_fp8(torch.from_numpy(xq), torch.from_numpy(xs), torch.from_numpy(wq),
                                     torch.from_numpy(wsc), off).numpy().astype(np.float64)
    d = np.abs(got - ref)
    assert d.max() / np.abs(ref).max() <= 1e-2
    assert d.mean() / np.abs(ref).mean() <= 1e-3
