"""Seeded random shapes for the path's main entry points against the oracle.

The parametrized tests elsewhere pick their edge cases by hand; these draw
expert counts (empty experts, single rows, counts just past and short of a
256-row tile), widths and depths at random from fixed seeds, so that shapes
nobody thought of are covered too.  Each case is small enough for the
float64 oracle to finish in well under a second:
- the router and the expert sort: ids, weights and maps bit-exact;
- the grouped GEMM, plain, packed and E8M0 (where the shape allows each):
  within the GEMM bar of the oracle on every row;
- the variable-K weight-gradient GEMM, C3 and E8M0 operands: within the GEMM
  bar, and zero for experts with no rows;
- the byte-moving stages (permute + quantise, SwiGLU + quantise, the column
  quantiser, the combine and both halves of its backward): bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import smoe_oracle as O
from smoe import ops, workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[sweep]", *a, flush=True)


def u16(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def u8(t):
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def close(got, ref, what, mx_tol=1e-2, mn_tol=1e-3):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    mx = d.max() / max(np.abs(ref).max(), 1e-30)
    mn = d.mean() / max(np.abs(ref).mean(), 1e-30)
    assert mx <= mx_tol and mn <= mn_tol, f"{what}: max_rel={mx:.3e} mean_rel={mn:.3e}"


def _counts(rng, E, R_max):
    """Expert row counts with the kinds of loads that stress tile edges."""
    kinds = rng.integers(0, 6, E)
    c = np.where(kinds == 0, 0,
        np.where(kinds == 1, 1,
        np.where(kinds == 2, 256 * rng.integers(1, 3, E) + rng.integers(-1, 2, E),
        np.where(kinds == 3, rng.integers(2, 128, E),
                 rng.integers(129, 600, E)))))
    c = np.maximum(c, 0)
    while c.sum() > R_max:
        c = c // 2
    return c.astype(np.int64)


ROUTE_SEEDS = list(range(8))


@pytest.mark.parametrize("seed", ROUTE_SEEDS)
def test_sweep_router_and_sort(dev, seed):
    rng = np.random.default_rng(100 + seed)
    E = int(rng.choice([1, 2, 7, 16, 64, 128, 256, 300]))
    K = int(rng.integers(1, min(E, 9) + 1))
    T = int(rng.integers(1, 3000))
    bias = rng.random() < 0.5
    say("router", seed, T, E, K, bias)
    logits = (rng.standard_normal((T, E)) * rng.choice([0.1, 1.0, 8.0])).astype(np.float32)
    if T > 2:
        logits[1] = logits[1, 0]  # a row of ties: lowest ids win
    b = (rng.standard_normal(E) * 0.5).astype(np.float32) if bias else None
    idx, w = ops.router_topk(torch.from_numpy(logits).to(dev), K,
                             None if b is None else torch.from_numpy(b).to(dev))
    ridx, rw = O.router_topk(logits, K, b)
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.astype(np.float32).view(np.uint32))
    row_map, inv_map, counts, offsets = ops.route_sort(idx, E)
    rrow, rinv, rcnt, roff = O.route_sort(ridx, E)
    for got, ref in ((row_map, rrow), (inv_map, rinv), (counts, rcnt), (offsets, roff)):
        assert np.array_equal(got.cpu().numpy(), ref)


GEMM_SEEDS = list(range(10))


@pytest.mark.parametrize("seed", GEMM_SEEDS)
def test_sweep_grouped_gemm(dev, seed):
    rng = np.random.default_rng(200 + seed)
    E = int(rng.integers(1, 24))
    counts = _counts(rng, E, 3000)
    N = 16 * int(rng.integers(1, 65))
    Kd = 128 * int(rng.choice([1, 2, 3, 4, 5, 6, 8, 12, 16]))
    say("gemm", seed, counts.tolist(), N, Kd)
    R = int(counts.sum())
    off = W.offsets_from_counts(counts.tolist(), dev)
    off_np = off.cpu().numpy()
    rows = max(R, 1)
    for pow2 in (False, True):
        scale = "pow2" if pow2 else "amax"
        xq, xs = ops.quant_rows(W.tokens(rows, Kd, device=dev, seed=300 + seed), scale=scale)
        wq, ws = ops.quantize_weight_blockwise(W.weights(E, N, Kd, device=dev, seed=400 + seed),
                                               scale=scale)
        ref = O.grouped_gemm_fp8(u8(xq), xs.cpu().numpy(), u8(wq), ws.cpu().numpy(), off_np)
        ref = O.bf16_to_f32(O.f32_to_bf16(ref.astype(np.float32)))[:R]
        runs = []
        if not pow2:
            runs.append(("plain", lambda: ops.grouped_gemm_fp8(xq, xs, wq, ws, off)))
            if ops.packed_gemm_ok(N, Kd):
                wp = ops.pack_weight_fp8(wq)
                runs.append(("packed", lambda: ops.grouped_gemm_fp8(xq, xs, wp, ws, off)))
        elif ops.packed_e8m0_ok(N, Kd):
            wp2 = ops.pack_weight_fp8(wq)
            runs.append(("e8m0", lambda: ops.grouped_gemm_fp8(xq, xs, wp2, ws, off, e8m0=True)))
        for name, run in runs:
            got = run()
            torch.cuda.synchronize()
            if R:
                close(O.bf16_to_f32(u16(got[:R])), ref, f"{name} gemm seed {seed}")


WGRAD_SEEDS = list(range(6))


@pytest.mark.parametrize("seed", WGRAD_SEEDS)
def test_sweep_wgrad(dev, seed):
    rng = np.random.default_rng(500 + seed)
    E = int(rng.integers(1, 12))
    counts = _counts(rng, E, 2500)
    if counts.sum() == 0:
        counts[0] = 3
    N = 16 * int(rng.integers(1, 49))
    K = 16 * int(rng.integers(1, 49))
    say("wgrad", seed, counts.tolist(), N, K)
    off = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    R = int(off[-1])
    dy = W.tokens(R, N, seed=600 + seed)
    h = W.tokens(R, K, seed=700 + seed)
    off_t = torch.from_numpy(off).to(dev)
    for pow2 in (False, True):
        cs = "pow2" if pow2 else "fp32"
        aq, as_, pad, ld = ops.quant_cols(dy.to(dev), off_t, col_scale=cs)
        bq, bs_, _, _ = ops.quant_cols(h.to(dev), off_t, col_scale=cs)
        got = ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld, e8m0=pow2).cpu().numpy()
        raq, ras, rpad = O.quant_cols_128x1(O.bf16_to_f32(u16(dy)), off, pow2=pow2)
        rbq, rbs, _ = O.quant_cols_128x1(O.bf16_to_f32(u16(h)), off, pow2=pow2)
        assert np.array_equal(pad.cpu().numpy(), rpad)
        ref = O.grouped_gemm_fp8_wgrad(raq, ras, rbq, rbs, rpad, E)
        for e in range(E):
            if counts[e] == 0:
                assert not got[e].any(), f"expert {e} has no rows but a non-zero gradient"
        close(got, ref, f"wgrad seed {seed} pow2={pow2}")


DATA_SEEDS = list(range(8))


@pytest.mark.parametrize("seed", DATA_SEEDS)
def test_sweep_data_path(dev, seed):
    """Permute + quantise, SwiGLU + quantise, the combine, the column
    quantiser and the combine backward (both halves), all bit-exact, on a
    random routing of random sizes (widths a multiple of 16, so the short
    last 128-group of the C9 rule shows up too), C3 and C10 scales."""
    rng = np.random.default_rng(800 + seed)
    E = int(rng.choice([1, 3, 8, 33, 128]))
    K = int(rng.integers(1, min(E, 8) + 1))
    T = int(rng.integers(1, 900))
    H = 16 * int(rng.integers(1, 97))
    I = 16 * int(rng.integers(1, 49))
    say("data path", seed, T, E, K, H, I)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    idx, w = ops.router_topk(torch.from_numpy(logits).to(dev), K)
    row_map, inv_map, _, offsets = ops.route_sort(idx, E)
    inv = inv_map.cpu().numpy()
    off = offsets.cpu().numpy()
    w_np = w.cpu().numpy()
    R = T * K
    x = W.tokens(T, H, device=dev, seed=900 + seed)
    y = W.tokens(R, H, device=dev, seed=1000 + seed)
    c1 = W.tokens(R, 2 * I, device=dev, seed=1100 + seed)
    dout = W.tokens(T, H, device=dev, seed=1200 + seed)
    for pow2 in (False, True):
        scale = "pow2" if pow2 else "amax"
        xq, xs = ops.permute_quant_rows(x, inv_map, K, scale=scale)
        rq, rs = O.permute_quant(u16(x), inv, K, pow2=pow2)
        assert np.array_equal(u8(xq), rq) and np.array_equal(xs.cpu().numpy(), rs), "permute"
        hq, hs = ops.swiglu_quant(c1, scale=scale)
        rq, rs = O.swiglu_quant(u16(c1), pow2=pow2)
        assert np.array_equal(u8(hq), rq) and np.array_equal(hs.cpu().numpy(), rs), "swiglu"
        cq, cs, pad, _ = ops.quant_cols(y, offsets, col_scale="pow2" if pow2 else "fp32")
        rq, rs, rpad = O.quant_cols_128x1(O.bf16_to_f32(u16(y)), off, pow2=pow2)
        Rp = int(rpad[-1])
        assert np.array_equal(pad.cpu().numpy(), rpad)
        assert np.array_equal(u8(cq)[:, :Rp], rq), "columns"
        assert np.array_equal(cs.cpu().numpy()[:, :Rp // 128], rs), "column scales"
    out = ops.unpermute_combine(y, inv_map, w)
    assert np.array_equal(u16(out), O.unpermute_combine(u16(y), inv, w_np, K)), "combine"
    dy, dw = ops.unpermute_combine_bwd(dout, y, inv_map, w)
    rdy, rdw = O.combine_bwd(u16(dout), u16(y), inv, w_np, K)
    assert np.array_equal(u16(dy), rdy), "combine backward dy"
    close(dw.cpu().numpy(), rdw, "combine backward dw")
    for cs_name, pow2 in (("fp32", False), ("pow2", True)):
        tq, ts, tpad, _ = ops.combine_bwd_quant_cols(dout, row_map, w, offsets, col_scale=cs_name)
        rq, rs, rpad = O.quant_cols_128x1(O.bf16_to_f32(rdy), off, pow2=pow2)
        Rp = int(rpad[-1])
        assert np.array_equal(tpad.cpu().numpy(), rpad)
        assert np.array_equal(u8(tq)[:, :Rp], rq), "dy columns"
        assert np.array_equal(ts.cpu().numpy()[:, :Rp // 128], rs), "dy column scales"
