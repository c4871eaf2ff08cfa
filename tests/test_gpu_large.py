"""Large sizes: dispatch and combine where the byte offsets pass 2^32, so
any 32-bit index arithmetic would wrap.  The oracle cannot run at this size,
so the checks are size-independent properties plus an oracle comparison on a
sample of tokens:
  * every token's K sorted rows hold byte-identical fp8 rows and scales;
  * sampled tokens (including the last one) match the oracle's 1x128 bytes;
  * the combine with one-hot weights is an exact inverse of the permutation."""
import sys

import numpy as np
import pytest
import torch

from oracle import smoe_oracle as O
from smoe import ops, workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def test_dispatch_and_combine_past_4gib(dev):
    T, K, H, E = 1 << 21, 8, 384, 64
    R = T * K
    say("large dispatch/combine", T, K, H, E, f"xq {R * H / 2**30:.0f} GiB")
    assert R * H > 2**32  # byte offsets into xq exceed 32 bits
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    idx = torch.randint(0, E, (T, K), generator=g, device=dev, dtype=torch.int32)
    xq, xs, rm, im, cnt, off = ops.permute_quant(x, idx, E)
    torch.cuda.synchronize()
    assert int(off[-1]) == R and int(cnt.sum()) == R
    q8 = xq.view(torch.uint8)
    inv = im.view(T, K).long()
    # replicas: chunk over tokens to bound the gathered copies
    step = 1 << 17
    for t0 in range(0, T, step):
        rows = inv[t0:t0 + step]
        first = q8[rows[:, 0]]
        firsts = xs[rows[:, 0]]
        for k in range(1, K):
            assert torch.equal(q8[rows[:, k]], first), f"token replicas differ near t={t0}"
            assert torch.equal(xs[rows[:, k]].view(torch.int32), firsts.view(torch.int32))
    # oracle on a sample, including the first and last tokens
    rng = np.random.default_rng(3)
    sample = np.unique(np.concatenate([[0, T - 1], rng.integers(0, T, 510)]))
    xs_np = x[torch.from_numpy(sample).to(dev)].cpu().view(torch.int16).numpy().view(np.uint16)
    rq, rs = O.quant_1x128(O.bf16_to_f32(xs_np))
    r0 = inv[torch.from_numpy(sample).to(dev), 0]
    assert np.array_equal(q8[r0].cpu().numpy(), rq)
    assert np.array_equal(xs[r0].cpu().numpy().view(np.uint32), rs.view(np.uint32))
    del q8, xq, xs
    torch.cuda.empty_cache()
    # combine: y[r] = x[row_map[r] // K] (bf16, 8 GiB); one-hot weights pick
    # k = 0, so out must reproduce x exactly
    y = x[(rm.long() // K)]
    w = torch.zeros((T, K), dtype=torch.float32, device=dev)
    w[:, 0] = 1.0
    out = ops.unpermute_combine(y, im, w)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), x.view(torch.int16))
    del y, out
    torch.cuda.empty_cache()


def test_gemm_activations_past_4gib(dev):
    """Grouped GEMM whose activation operand is 8 GiB (2^20 rows x K = 8192):
    row offsets pass 2^32 bytes.  Sampled rows, including the first and
    last rows of every expert, are checked against the float64 oracle."""
    R, N, Kd = 1 << 20, 256, 8192
    counts = [200_000, 1, 500_000, R - 700_001]
    assert sum(counts) == R
    E = len(counts)
    say("large gemm", R, N, Kd, counts)
    assert R * Kd > 2**32
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    # random finite e4m3 bytes (0x7f / 0xff are NaN), generated in 2^16-row
    # chunks so that no elementwise op spans more than 2^31 elements
    a = torch.empty((R, Kd), dtype=torch.uint8, device=dev)
    for r0 in range(0, R, 1 << 16):
        blk = torch.randint(0, 0x7f, (1 << 16, Kd), generator=g, device=dev, dtype=torch.uint8)
        sign = torch.randint(0, 2, (1 << 16, Kd), generator=g, device=dev, dtype=torch.uint8)
        a[r0:r0 + (1 << 16)] = blk | (sign << 7)
    del blk, sign
    a_s = torch.rand((R, Kd // 128), generator=g, device=dev) * 1e-2 + 1e-3
    w = (torch.randn((E, N, Kd), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    wq, ws = ops.quantize_weight_blockwise(w)
    off = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32, device=dev)
    out = ops.grouped_gemm_fp8(a, a_s, wq, ws, off)
    # the packed-weight kernel on the same operands; these activation bytes
    # span the whole e4m3 range, so a K block's 128 products need not sum
    # exactly in fp32 and the two kernels' MFMA K orders may differ in the
    # last bit: each is held to the oracle
    outp = ops.grouped_gemm_fp8(a, a_s, ops.pack_weight_fp8(wq), ws, off)
    torch.cuda.synchronize()
    offs = np.concatenate([[0], np.cumsum(counts)])
    rng = np.random.default_rng(9)
    rows = np.unique(np.concatenate([offs[:-1], offs[1:] - 1, rng.integers(0, R, 200)]))
    ridx = torch.from_numpy(rows).to(dev)
    aq_np = a[ridx].cpu().numpy()
    as_np = a_s[ridx].cpu().numpy()
    wq_np, ws_np = wq.view(torch.uint8).cpu().numpy(), ws.cpu().numpy()
    ref = np.empty((len(rows), N))
    for i, r in enumerate(rows):
        e = int(np.searchsorted(offs, r, side="right") - 1)
        ref[i] = O.dequant_rows(aq_np[i:i + 1], as_np[i:i + 1]) @ O.dequant_weight(wq_np[e], ws_np[e]).T
    ref_b = O.bf16_to_f32(O.f32_to_bf16(ref.astype(np.float32))).astype(np.float64)
    for res in (out, outp):
        got = O.bf16_to_f32(res[ridx].cpu().view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
        d = np.abs(got - ref_b)
        assert d.max() / np.abs(ref_b).max() <= 1e-2 and d.mean() / np.abs(ref_b).mean() <= 1e-3
    del a, a_s, out, outp
    torch.cuda.empty_cache()
