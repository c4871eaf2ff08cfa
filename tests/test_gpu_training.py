"""The training path around the fp8 backward: the wgrad output modes
(fp32 / bf16, written / accumulated into a main_grad buffer), gradient
accumulation through autograd, a second backward with retain_graph, the
dgrad running on the weights its forward used, and the fp8 weight cache
following optimizer steps that write parameters through ``.data``.

Bars: the accumulating modes are bit-identical to a separate fp32 (or
fp32-then-bf16) addition of the written fp32 gradient, since they perform
the same one addition per value; main_grad after two accumulated backwards
equals the sum of the two backwards' fp32 weight gradients exactly and the
float64 oracle's dW1 + dW1' within the backward tolerance (max 2e-2, mean
5e-3 of the weight gradient, as for w1.grad in test_gpu_configs)."""
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


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


def close(got, ref, what, mx_tol=1e-2, mn_tol=1e-3):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    mx = d.max() / max(np.abs(ref).max(), 1e-30)
    mn = d.mean() / max(np.abs(ref).mean(), 1e-30)
    assert mx <= mx_tol and mn <= mn_tol, f"{what}: max_rel={mx:.3e} mean_rel={mn:.3e}"


def _model(dev, c, seed=0):
    m = smoe.SimpleMoE(c.H, c.I, c.E, c.K, device=dev)
    with torch.no_grad():
        m.w1.copy_(W.weights(c.E, 2 * c.I, c.H, device=dev, seed=3 + seed))
        m.w2.copy_(W.weights(c.E, c.H, c.I, device=dev, seed=13 + seed))
    return m


def _wgrad_operands(dev, R, N, K, counts, seed):
    off = W.offsets_from_counts(torch.tensor(counts), dev)
    a = W.tokens(R, N, device=dev, seed=seed)
    b = W.tokens(R, K, device=dev, seed=seed + 1)
    aTq, aTs, pad, ld = ops.quant_cols(a, off)
    bTq, bTs, _, _ = ops.quant_cols(b, off)
    return aTq, aTs, bTq, bTs, pad, ld


def test_wgrad_output_modes(dev):
    """fp32 accumulate == buffer + fp32 gradient; bf16 == RNE(fp32 gradient);
    bf16 accumulate == RNE(float(buffer) + fp32 gradient); all bit for bit,
    and experts without rows leave an accumulation buffer untouched (an
    empty expert, and tiles past N and K of a 384 x 640 gradient)."""
    E, N, K = 6, 384, 640
    counts = [300, 0, 129, 1, 0, 500]
    R = sum(counts)
    say("wgrad modes", E, N, K, counts)
    aTq, aTs, bTq, bTs, pad, ld = _wgrad_operands(dev, R, N, K, counts, 31)
    ref = ops.grouped_gemm_fp8_wgrad(aTq, aTs, bTq, bTs, pad, ld)
    g = torch.Generator(device=dev).manual_seed(5)
    base = torch.randn((E, N, K), generator=g, device=dev)
    acc = base.clone()
    ops.grouped_gemm_fp8_wgrad(aTq, aTs, bTq, bTs, pad, ld, out=acc, accumulate=True)
    want = base + ref
    assert torch.equal(acc.view(torch.int32), want.view(torch.int32))
    for e in (1, 4):
        assert torch.equal(acc[e], base[e]) and torch.equal(ref[e], torch.zeros_like(ref[e]))
    b16 = ops.grouped_gemm_fp8_wgrad(aTq, aTs, bTq, bTs, pad, ld, dtype=torch.bfloat16)
    assert b16.dtype == torch.bfloat16
    assert torch.equal(b16.view(torch.int16), ref.to(torch.bfloat16).view(torch.int16))
    base16 = base.to(torch.bfloat16)
    acc16 = base16.clone()
    ops.grouped_gemm_fp8_wgrad(aTq, aTs, bTq, bTs, pad, ld, out=acc16, accumulate=True)
    want16 = (base16.float() + ref).to(torch.bfloat16)
    assert torch.equal(acc16.view(torch.int16), want16.view(torch.int16))
    # and against the oracle (fp32 mode), at the GEMM tolerance
    r = O.grouped_gemm_fp8_wgrad(u8(aTq), aTs.cpu().numpy(), u8(bTq), bTs.cpu().numpy(),
                                 pad.cpu().numpy(), E)
    close(ref.cpu().numpy(), r, "dW")
    with pytest.raises(ValueError):
        ops.grouped_gemm_fp8_wgrad(aTq, aTs, bTq, bTs, pad, ld, accumulate=True)
    lib = smoe._C.lib()
    st = lib.smoe_grouped_gemm_fp8_wgrad_ex(aTq.data_ptr(), aTs.data_ptr(), bTq.data_ptr(),
                                            bTs.data_ptr(), pad.data_ptr(), E, N, K, ld,
                                            acc.data_ptr(), 8, None)
    assert st == -8  # SMOE_EINVAL_MODE, rejected before any launch


def test_main_grad_accumulates_two_backwards(dev):
    """Two forward + backward passes through autograd on different inputs with
    fp32 main_grad buffers on w1 and w2: main_grad equals the two fp32 weight
    gradients of backward_from summed (bit for bit), and the oracle's
    dW1 + dW1' within tolerance; the parameters' .grad stays None.  A bf16
    main_grad gets RNE(float(bf16 buffer) + fp32 gradient) per backward."""
    T, H, I, E, K = 512, 256, 256, 8, 2
    c = W.Config("mg", T=T, H=H, E=E, K=K, I=I)
    say("main_grad accumulation", T, H, I, E, K)
    m = _model(dev, c)
    m.w1.main_grad = torch.zeros(m.w1.shape, dtype=torch.float32, device=dev)
    m.w2.main_grad = torch.zeros(m.w2.shape, dtype=torch.float32, device=dev)
    runs = []
    for s in (0, 1):
        x = W.tokens(T, H, seed=40 + s).to(dev)
        lg = W.logits(T, E, seed=50 + s).to(dev).requires_grad_(True)
        dout = W.tokens(T, H, seed=60 + s).to(dev)
        m(x, lg).backward(dout)
        _, st = m(x, lg.detach(), return_intermediates=True)
        g = m.backward_from(st, dout)
        runs.append((x, st, dout, g))
    assert m.w1.grad is None and m.w2.grad is None
    want1 = runs[0][3]["dw1"] + runs[1][3]["dw1"]
    want2 = runs[0][3]["dw2"] + runs[1][3]["dw2"]
    assert torch.equal(m.w1.main_grad, want1) and torch.equal(m.w2.main_grad, want2)
    w1q, w1s, w2q, w2s = m.fp8_weights()
    r_sum = None
    for x, st, dout, _ in runs:
        fwd = {k: (u16(v) if v.dtype == torch.bfloat16 else v.cpu().numpy())
               for k, v in st.items()
               if isinstance(v, torch.Tensor) and k in ("topk_w", "row_map", "inv_map", "offsets", "c1", "y")}
        r = O.moe_backward(fwd, u16(x), u8(w1q), w1s.cpu().numpy(), u8(w2q), w2s.cpu().numpy(),
                           u16(dout), K)
        r_sum = r if r_sum is None else {k: r_sum[k] + r[k] for k in ("dW1", "dW2")}
    close(m.w1.main_grad.cpu().numpy(), r_sum["dW1"], "main_grad w1", mx_tol=2e-2, mn_tol=5e-3)
    close(m.w2.main_grad.cpu().numpy(), r_sum["dW2"], "main_grad w2", mx_tol=2e-2, mn_tol=5e-3)
    # bf16 main_grad: one rounding per backward
    m.w1.main_grad = torch.zeros(m.w1.shape, dtype=torch.bfloat16, device=dev)
    del m.w2.main_grad
    want = torch.zeros(m.w1.shape, dtype=torch.bfloat16, device=dev)
    for x, st, dout, g in runs:
        lg = st["logits"].clone().requires_grad_(True)
        m(x, lg).backward(dout)
        want = (want.float() + g["dw1"]).to(torch.bfloat16)
    assert torch.equal(m.w1.main_grad.view(torch.int16), want.view(torch.int16))
    assert m.w2.grad is not None and m.w2.grad.dtype == torch.bfloat16
    del m.w1.main_grad


def test_retain_graph_second_backward(dev):
    """backward(retain_graph=True) twice accumulates the same gradients twice;
    a second backward without retain_graph raises PyTorch's error about
    freed saved tensors instead of failing inside the layer."""
    c = W.Config("rg", T=256, H=256, E=4, K=2, I=256)
    say("retain_graph")
    m = _model(dev, c)
    x = W.tokens(c.T, c.H).to(dev).requires_grad_(True)
    lg = W.logits(c.T, c.E).to(dev).requires_grad_(True)
    dout = W.tokens(c.T, c.H, seed=4).to(dev)
    out = m(x, lg)
    out.backward(dout, retain_graph=True)
    g1 = (x.grad.clone(), lg.grad.clone(), m.w1.grad.clone(), m.w2.grad.clone())
    out.backward(dout)
    assert torch.equal(x.grad, (g1[0].float() * 2).to(x.grad.dtype))
    assert torch.equal(lg.grad, g1[1] * 2)
    assert torch.equal(m.w1.grad, (g1[2].float() * 2).to(torch.bfloat16))
    out2 = m(x, lg)
    out2.backward(dout)
    with pytest.raises(RuntimeError, match="backward through the graph a second time"):
        out2.backward(dout)


def test_backward_uses_forward_weights(dev):
    """Weights updated in place between a forward and its backward: the
    dgrad still runs on the transposes of the fp8 weights the forward used
    (dx equals a backward with the weights left alone), and the next forward
    re-quantises."""
    c = W.Config("fw", T=256, H=256, E=4, K=2, I=256)
    say("backward on forward weights")
    m = _model(dev, c)
    x, lg = W.tokens(c.T, c.H).to(dev), W.logits(c.T, c.E).to(dev)
    dout = W.tokens(c.T, c.H, seed=4).to(dev)
    xr = x.clone().requires_grad_(True)
    m(xr, lg).backward(dout)
    ref = xr.grad.clone()
    m.zero_grad(set_to_none=True)
    xg = x.clone().requires_grad_(True)
    out = m(xg, lg)
    with torch.no_grad():
        m.w1.mul_(3.0)
        m.w2.mul_(0.5)
    y_new = m(x, lg).detach()  # re-quantises the cache
    out.backward(dout)
    assert torch.equal(xg.grad.view(torch.int16), ref.view(torch.int16))
    assert not torch.equal(y_new, out.detach())


def test_fp8_cache_follows_optimizer_data_writes(dev):
    """An optimizer that writes stepped weights back through ``p.data``
    (Megatron's main-param copy) leaves the version counter alone; the step
    of any torch optimizer re-keys the cache, so the next forward sees the
    new weights.  A bare ``.data`` write is picked up by
    ``refresh_fp8_cache()``."""
    c = W.Config("od", T=256, H=256, E=4, K=2, I=256)
    say("fp8 cache after .data writes")
    m = _model(dev, c)
    x, lg = W.tokens(c.T, c.H).to(dev), W.logits(c.T, c.E).to(dev)
    with torch.no_grad():
        y0 = m(x, lg)
    # a master copy stepped by a torch optimizer, then copied back via .data
    master = m.w1.detach().float().clone().requires_grad_(True)
    opt = torch.optim.SGD([master], lr=1.0)
    master.grad = torch.full_like(master, 0.01)
    opt.step()
    m.w1.data.copy_(master.detach())
    with torch.no_grad():
        y1 = m(x, lg)
    fresh = _model(dev, c)
    with torch.no_grad():
        fresh.w1.copy_(m.w1)
        y_ref = fresh(x, lg)
    assert not torch.equal(y0, y1)
    assert torch.equal(y1.view(torch.int16), y_ref.view(torch.int16))
    # a bare .data write, then an explicit refresh
    m.w2.data.mul_(2.0)
    m.refresh_fp8_cache()
    with torch.no_grad():
        fresh.w2.copy_(m.w2)
        assert torch.equal(m(x, lg).view(torch.int16), fresh(x, lg).view(torch.int16))
