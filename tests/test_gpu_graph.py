"""Graph capture: the layer's launches are stream-ordered with no host
synchronisation, memset or allocation inside the library, so a caller can
capture them in a HIP graph (torch.cuda.CUDAGraph).  Each captured graph is
replayed several times with the program's own eager work and
synchronisations in between, and every replay must reproduce the eager
result bit for bit."""
import sys

import pytest
import torch

import smoe
from smoe import workloads as W

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def _layer(dev, c):
    m = smoe.SimpleMoE(c.H, c.I, c.E, c.K, device=dev)
    with torch.no_grad():
        m.w1.copy_(W.weights(c.E, 2 * c.I, c.H).to(dev))
        m.w2.copy_(W.weights(c.E, c.H, c.I, seed=13).to(dev))
    m.fp8_weights()  # weight quantisation stays outside the graph
    return m


def _i16(t):
    return t.contiguous().view(torch.int16)


def _capture(fn):
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up outside the graph (allocator pools, one-time set-up)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def test_forward_graph_replays(dev):
    say("graph: SimpleMoE forward")
    c = W.CONFIGS["tiny"]
    m = _layer(dev, c)
    x, lg = W.tokens(c.T, c.H).to(dev), W.logits(c.T, c.E).to(dev)
    x2, lg2 = W.tokens(c.T, c.H, seed=9).to(dev), W.logits(c.T, c.E, seed=8).to(dev)
    ref = m(x, lg).clone()
    torch.cuda.synchronize()
    g, out = _capture(lambda: m(x, lg))
    for i in range(4):
        out.zero_()
        other = m(x2, lg2)  # eager work on other data between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(_i16(out), _i16(ref)), f"replay {i} differs from the eager forward"
        del other


def test_forward_backward_graph_replays(dev):
    say("graph: SimpleMoE forward + backward")
    c = W.CONFIGS["tiny"]
    m = _layer(dev, c)
    x, lg = W.tokens(c.T, c.H).to(dev), W.logits(c.T, c.E).to(dev)
    dout = (W.tokens(c.T, c.H, seed=4).float() * 1e-3).to(torch.bfloat16).to(dev)

    def step():
        out, inter = m(x, lg, return_intermediates=True)
        g = m.backward_from(inter, dout)
        return out, g["dx"], g["dw1"], g["dw2"], g["dtopk_w"]

    ref = [t.clone() for t in step()]
    torch.cuda.synchronize()
    graph, outs = _capture(step)
    for i in range(3):
        for t in outs:
            t.zero_()
        step()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, want in zip(("out", "dx", "dw1", "dw2", "dtopk_w"), outs, ref):
            assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), \
                f"replay {i}: {name} differs from the eager step"


def test_two_streams_concurrent(dev):
    """Calls on two streams at once (each with its own buffers and sort
    workspace) give the same bytes as the same calls run one after the
    other."""
    say("two streams")
    from smoe import ops
    c = W.CONFIGS["tiny"]
    m = _layer(dev, c)
    w1q, w1s, _, _ = m.fp8_weights()
    xs_ = [W.tokens(c.T, c.H, seed=s).to(dev) for s in (1, 2)]
    idx = [ops.router_topk(W.logits(c.T, c.E, seed=s).to(dev), c.K)[0] for s in (3, 4)]

    def work(i):
        xq, xsc, rm, im, cnt, off = ops.permute_quant(xs_[i], idx[i], c.E)
        return xq, xsc, rm, ops.grouped_gemm_fp8(xq, xsc, w1q, w1s, off)

    serial = [[t.clone() for t in work(i)] for i in (0, 1)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    res = [None, None]
    for rep in range(3):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                res[i] = work(i)
        torch.cuda.synchronize()
        for i in (0, 1):
            for got, want in zip(res[i], serial[i]):
                assert torch.equal(got.view(torch.uint8), want.view(torch.uint8)), f"stream {i} rep {rep}"


def test_backward_on_a_caller_stream(dev):
    """backward_from orders its weight-gradient stream after whatever stream
    the caller runs on, and that stream after it: forward + backward on a
    non-default stream, twice, with the caller's stream reading the results
    right away (no host sync in between), give the default-stream bytes."""
    say("backward on a caller stream")
    c = W.CONFIGS["tiny"]
    m = _layer(dev, c)
    x, lg = W.tokens(c.T, c.H).to(dev), W.logits(c.T, c.E).to(dev)
    dout = (W.tokens(c.T, c.H, seed=4).float() * 1e-3).to(torch.bfloat16).to(dev)

    def step():
        out, inter = m(x, lg, return_intermediates=True)
        g = m.backward_from(inter, dout)
        return [out, g["dx"], g["dw1"], g["dw2"], g["dtopk_w"]]

    ref = [t.clone() for t in step()]
    torch.cuda.synchronize()
    user = torch.cuda.Stream()  # default priority
    user.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(user):
        for rep in range(2):
            got = step()
            # copies enqueued on the caller's stream straight after the call
            snap = [t.clone() for t in got]
            del got
    torch.cuda.current_stream().wait_stream(user)
    torch.cuda.synchronize()
    for name, a, b in zip(("out", "dx", "dw1", "dw2", "dtopk_w"), snap, ref):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"{name} differs on a caller stream"
