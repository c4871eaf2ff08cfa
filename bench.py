#!/usr/bin/env python3
"""Benchmark of the SimpleMoE expert-layer hot path on one MI355X.

Headline (benchmark config 2, the permute+quantise shape the metric is quoted on): one step is
the dispatch of one batch — stable expert sort + fused permute/1x128 fp8
quantisation — for T=16384 tokens, H=7168, E=256, top-8, inputs resident in
HBM.  ``value`` is the algorithmic HBM traffic of that step
(T*H*2 + T*K*H + T*K*(H/128)*4 + T*K*4 + T*K*8 + (E+1)*4 bytes) per second,
from the median of K event-timed steps, each after a 1 GiB cache flush (the
input is 235 MB, so back to back it would partly sit in the last-level
cache).

Also reported on the same line:
  roofline      the dominant kernel (permute_quant) timed alone with HIP
                events on the launch stream, algorithmic bytes / duration,
                median of >= 20 flushed launches;
  cpu_baseline  the PyTorch-CPU restatement of the same dispatch step
                (oracle/cpu_torch.py) on a bounded sample of the same
                workload, multi-threaded on this host's CPU share;
  extra         the HBM ceiling for the dispatch step's read:write mix
                (smoe_bw_probe), the fused router + sort at config 2,
                fp8 grouped GEMM TFLOPS on benchmark config 4 (DeepSeek-V3
                local experts, Zipf loads, fc1 + fc2), the combine GB/s at
                config-2 size, the whole SimpleMoE forward of config 3 and the
                forward+backward step of config 5.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--skip-extra]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "system-lab_amd"))

HBM_PEAK_GBS = 8000.0
# HBM bytes per permute_quant launch at config 2 from rocprofv3 FETCH_SIZE
# (115,777 KiB x 2.0 copy calibration) + WRITE_SIZE (948,344 KiB x 1.0):
# profiles/permute_quant_cfg2.md
PERMUTE_TRAFFIC_BYTES = 1_208_214_832
FP8_PEAK_TFLOPS = 5000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed(fn, iters, warmup, blocks=3):
    """Mean ms per call over ``iters`` back-to-back calls on the current
    stream, bracketed by HIP events recorded on that stream (the stream the
    kernels use); the median over ``blocks`` such runs, so that a one-off
    host stall in one run does not set the figure.  Inputs may stay in L2 /
    the last-level cache between calls: reported as the warm figure only."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    means = []
    for _ in range(blocks):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        torch.cuda.synchronize()
        means.append(s.elapsed_time(e) / iters)
    return sorted(means)[len(means) // 2]


class Flush:
    """A ``mib`` MiB device buffer whose read (a max-reduction) evicts L2 and
    the 256 MiB last-level cache.  It reads rather than writes: a write
    leaves dirty lines whose write-back would be charged to the next timed
    call."""

    def __init__(self, mib=1024):
        import torch
        self.buf = torch.ones(mib << 18, dtype=torch.int32, device="cuda")

    def __call__(self):
        self.buf.max()


def timed_median(fn, iters=20, warmup=5, flush=None):
    """Median ms of ``iters`` single calls, each bracketed by its own HIP
    events on the current stream; with ``flush`` (a Flush), each call runs
    after the caches were flushed, so no call finds its inputs cached.  The
    stream is kept busy (the flush, or a short device spin) while fn is
    submitted, so the host's launch latency is not timed.  The
    benchmark contract's timing: median of >= 20 event-timed calls after 5
    warm-ups, flushed for the HBM-bound kernels."""
    import numpy as np
    import torch
    for _ in range(warmup):
        if flush:
            flush()
        fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(iters):
        torch.cuda.synchronize()
        # queued ahead of the start event with no host wait: the stream is
        # busy (the flush read, >100 us, or a device spin of about 50 us)
        # while the host records the start event and submits fn, so the timed
        # region holds fn's GPU work and not the host's submission latency
        if flush:
            flush()
        elif hasattr(torch.cuda, "_sleep"):  # torch's device spin (a private helper)
            torch.cuda._sleep(100_000)
        s.record()
        fn()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    return float(np.median(times))


def timed_cold(fn, iters=20, warmup=5, flush_mib=1024):
    """Median ms of ``iters`` calls, each after a ``flush_mib`` MiB read."""
    f = Flush(flush_mib)
    t = timed_median(fn, iters, warmup, f)
    del f
    return t


def dispatch_bytes(T, H, E, K):
    return T * H * 2 + T * K * H + T * K * (H // 128) * 4 + T * K * 4 + T * K * 8 + (E + 1) * 4


def permute_kernel_bytes(T, H, K):
    # read x once, read inv_map, write K fp8 rows and their scales
    return T * H * 2 + T * K * 4 + T * K * H + T * K * (H // 128) * 4


def cpu_baseline(c, budget_s=12.0):
    """The dispatch step on the host: the PyTorch-CPU restatement of route
    sort + permute + 1x128 quantisation (oracle/cpu_torch.py, byte-identical
    to the numpy oracle), multi-threaded on this host's CPU share, on a
    bounded sample of the config-2 tokens."""
    import numpy as np
    import torch
    from oracle import cpu_torch, smoe_oracle as O
    from smoe import workloads as W
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    Ts = 4096
    x = W.tokens(Ts, c.H, outliers=True)
    idx = torch.from_numpy(O.router_topk(W.logits(Ts, c.E).numpy(), c.K,
                                         W.router_bias(c.E).numpy())[0])
    cpu_torch.dispatch_quant(x, idx, c.E)  # warm-up
    times = []
    t_end = time.time() + budget_s
    while time.time() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        cpu_torch.dispatch_quant(x, idx, c.E)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    gbs = dispatch_bytes(Ts, c.H, c.E, c.K) / t / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"PyTorch-CPU route sort + permute + 1x128 quantisation (oracle/cpu_torch.py, "
                      f"byte-identical to the oracle) on {Ts} of {c.T} tokens (H={c.H}, E={c.E}, "
                      f"top-{c.K}), {threads} threads, median of {len(times)} runs, "
                      f"{t * 1e3:.1f} ms each"}


def cpu_gemm_baseline(xq, xs, w1q, w1s, c, rows=1024, experts=2, budget_s=8.0):
    """The grouped GEMM on the host: fp32 dequantise + matmul per expert
    (oracle/cpu_torch.py, within the GEMM tolerance of the float64 oracle),
    multi-threaded, on a bounded sample of the config-4 fc1 shape: ``experts``
    experts of ``rows`` rows each, K = H, N = 2I.  TFLOP/s counts the matmul
    FLOP only; the time includes the dequantisation."""
    import numpy as np
    import torch
    from oracle import cpu_torch
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    torch.set_num_threads(threads)
    R = rows * experts
    a = xq[:R].view(torch.uint8).cpu()
    a_s = xs[:R].cpu()
    w = w1q[:experts].view(torch.uint8).cpu()
    w_s = w1s[:experts].cpu()
    off = [i * rows for i in range(experts + 1)]
    flop = 2.0 * R * w.shape[1] * w.shape[2]
    cpu_torch.grouped_gemm_fp8(a, a_s, w, w_s, off)  # warm-up
    times = []
    t_end = time.time() + budget_s
    while time.time() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        cpu_torch.grouped_gemm_fp8(a, a_s, w, w_s, off)
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    return {"value": round(flop / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"PyTorch-CPU fp32 dequantise + matmul (oracle/cpu_torch.py) on {experts} experts "
                      f"x {rows} rows of the config-4 fc1 shape (K={c.H}, N={2 * c.I}), {flop:.3e} "
                      f"FLOP per run, {threads} threads, median of {len(times)} runs, "
                      f"{t * 1e3:.0f} ms each"}


def bench_gemm(dev, steps, warmup, skip_cpu=True):
    import torch
    from smoe import ops, workloads as W
    c = W.CONFIGS["dsv3"]
    counts = W.zipf_counts()
    off = W.offsets_from_counts(counts, dev)
    R = c.T
    inv = torch.arange(R, dtype=torch.int32, device=dev)
    xq, xs = ops.permute_quant_rows(W.tokens(R, c.H, device=dev), inv, 1)
    hq, hs = ops.permute_quant_rows(W.tokens(R, c.I, device=dev, seed=17), inv, 1)
    w1q, w1s = ops.quantize_weight_blockwise(W.weights(c.E, 2 * c.I, c.H, device=dev))
    w2q, w2s = ops.quantize_weight_blockwise(W.weights(c.E, c.H, c.I, device=dev, seed=13))
    torch.cuda.empty_cache()
    # the weights as SimpleMoE caches them for these shapes (K % 512 == 0):
    # packed in MFMA fragment order for the register-loaded kernel
    w1p, w2p = ops.pack_weight_fp8(w1q), ops.pack_weight_fp8(w2q)
    c1 = torch.empty((R, 2 * c.I), dtype=torch.bfloat16, device=dev)
    y = torch.empty((R, c.H), dtype=torch.bfloat16, device=dev)
    # median of per-launch event timings (MFMA-bound: no cache flush)
    t1 = timed_median(lambda: ops.grouped_gemm_fp8(xq, xs, w1p, w1s, off, out=c1), steps, warmup)
    t2 = timed_median(lambda: ops.grouped_gemm_fp8(hq, hs, w2p, w2s, off, out=y), steps, warmup)
    # the plain kernel (smoe_grouped_gemm_fp8 on [E, N, K] weights, the C-ABI
    # drop-in, which every shape can use)
    t1u = timed_median(lambda: ops.grouped_gemm_fp8(xq, xs, w1q, w1s, off, out=c1), steps, warmup)
    t2u = timed_median(lambda: ops.grouped_gemm_fp8(hq, hs, w2q, w2s, off, out=y), steps, warmup)
    # fc1 with SwiGLU + requant fused into the epilogue (the inference path),
    # against fc1 followed by the stand-alone SwiGLU kernel
    t_sw = timed_median(lambda: ops.swiglu_quant(c1), steps, warmup)
    t1s = timed_median(lambda: ops.grouped_gemm_fp8_swiglu(xq, xs, w1p, w1s, off), steps, warmup)
    fl1 = 2.0 * R * (2 * c.I) * c.H
    fl2 = 2.0 * R * c.H * c.I
    tf = (fl1 + fl2) / ((t1 + t2) * 1e-3) / 1e12
    # the E8M0 recipe: the same shapes with power-of-two scales, on the
    # kernel that applies them in the MFMA (smoe_grouped_gemm_fp8_packed_e8m0)
    del w1p, w2p
    xq, xs = ops.permute_quant_rows(W.tokens(R, c.H, device=dev), inv, 1, scale="pow2")
    hq, hs = ops.permute_quant_rows(W.tokens(R, c.I, device=dev, seed=17), inv, 1, scale="pow2")
    w1q, w1s = ops.quantize_weight_blockwise(W.weights(c.E, 2 * c.I, c.H, device=dev), scale="pow2")
    w2q, w2s = ops.quantize_weight_blockwise(W.weights(c.E, c.H, c.I, device=dev, seed=13),
                                             scale="pow2")
    w1p, w2p = ops.pack_weight_fp8(w1q), ops.pack_weight_fp8(w2q)
    t1e = timed_median(lambda: ops.grouped_gemm_fp8(xq, xs, w1p, w1s, off, out=c1, e8m0=True),
                       steps, warmup)
    t2e = timed_median(lambda: ops.grouped_gemm_fp8(hq, hs, w2p, w2s, off, out=y, e8m0=True),
                       steps, warmup)
    t1se = timed_median(lambda: ops.grouped_gemm_fp8_swiglu(xq, xs, w1p, w1s, off, scale="pow2"),
                        steps, warmup)
    t_swe = timed_median(lambda: ops.swiglu_quant(c1, scale="pow2"), steps, warmup)
    tfe = (fl1 + fl2) / ((t1e + t2e) * 1e-3) / 1e12
    tfu = (fl1 + fl2) / ((t1u + t2u) * 1e-3) / 1e12
    out = {"workload": "dsv3 local experts R=65536 H=7168 I=2048 E=32 zipf1.2",
           "weights": "packed (smoe_grouped_gemm_fp8_packed)",
           "fc1_ms": round(t1, 4), "fc1_tflops": round(fl1 / (t1 * 1e-3) / 1e12, 1),
           "fc2_ms": round(t2, 4), "fc2_tflops": round(fl2 / (t2 * 1e-3) / 1e12, 1),
           "fc1_swiglu_fused_ms": round(t1s, 4), "fc1_then_swiglu_ms": round(t1 + t_sw, 4),
           "tflops": round(tf, 1), "roofline_frac": round(tf / FP8_PEAK_TFLOPS, 4),
           "plain_fc1_ms": round(t1u, 4), "plain_fc2_ms": round(t2u, 4),
           "plain_tflops": round(tfu, 1), "plain_roofline_frac": round(tfu / FP8_PEAK_TFLOPS, 4),
           "e8m0_fc1_ms": round(t1e, 4), "e8m0_fc2_ms": round(t2e, 4),
           "e8m0_fc1_swiglu_fused_ms": round(t1se, 4),
           "e8m0_fc1_then_swiglu_ms": round(t1e + t_swe, 4),
           "e8m0_tflops": round(tfe, 1), "e8m0_roofline_frac": round(tfe / FP8_PEAK_TFLOPS, 4),
           "e8m0_note": "power-of-two 1x128 / 128x128 scales (recipe e8m0), "
                        "smoe_grouped_gemm_fp8_packed_e8m0",
           "peak_tflops": FP8_PEAK_TFLOPS}
    if not skip_cpu:
        out["cpu_baseline"] = cpu_gemm_baseline(xq, xs, w1q, w1s, c)
    del xq, xs, hq, hs, w1q, w1s, w2q, w2s, w1p, w2p, c1, y
    torch.cuda.empty_cache()
    return out


def bench_combine(dev, c, steps, warmup):
    import torch
    from smoe import ops
    R = c.T * c.K
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    y = torch.randn((R, c.H), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    inv = torch.randperm(R, generator=g, device=dev).to(torch.int32)
    w = torch.rand((c.T, c.K), generator=g, device=dev)
    out = torch.empty((c.T, c.H), dtype=torch.bfloat16, device=dev)
    fn = lambda: ops.unpermute_combine(y, inv, w, out=out)
    tf = timed_cold(fn, max(20, steps), warmup)
    t = timed(fn, steps, warmup)
    nb = R * c.H * 2 + R * 8 + c.T * c.H * 2
    del y, out
    torch.cuda.empty_cache()
    return {"ms": round(tf, 4), "gbs": round(nb / (tf * 1e-3) / 1e9, 1),
            "roofline_frac": round(nb / (tf * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "timing": "median of >= 20 launches, each after a 1 GiB cache flush",
            "ms_warm_back_to_back": round(t, 4),
            "gbs_warm_back_to_back": round(nb / (t * 1e-3) / 1e9, 1)}


def bench_layer(dev, steps, warmup):
    import torch
    import smoe
    from smoe import workloads as W
    c = W.CONFIGS["mixtral"]
    m = smoe.SimpleMoE(c.H, c.I, c.E, c.K, device=dev)
    with torch.no_grad():
        m.w1.copy_(W.weights(c.E, 2 * c.I, c.H, device=dev))
        m.w2.copy_(W.weights(c.E, c.H, c.I, device=dev, seed=13))
    m.refresh_fp8_cache()
    x, lg = W.tokens(c.T, c.H, device=dev), W.logits(c.T, c.E, device=dev)
    # a whole layer is ~10 launches from Python: back-to-back calls measure
    # its throughput with the host enqueueing ahead of the GPU.  Without
    # autograd the layer runs fc1 with the fused SwiGLU epilogue; with it,
    # the forward also keeps what the backward needs (c1, bf16 h).
    with torch.no_grad():
        t = timed(lambda: m(x, lg), steps, warmup)
    t_train = timed(lambda: m(x, lg), steps, warmup)
    # the same layer with power-of-two scales everywhere (recipe "e8m0":
    # its packed GEMMs apply the scales in the MFMA)
    m.recipe = "e8m0"
    m.refresh_fp8_cache()
    with torch.no_grad():
        te = timed(lambda: m(x, lg), steps, warmup)
    fl = 2.0 * c.T * c.K * (2 * c.I) * c.H + 2.0 * c.T * c.K * c.H * c.I
    del m
    torch.cuda.empty_cache()
    return {"workload": "mixtral layer fwd T=8192 H=4096 I=14336 E=8 top2",
            "ms": round(t, 4), "tflops": round(fl / (t * 1e-3) / 1e12, 1),
            "ms_with_autograd": round(t_train, 4),
            "tflops_with_autograd": round(fl / (t_train * 1e-3) / 1e12, 1),
            "ms_e8m0_recipe": round(te, 4), "tflops_e8m0_recipe": round(fl / (te * 1e-3) / 1e12, 1)}


def bench_fwd_bwd(dev, steps, warmup):
    """Benchmark config 5 (Qwen3-30B-A3B-shaped expert layer, T=16384, H=2048,
    I=768, E=128, top-8): one forward with saved intermediates plus the full
    fp8 backward (dgrad + wgrad for fc1 and fc2), 3.71e12 FLOP per step;
    median of ``steps`` event-timed steps (warm caches), so one slow step
    (the chip's clock moves under its power limit) does not move it."""
    import torch
    import smoe
    from smoe import workloads as W
    c = W.CONFIGS["qwen3"]
    m = smoe.SimpleMoE(c.H, c.I, c.E, c.K, device=dev)
    with torch.no_grad():
        m.w1.copy_(W.weights(c.E, 2 * c.I, c.H, device=dev))
        m.w2.copy_(W.weights(c.E, c.H, c.I, device=dev, seed=13))
    m.refresh_fp8_cache()
    x, lg = W.tokens(c.T, c.H, device=dev), W.logits(c.T, c.E, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    dout = (torch.randn((c.T, c.H), generator=g, device=dev) * 1e-3).to(torch.bfloat16)

    def step():
        _, st = m(x, lg, return_intermediates=True)
        m.backward_from(st, dout)

    t = timed_median(step, steps, warmup)
    # The same step captured once in a HIP graph and replayed: the host's
    # per-launch work (Python, argument checks, allocator) leaves the step,
    # which removes the idle gaps between the short launches at its start.
    # Capture as the graph tests do: a warm-up on a side stream first.
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    tg = timed_median(graph.replay, steps, warmup)
    del graph
    R = c.T * c.K
    fwd = 2.0 * R * (2 * c.I) * c.H + 2.0 * R * c.H * c.I
    tf = lambda ms: round(3 * fwd / (ms * 1e-3) / 1e12, 1)
    out = {"workload": "qwen3 layer fwd+bwd T=16384 H=2048 I=768 E=128 top8",
           "ms": round(t, 4), "tflops": tf(t), "ms_graph": round(tg, 4), "tflops_graph": tf(tg)}
    # The training path a framework runs: loss.backward() through the
    # autograd node (x a leaf that needs its gradient, as a layer input
    # does), with the parameters' gradients reset each step.  Without
    # main_grad the bf16 parameters receive bf16 weight gradients written by
    # the wgrad kernel; with fp32 main_grad buffers (Megatron's gradient
    # accumulation) the wgrad kernel adds into them.  The last figure is the
    # same accumulation done the unfused way: fp32 gradients, then add_.
    xg = x.detach().clone().requires_grad_(True)

    def train_step():
        m.zero_grad(set_to_none=True)
        xg.grad = None
        m(xg, lg).backward(dout)

    ta = timed_median(train_step, steps, warmup)
    m.w1.main_grad = torch.zeros(m.w1.shape, dtype=torch.float32, device=dev)
    m.w2.main_grad = torch.zeros(m.w2.shape, dtype=torch.float32, device=dev)
    tm = timed_median(train_step, steps, warmup)

    def unfused_step():
        xg.grad = None
        _, st = m(xg.detach(), lg, return_intermediates=True)
        g = m.backward_from(st, dout)
        m.w1.main_grad.add_(g["dw1"])
        m.w2.main_grad.add_(g["dw2"])

    tu = timed_median(unfused_step, steps, warmup)
    del m.w1.main_grad, m.w2.main_grad
    # the opt-in E8M0 weight-gradient recipe on the same step, then the
    # whole step with power-of-two scales (recipe "e8m0")
    m.wgrad_recipe = "e8m0"
    te = timed_median(step, steps, warmup)
    m.recipe = "e8m0"
    m.refresh_fp8_cache()
    tr = timed_median(step, steps, warmup)
    del m
    torch.cuda.empty_cache()
    out.update({"ms_autograd": round(ta, 4), "tflops_autograd": tf(ta),
                "ms_autograd_main_grad": round(tm, 4), "tflops_autograd_main_grad": tf(tm),
                "ms_main_grad_unfused_add": round(tu, 4),
                "ms_e8m0_wgrad": round(te, 4), "tflops_e8m0_wgrad": tf(te),
                "ms_e8m0_recipe": round(tr, 4), "tflops_e8m0_recipe": tf(tr),
                "autograd_note": "loss.backward() through SimpleMoE, grads reset per step; "
                                 "main_grad = fp32 buffers accumulated in the wgrad epilogue; "
                                 "unfused = fp32 dW then main_grad.add_"})
    return out


def bench_fwd_bwd_one_stream(dev, steps, warmup, recipe="blockwise"):
    """The config-5 step of ``bench_fwd_bwd`` (forward with saved
    intermediates + ``backward_from``) with the weight-gradient stream
    replaced by the caller's stream: every kernel runs alone, which gives
    their isolated durations in a kernel trace, and the step time shows what
    the second stream's overlap is worth."""
    import torch
    import smoe
    from smoe import workloads as W
    c = W.CONFIGS["qwen3"]
    m = smoe.SimpleMoE(c.H, c.I, c.E, c.K, device=dev, recipe=recipe)
    with torch.no_grad():
        m.w1.copy_(W.weights(c.E, 2 * c.I, c.H, device=dev))
        m.w2.copy_(W.weights(c.E, c.H, c.I, device=dev, seed=13))
    m.refresh_fp8_cache()
    x, lg = W.tokens(c.T, c.H, device=dev), W.logits(c.T, c.E, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    dout = (torch.randn((c.T, c.H), generator=g, device=dev) * 1e-3).to(torch.bfloat16)

    def step():
        _, st = m(x, lg, return_intermediates=True)
        m.backward_from(st, dout)

    t2 = timed_median(step, steps, warmup)
    m._side_stream = lambda device: torch.cuda.current_stream()
    t1 = timed_median(step, steps, warmup)
    del m
    torch.cuda.empty_cache()
    return {"workload": "qwen3 layer fwd+bwd T=16384 H=2048 I=768 E=128 top8", "recipe": recipe,
            "ms_two_streams": round(t2, 4), "ms_one_stream": round(t1, 4)}


def bench_ceiling(dev, c, iters=20):
    """The HBM's rate for the dispatch step's traffic mix without the
    quantisation: smoe_bw_probe reads the config-2 input (T rows of H bf16)
    with permute_quant's access pattern and writes half its bytes to
    ``fanout`` scattered rows (fanout 8 = the permute's 1:4 read:write byte
    mix), each launch after a cache flush; fanout 0 only reads."""
    import torch
    import smoe
    row_bytes = c.H * 2
    src = torch.ones(c.T * row_bytes // 4, dtype=torch.int32, device=dev)
    dst = torch.empty(c.T * 8 * row_bytes // 2, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    flush = Flush()
    out = {"bytes_in": c.T * row_bytes, "pattern": "permute_quant's (a row split over 2 waves, each part "
           "loaded whole, then written front to back into each scattered destination row)"}
    for fanout in (0, 2, 4, 8):
        fn = lambda: smoe._C.probe_call("smoe_bw_probe", src.data_ptr(), c.T, row_bytes, fanout,
                                        dst.data_ptr(), dst.numel(), sink.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream)
        ms = timed_median(fn, iters, 3, flush)
        nb = c.T * row_bytes * (2 + fanout) // 2
        out[f"read2_write{fanout}"] = {"ms": round(ms, 4), "gbs": round(nb / (ms * 1e-3) / 1e9, 1),
                                       "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    del src, dst, flush
    torch.cuda.empty_cache()
    return out


def bench_blaslt(dev, iters=20):
    """hipBLASLt's fp8 GEMM (torch._scaled_mm, one tensor-wide scale per
    operand, dense) at the config-4 fc1 and fc2 shapes with all 65536 rows in
    one GEMM: the vendor library's rate without block scales or expert
    grouping, a practical reference for the grouped kernel's MFMA ceiling."""
    import torch
    c = __import__("smoe").workloads.CONFIGS["dsv3"]
    out = {}
    one = torch.ones((), device=dev)
    for name, (M, N, K) in (("fc1", (c.T, 2 * c.I, c.H)), ("fc2", (c.T, c.H, c.I))):
        a = torch.randn(M, K, device=dev).to(torch.float8_e4m3fn)
        b = torch.randn(N, K, device=dev).to(torch.float8_e4m3fn).t()
        fn = lambda: torch._scaled_mm(a, b, scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
        ms = timed_median(fn, iters, 5)
        out[name] = {"M": M, "N": N, "K": K, "ms": round(ms, 4),
                     "tflops": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)}
        del a, b
    torch.cuda.empty_cache()
    return out


def run_only(args, dev, c):
    """One kernel family, for profiler runs: permute = the dispatch step
    (route sort + permute_quant) back to back, gemm = DSv3 fc1 + fc2,
    combine = config-2 sized combine, copy = a plain 1 GiB device copy
    (calibrates the FETCH_SIZE / WRITE_SIZE counters against known traffic),
    ceiling = the HBM traffic-mix probe, blaslt = hipBLASLt's dense fp8 GEMM
    at the config-4 shapes, router = the fused router + sort at config 2,
    wgrad = the config-5 fc1 weight gradient, fwdbwd = the config-5 layer
    forward + backward, fwdbwd1 = the same with the weight gradients on the
    caller's stream (every kernel alone; --recipe picks its scale recipe), layer = the config-3 (Mixtral)
    layer forward."""
    import torch
    from smoe import ops, workloads as W
    if args.only == "copy":
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        ms = timed(lambda: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"only": "copy", "bytes_read": 1 << 30, "bytes_written": 1 << 30, "ms": ms}))
    elif args.only == "permute":
        x = W.tokens(c.T, c.H, device=dev, outliers=True)
        idx, _ = ops.router_topk(W.logits(c.T, c.E, device=dev), c.K, W.router_bias(c.E, device=dev))
        ms = timed(lambda: ops.permute_quant(x, idx, c.E), args.steps, args.warmup)
        print(json.dumps({"only": "permute", "ms": ms,
                          "gbs": dispatch_bytes(c.T, c.H, c.E, c.K) / (ms * 1e-3) / 1e9}))
    elif args.only == "wgrad":
        print(json.dumps({"only": "wgrad", **bench_wgrad(dev, max(20, args.steps), args.warmup)}))
    elif args.only == "bwdparts":
        print(json.dumps({"only": "bwdparts", **bench_backward_parts(dev, args.steps, args.warmup)}))
    elif args.only == "refshapes":
        print(json.dumps({"only": "refshapes", **bench_reference_shapes(dev, args.steps, args.warmup)}))
    elif args.only == "router":
        print(json.dumps({"only": "router", **bench_router(dev, c, args.steps, args.warmup)}))
    elif args.only == "fwdbwd":
        print(json.dumps({"only": "fwdbwd", **bench_fwd_bwd(dev, args.steps, args.warmup)}))
    elif args.only == "fwdbwd1":
        print(json.dumps({"only": "fwdbwd1", **bench_fwd_bwd_one_stream(dev, args.steps, args.warmup,
                                                                         args.recipe)}))
    elif args.only == "layer":
        print(json.dumps({"only": "layer", **bench_layer(dev, args.steps, args.warmup)}))
    elif args.only == "gemm":
        print(json.dumps({"only": "gemm", **bench_gemm(dev, args.steps, args.warmup)}))
    elif args.only == "ceiling":
        print(json.dumps({"only": "ceiling", **bench_ceiling(dev, c, max(20, args.steps))}))
    elif args.only == "blaslt":
        print(json.dumps({"only": "blaslt", **bench_blaslt(dev, max(20, args.steps))}))
    else:
        print(json.dumps({"only": "combine", **bench_combine(dev, c, args.steps, args.warmup)}))


def bench_wgrad(dev, steps, warmup):
    """The fc1 weight-gradient GEMM at the config-5 shape (R=131072 routed
    rows, N=2I=1536, K=H=2048, E=128) with near-uniform loads (the config's
    router) and with Zipf(1.2) loads over the 128 experts (4 empty): the
    tile order balances work over the 8 XCDs in both.  Median of per-launch
    event timings."""
    import torch
    from smoe import ops, workloads as W
    c = W.CONFIGS["qwen3"]
    R, N, K = c.T * c.K, 2 * c.I, c.H
    dc1 = W.tokens(R, N, device=dev, seed=21)
    xs = W.tokens(R, K, device=dev, seed=22)
    out = {}
    idx, _ = ops.router_topk(W.logits(c.T, c.E, device=dev), c.K)
    _, _, cnt_r, _ = ops.route_sort(idx, c.E)
    for name, counts in (("router", cnt_r.cpu().tolist()),
                         ("zipf1.2", W.zipf_counts(R=R, E=c.E, zeros=4))):
        off = W.offsets_from_counts(counts, dev)
        aq, as_, pad, ld = ops.quant_cols(dc1, off)
        bq, bs_, _, _ = ops.quant_cols(xs, off)
        dW = torch.empty((c.E, N, K), dtype=torch.float32, device=dev)
        ms = timed_median(lambda: ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld, out=dW),
                          steps, warmup)
        tfl = lambda t: round(2.0 * R * N * K / (t * 1e-3) / 1e12, 1)
        out[name] = {"ms": round(ms, 4), "tflops": tfl(ms),
                     "max_expert_share": round(max(counts) / R, 3)}
        # the E8M0 recipe: power-of-two operand scales applied by the MFMA
        aq, as_, pad, ld = ops.quant_cols(dc1, off, col_scale="pow2")
        bq, bs_, _, _ = ops.quant_cols(xs, off, col_scale="pow2")
        me = timed_median(lambda: ops.grouped_gemm_fp8_wgrad(aq, as_, bq, bs_, pad, ld, out=dW,
                                                             e8m0=True), steps, warmup)
        out[name].update({"e8m0_ms": round(me, 4), "e8m0_tflops": tfl(me)})
        del aq, bq, dW
    torch.cuda.empty_cache()
    return out


def bench_router(dev, c, steps, warmup):
    """The fused router + expert sort at config 2 (T=16384, E=256, top-8,
    with bias): three launches, median of per-call event timings after a
    cache flush.  Algorithmic bytes: logits T*E*4 + bias E*4 read, ids and
    weights T*K*8, row_map/inv_map R*8 and offsets/counts written (the
    router launch alone: T*E*4 + T*K*8)."""
    from smoe import ops, workloads as W
    lg = W.logits(c.T, c.E, device=dev)
    b = W.router_bias(c.E, device=dev)
    flush = Flush()
    ms = timed_median(lambda: ops.route_topk_sort(lg, c.K, b), max(20, steps), warmup, flush)
    ms_r = timed_median(lambda: ops.router_topk(lg, c.K, b), max(20, steps), warmup, flush)
    R = c.T * c.K
    nb = c.T * c.E * 4 + c.E * 4 + R * 8 + R * 8 + (2 * c.E + 1) * 4
    nr = c.T * c.E * 4 + R * 8
    return {"route_topk_sort_ms": round(ms, 4), "route_topk_sort_gbs": round(nb / (ms * 1e-3) / 1e9, 1),
            "router_topk_ms": round(ms_r, 4), "router_topk_gbs": round(nr / (ms_r * 1e-3) / 1e9, 1)}


def bench_reference_shapes(dev, steps, warmup):
    """This build's kernels at the shapes where the reference's notes report
    MI355X numbers for external code (reported beside them, not a target):
    - the fp8 grouped GEMM at E=32, K=7168, N=2048, M=8192 rows
      (summary/fp8_expert_gemm_optimization.md:149-155: fused Triton with
      one per-tensor scale, FWD GEMM 0.310 ms, dA GEMM 0.372 ms, quant + FWD
      0.524 ms).  Here with 1x128 / 128x128 block scales, 256 rows per
      expert, packed weights, warm-cache medians as the notes' GEMM timings
      are; dA is the dgrad GEMM (dY [8192, 2048] times the transposed
      weights [32, 7168, 2048]), quant + FWD adds the 1x128 row quantisation
      of bf16 activations;
    - the expert-sorted dispatch of T tokens, top-8, H=7168
      (notes/2026-04/2026-04-10_monolithmoe_layout_c_pack_optimization.md:
      158-163: sort + bf16 scatter, 0.458 ms at T=4096 and 1.533 ms at
      T=16384).  Here sort + permute with the fp8 quantisation (fewer bytes
      written, the quantisation's work added), cold caches."""
    import torch
    from smoe import ops, workloads as W
    E, M, K, N = 32, 8192, 7168, 2048
    off = W.offsets_from_counts([M // E] * E, dev)
    x = W.tokens(M, K, device=dev)
    xq, xs = ops.quant_rows(x)
    wq, ws = ops.quantize_weight_blockwise(W.weights(E, N, K, device=dev))
    wp = ops.pack_weight_fp8(wq)
    wtq, wts = ops.transpose_blockwise(wq, ws)
    wtp = ops.pack_weight_fp8(wtq)
    dy = W.tokens(M, N, device=dev, seed=21)
    dyq, dys = ops.quant_rows(dy)
    c = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    t_fwd = timed_median(lambda: ops.grouped_gemm_fp8(xq, xs, wp, ws, off, out=c), steps, warmup)
    t_da = timed_median(lambda: ops.grouped_gemm_fp8(dyq, dys, wtp, wts, off, out=dx), steps, warmup)

    def full_fwd():
        q, s = ops.quant_rows(x)
        ops.grouped_gemm_fp8(q, s, wp, ws, off, out=c)

    t_full = timed_median(full_fwd, steps, warmup)
    # the same GEMMs with power-of-two scales on the E8M0 kernel
    xq2, xs2 = ops.quant_rows(x, scale="pow2")
    wq2, ws2 = ops.quantize_weight_blockwise(W.weights(E, N, K, device=dev), scale="pow2")
    wp2 = ops.pack_weight_fp8(wq2)
    wtq2, wts2 = ops.transpose_blockwise(wq2, ws2)
    wtp2 = ops.pack_weight_fp8(wtq2)
    dyq2, dys2 = ops.quant_rows(dy, scale="pow2")
    t_fwd_e = timed_median(lambda: ops.grouped_gemm_fp8(xq2, xs2, wp2, ws2, off, out=c, e8m0=True),
                           steps, warmup)
    t_da_e = timed_median(lambda: ops.grouped_gemm_fp8(dyq2, dys2, wtp2, wts2, off, out=dx,
                                                       e8m0=True), steps, warmup)
    del xq2, xs2, wq2, ws2, wp2, wtq2, wts2, wtp2, dyq2, dys2
    fl = 2.0 * M * N * K
    out = {"gemm_E32_M8192_K7168_N2048": {
        "fwd_ms": round(t_fwd, 4), "fwd_tflops": round(fl / (t_fwd * 1e-3) / 1e12, 1),
        "reference_fwd_ms": 0.310,
        "dA_ms": round(t_da, 4), "dA_tflops": round(fl / (t_da * 1e-3) / 1e12, 1),
        "reference_dA_ms": 0.372,
        "quant_fwd_ms": round(t_full, 4), "reference_quant_fwd_ms": 0.524,
        "e8m0_fwd_ms": round(t_fwd_e, 4), "e8m0_fwd_tflops": round(fl / (t_fwd_e * 1e-3) / 1e12, 1),
        "e8m0_dA_ms": round(t_da_e, 4), "e8m0_dA_tflops": round(fl / (t_da_e * 1e-3) / 1e12, 1),
        "scales": "1x128 activations, 128x128 weights (reference: one per-tensor scale each)"}}
    del x, xq, xs, wq, ws, wp, wtq, wts, wtp, dy, dyq, dys, c, dx
    torch.cuda.empty_cache()
    flush = Flush()
    H, Ek, Kk = 7168, 256, 8
    for T, ref in ((4096, 0.458), (16384, 1.533)):
        xt = W.tokens(T, H, device=dev)
        idx = ops.router_topk(W.logits(T, Ek, device=dev), Kk)[0]
        ms = timed_median(lambda: ops.permute_quant(xt, idx, Ek), max(20, steps), warmup, flush)
        out[f"dispatch_T{T}_top8_H7168"] = {"ms": round(ms, 4), "reference_sort_scatter_ms": ref,
                                            "gbs": round(dispatch_bytes(T, H, Ek, Kk) / (ms * 1e-3) / 1e9, 1)}
        del xt, idx
    del flush
    torch.cuda.empty_cache()
    out["fp8_blockwise_fwd_bwd_E32_M4096_H2880"] = _grouped_fc_fwd_bwd(dev, 2880, steps, warmup)
    e = _grouped_fc_fwd_bwd(dev, 2880, steps, warmup, e8m0=True)
    out["fp8_e8m0_fwd_bwd_E32_M4096_H2880"] = {k: e[k] for k in ("fc1_ms", "fc2_ms", "sum_ms",
                                                                 "tflops")}
    return out


def _grouped_fc_fwd_bwd(dev, hid, steps, warmup, e8m0=False):
    """fc1 and fc2 of the GPT-OSS expert shape (32 experts x 4096 rows, fc1
    N = 2I K = H, fc2 N = H K = I, H = I = ``hid``) forward and backward with
    1x128 / 128x1 / 128x128 block scales, each as its autograd function runs
    it: row quantisation of the input and the forward GEMM; both
    quantisations of the output gradient and the dgrad GEMM on the
    transposed weights; column quantisation of the input and the wgrad GEMM
    (fp32 dW).  Weights are quantised, transposed and packed (where the
    packed kernel covers the shape) once outside the timed steps, as a weight
    cache does.  The reference's number for this sequence
    (notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:62-85)
    is at H = I = 2880, 22.5 groups of 128: the fp8 operands are quantised as
    zero-padded to 2944 (the short last group's scale from its 64 valid
    values), so fc1 runs K = 2944 and fc2 N = 2880 with a partial last tile.
    The FLOP count is the reference's, at 2880.  ``e8m0``: every
    quantisation takes power-of-two scales (the opt-in E8M0 recipe); the
    wgrad GEMM and the packed GEMMs (where K is a multiple of 512, not the
    case at 2880) then apply them in the MFMA."""
    import torch
    from smoe import ops, workloads as W
    E, M = 32, 4096
    R = E * M
    off = W.offsets_from_counts([M] * E, dev)
    cs = "pow2" if e8m0 else "fp32"
    rs = "pow2" if e8m0 else "amax"
    res = {}
    for name, N, Kd in (("fc1", 2 * hid, hid), ("fc2", hid, hid)):
        a = W.tokens(R, Kd, device=dev, seed=31)
        dyv = (W.tokens(R, N, device=dev, seed=32).float() * 1e-2).to(torch.bfloat16)
        wq, ws = ops.quantize_weight_blockwise(W.weights(E, N, Kd, device=dev), scale=rs)
        wtq, wts = ops.transpose_blockwise(wq, ws, k=Kd)
        ok = ops.packed_e8m0_ok if e8m0 else ops.packed_gemm_ok
        wf = ops.pack_weight_fp8(wq) if ok(N, wq.shape[2]) else wq
        wtf = ops.pack_weight_fp8(wtq) if ok(Kd, wtq.shape[2]) else wtq
        y = torch.empty((R, N), dtype=torch.bfloat16, device=dev)
        da = torch.empty((R, Kd), dtype=torch.bfloat16, device=dev)
        dw = torch.empty((E, N, Kd), dtype=torch.float32, device=dev)

        def fwd_bwd():
            aq, as_ = ops.quant_rows(a, scale=rs)
            ops.grouped_gemm_fp8(aq, as_, wf, ws, off, out=y, e8m0=e8m0)
            dq, ds, dTq, dTs, pad, ld = ops.quant_rows_cols(dyv, off, col_scale=cs, row_scale=rs)
            ops.grouped_gemm_fp8(dq, ds, wtf, wts, off, out=da, e8m0=e8m0)
            aTq, aTs, _, _ = ops.quant_cols(a, off, col_scale=cs)
            ops.grouped_gemm_fp8_wgrad(dTq, dTs, aTq, aTs, pad, ld, out=dw, e8m0=e8m0)

        res[name + "_ms"] = round(timed_median(fwd_bwd, steps, warmup), 4)
        res[name + "_kernels"] = "packed" if isinstance(wf, ops.PackedWeight) else "plain"
        del a, dyv, wq, ws, wtq, wts, wf, wtf, y, da, dw
        torch.cuda.empty_cache()
    ms = res["fc1_ms"] + res["fc2_ms"]
    flop = 6.0 * R * (2 * hid * hid + hid * hid)
    res.update({"sum_ms": round(ms, 4), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                "reference_H2880": {"fp8_blockwise_triton_sum_ms": 27.42, "tflops": 700,
                                    "fp8_tensorwise_triton_sum_ms": 13.47, "tensorwise_tflops": 1430}})
    return res


def bench_backward_parts(dev, steps, warmup):
    """The config-5 layer's HBM-bound forward and backward kernels one at a
    time (inputs from one forward with saved intermediates), median of
    per-call event timings warm and after the 1 GiB flush, with each call's
    unique algorithmic bytes.  The gathered column quantisers read every
    token row K times through row_map (T*H*2 unique bytes, R*H*2 requested)."""
    import torch
    import smoe
    from smoe import ops, workloads as W
    c = W.CONFIGS["qwen3"]
    m = smoe.SimpleMoE(c.H, c.I, c.E, c.K, device=dev)
    with torch.no_grad():
        m.w1.copy_(W.weights(c.E, 2 * c.I, c.H, device=dev))
        m.w2.copy_(W.weights(c.E, c.H, c.I, device=dev, seed=13))
    m.refresh_fp8_cache()
    x, lg = W.tokens(c.T, c.H, device=dev), W.logits(c.T, c.E, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    dout = (torch.randn((c.T, c.H), generator=g, device=dev) * 1e-3).to(torch.bfloat16)
    with torch.no_grad():
        _, st = m(x, lg, return_intermediates=True)
    off, inv, rm, K = st["offsets"], st["inv_map"], st["row_map"], c.K
    R, H, I, T = c.T * c.K, c.H, c.I, c.T
    dh = (torch.randn((R, I), generator=g, device=dev) * 1e-3).to(torch.bfloat16)
    dxs = torch.randn((R, H), generator=g, device=dev).to(torch.bfloat16)
    ones = torch.ones_like(st["topk_w"])
    parts = {
        "swiglu_quant_save_h": (lambda: ops.swiglu_quant(st["c1"], save_h=True),
                                R * 2 * I * 2 + R * I + R * (I // 128) * 4 + R * I * 2),
        "quant_cols_h": (lambda: ops.quant_cols(st["h"], off), R * I * 2 + R * I),
        "quant_cols_x_gathered": (lambda: ops.quant_cols(st["x"], off, gather=rm, gather_div=K),
                                  T * H * 2 + R * H),
        "combine_bwd_quant": (lambda: ops.unpermute_combine_bwd_quant(dout, st["y"], inv, rm,
                                                                      st["topk_w"], off),
                              T * H * 2 + R * H * 2 + 2 * R * H + R * 4),
        "swiglu_bwd_quant": (lambda: ops.swiglu_bwd_quant(st["c1"], dh, off),
                             R * 2 * I * 2 + R * I * 2 + 2 * R * 2 * I),
        "combine_dx": (lambda: ops.unpermute_combine(dxs, inv, ones), R * H * 2 + T * H * 2),
    }
    flush = Flush()
    out = {"workload": "qwen3 layer T=16384 H=2048 I=768 E=128 top8"}
    for name, (fn, nb) in parts.items():
        warm = timed_median(fn, steps, warmup)
        cold = timed_median(fn, steps, warmup, flush)
        out[name] = {"unique_bytes": nb, "warm_us": round(warm * 1e3, 1),
                     "warm_gbs": round(nb / (warm * 1e-3) / 1e9, 1),
                     "cold_us": round(cold * 1e3, 1), "cold_gbs": round(nb / (cold * 1e-3) / 1e9, 1)}
    del m, st, flush
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip-extra", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--recipe", choices=["blockwise", "e8m0"], default="blockwise",
                    help="scale recipe of the --only fwdbwd1 layer step")
    ap.add_argument("--only", choices=["permute", "gemm", "combine", "copy", "fwdbwd", "ceiling",
                                       "blaslt", "router", "wgrad", "layer", "refshapes",
                                       "bwdparts", "fwdbwd1"],
                    help="run one kernel family only (for rocprofv3 runs) and print its timing")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has expert-parallel degree 1 "
              "and no collectives, so --gpus must be 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import smoe
    from smoe import ops, workloads as W
    smoe._C.lib()  # fail loudly when the HIP library is missing
    dev = torch.device("cuda:0")
    c = W.CONFIGS["permute"]
    if args.only:
        return run_only(args, dev, c)

    x = W.tokens(c.T, c.H, device=dev, outliers=True)
    idx, _ = ops.router_topk(W.logits(c.T, c.E, device=dev), c.K, W.router_bias(c.E, device=dev))
    R = c.T * c.K
    row_map = torch.empty(R, dtype=torch.int32, device=dev)
    inv_map = torch.empty(R, dtype=torch.int32, device=dev)
    counts = torch.empty(c.E, dtype=torch.int32, device=dev)
    offsets = torch.empty(c.E + 1, dtype=torch.int32, device=dev)
    xq = torch.empty((R, c.H), dtype=torch.uint8, device=dev)
    xs = torch.empty((R, c.H // 128), dtype=torch.float32, device=dev)
    lib = smoe._C.lib()
    ws_n = int(lib.smoe_route_sort_workspace_size(c.T, c.K, c.E))
    ws = torch.empty(max(ws_n, 16), dtype=torch.uint8, device=dev)

    def step():
        smoe._C.call("smoe_dispatch_quant", x.data_ptr(), idx.data_ptr(), c.T, c.H, c.K, c.E,
                     row_map.data_ptr(), inv_map.data_ptr(), counts.data_ptr(),
                     offsets.data_ptr(), xq.data_ptr(), xs.data_ptr(), ws.data_ptr(), ws.numel(),
                     torch.cuda.current_stream().cuda_stream)

    def permute_only():
        smoe._C.call("smoe_permute_quant", x.data_ptr(), inv_map.data_ptr(), c.T, c.H, c.K,
                     xq.data_ptr(), xs.data_ptr(), torch.cuda.current_stream().cuda_stream)

    # The timed steps: W warm-ups, then exactly K steps, each bracketed by
    # HIP events after a synchronise and a 1 GiB cache flush (x is not in
    # L2 or the last-level cache when a step starts); ms_per_step is their
    # median.  Every permute_quant launch of this run is a flushed one, so a
    # profiler's average over the run is the cold figure too.
    flush = Flush()
    ms = timed_median(step, args.steps, args.warmup, flush)
    nbytes = dispatch_bytes(c.T, c.H, c.E, c.K)
    value = nbytes / (ms * 1e-3) / 1e9
    log(f"dispatch step {ms:.4f} ms  {value:.1f} GB/s (median of {args.steps}, flushed)")

    pk_ms = timed_median(permute_only, max(20, args.steps), args.warmup, flush)
    del flush
    pk_bytes = permute_kernel_bytes(c.T, c.H, c.K)
    pk_gbs = pk_bytes / (pk_ms * 1e-3) / 1e9
    log(f"permute_quant kernel {pk_ms:.4f} ms  {pk_gbs:.1f} GB/s (median, flushed)")
    roof = {"kernel": "smoe::permute_quant_row_kernel<4, 2, false>", "bound": "hbm", "achieved": round(pk_gbs, 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(pk_gbs / HBM_PEAK_GBS, 4),
            "traffic": PERMUTE_TRAFFIC_BYTES, "kernel_ms": round(pk_ms, 4),
            "bytes_per_launch": pk_bytes,
            "timing": "median of >= 20 launches, each after a 1 GiB cache flush"}
    del x, xq, xs
    torch.cuda.empty_cache()

    extra = {}
    if not args.skip_extra:
        sx = max(20, args.steps)
        extra["hbm_ceiling_dispatch_mix"] = bench_ceiling(dev, c)
        log("ceiling", extra["hbm_ceiling_dispatch_mix"])
        extra["router_cfg2"] = bench_router(dev, c, sx, 3)
        log("router", extra["router_cfg2"])
        extra["grouped_gemm_fp8"] = bench_gemm(dev, sx, 3, skip_cpu=args.skip_cpu)
        log("gemm", extra["grouped_gemm_fp8"])
        extra["reference_shapes"] = bench_reference_shapes(dev, sx, 3)
        log("reference shapes", extra["reference_shapes"])
        extra["combine_cfg2"] = bench_combine(dev, c, sx, 3)
        log("combine", extra["combine_cfg2"])
        extra["layer_mixtral"] = bench_layer(dev, 10, 3)
        log("layer", extra["layer_mixtral"])
        extra["wgrad_cfg5_fc1"] = bench_wgrad(dev, sx, 3)
        log("wgrad", extra["wgrad_cfg5_fc1"])
        extra["layer_qwen3_fwd_bwd"] = bench_fwd_bwd(dev, 20, 3)
        log("fwd+bwd", extra["layer_qwen3_fwd_bwd"])

    cpu = None if args.skip_cpu else cpu_baseline(c)
    line = {"metric": "fp8 grouped-GEMM TFLOPS & permute-quant GB/s, % of MI355X roofline, 1 GPU",
            "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp8-e4m3 (bf16 in, fp32 scales)",
            "data": "synthetic (seeded N(0,1) bf16 tokens with 0.1% x50 outliers, N(0,1) logits + N(0,0.5) bias)",
            "config": {"workload": "permute+quantize cfg2: route_sort + permute_quant",
                       "T": c.T, "H": c.H, "E": c.E, "top_k": c.K, "parallelism": "ep1",
                       "timing": "median of K steps, each after a 1 GiB cache flush"},
            "roofline": roof, "cpu_baseline": cpu, "extra": extra}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
