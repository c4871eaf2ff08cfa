"""SimpleMoE: the expert layer forward built from the smoe ops.

    Route -> Dispatch (permute + 1x128 quant) -> grouped fc1 -> SwiGLU+requant
          -> grouped fc2 -> weighted combine
(moe/MoE_detailed_computation_dataflow.md:295-317; Megatron MoELayer stages,
moe/MegatronCore_MoE_reading_notes.md:84-116).  EP degree 1: every expert is
local, so dispatch is a local permute and there is no all-to-all.  The whole
forward is stream-ordered with no host synchronisation.
"""
from __future__ import annotations

import torch
from torch import nn

from . import ops


class _SimpleMoEFunction(torch.autograd.Function):
    """Autograd node of one SimpleMoE forward.  The forward keeps the
    intermediates the fp8 backward needs; the backward is
    ``SimpleMoE.backward_from`` (every stage a HIP kernel) plus the router
    backward into the logits.  The gating linear that produces the logits
    (x @ w_gate) sits outside this node, so autograd carries dlogits on into
    x and w_gate.  Weight gradients are computed in fp32; a parameter with a
    ``main_grad`` fp32 buffer (Megatron's gradient-accumulation convention)
    has them accumulated there, otherwise they are returned in the
    parameter's dtype."""

    @staticmethod
    def forward(ctx, x, logits, w1, w2, module):
        out, inter = module._forward_impl(x, logits, save=True)
        ctx.module = module
        ctx.inter = inter
        ctx.dtypes = (x.dtype, w1.dtype, w2.dtype)
        ctx.main_grads = (getattr(w1, "main_grad", None), getattr(w2, "main_grad", None))
        return out

    @staticmethod
    def backward(ctx, dout):
        g = ctx.module.backward_from(ctx.inter, dout.to(torch.bfloat16).contiguous())
        ctx.inter = None
        grads = []
        for dw, mg, dt in zip((g["dw1"], g["dw2"]), ctx.main_grads, ctx.dtypes[1:]):
            if mg is not None:
                mg.add_(dw)
                grads.append(None)
            else:
                grads.append(dw.to(dt))
        return g["dx"].to(ctx.dtypes[0]), g["dlogits"], grads[0], grads[1], None


class SimpleMoE(nn.Module):
    """Dropless top-k MoE FFN with SwiGLU experts in blockwise fp8.

    Parameters follow the notes' naming: ``w1`` [E, 2I, H] holds the gate
    rows [0, I) and up rows [I, 2I) of fc1 in [N, K] layout; ``w2`` [E, H, I]
    is fc2.  ``w_gate`` [H, E] is the router's gating linear.
    Weights are quantised to fp8 with 128x128 block scales on first use; the
    cache is keyed on the parameters' storage and version counters, so an
    in-place update (an optimizer step) re-quantises on the next call.  Where
    a GEMM's K is a multiple of 512 its weights are also cached packed in MFMA
    fragment order for the register-loaded kernel (``ops.pack_weight_fp8``;
    the same result, see ``ops.grouped_gemm_fp8``), which adds the packed
    copy's E*N*K bytes.

    Under autograd (grad mode on and an input or parameter requiring grad),
    ``forward`` records one graph node whose backward runs the fp8 backward
    (``loss.backward()`` fills w1.grad, w2.grad, w_gate.grad and x.grad).
    Without autograd it is the inference path: SwiGLU and its requantisation
    run in the fc1 epilogue and nothing is saved.
    """

    def __init__(self, hidden: int, intermediate: int, num_experts: int, top_k: int,
                 device=None, dtype=torch.bfloat16, router_bias: bool = False):
        super().__init__()
        self.hidden, self.intermediate = hidden, intermediate
        self.num_experts, self.top_k = num_experts, top_k
        kw = dict(device=device, dtype=dtype)
        self.w_gate = nn.Parameter(torch.empty(hidden, num_experts, device=device, dtype=torch.float32))
        self.w1 = nn.Parameter(torch.empty(num_experts, 2 * intermediate, hidden, **kw))
        self.w2 = nn.Parameter(torch.empty(num_experts, hidden, intermediate, **kw))
        self.register_buffer("router_bias", torch.zeros(num_experts, device=device) if router_bias else None)
        self._fp8 = None
        self._fp8_key = None
        self._fp8_t = None
        self._gemm = None
        self._gemm_t = None

    @torch.no_grad()
    def reset_parameters(self, generator: torch.Generator | None = None, std: float = 0.02):
        for p in (self.w_gate, self.w1, self.w2):
            p.copy_(torch.randn(p.shape, generator=generator, dtype=torch.float32,
                                device=generator.device if generator is not None else p.device).to(p) * std)

    def _weights_key(self):
        return tuple((p.data_ptr(), p._version, tuple(p.shape)) for p in (self.w1, self.w2))

    @torch.no_grad()
    def refresh_fp8_cache(self):
        w1q, w1s = ops.quantize_weight_blockwise(self.w1.detach().to(torch.bfloat16).contiguous())
        w2q, w2s = ops.quantize_weight_blockwise(self.w2.detach().to(torch.bfloat16).contiguous())
        self._fp8 = (w1q, w1s, w2q, w2s)
        self._fp8_key = self._weights_key()
        self._fp8_t = None
        self._gemm = (self._for_gemm(w1q), w1s, self._for_gemm(w2q), w2s)
        self._gemm_t = None
        return self._fp8

    @staticmethod
    def _for_gemm(wq):
        """The form the GEMM ops take: packed in MFMA fragment order where the
        register-loaded kernel covers the shape (K a multiple of 512; the same
        bytes out, faster), else the plain [E, N, K] weights."""
        E, N, Kd = wq.shape
        return ops.pack_weight_fp8(wq) if ops.packed_gemm_ok(N, Kd) else wq

    def fp8_weights(self):
        """(w1q, w1s, w2q, w2s), re-quantised when w1 or w2 changed since the
        cache was filled (storage moved or version counter advanced)."""
        if self._fp8 is None or self._fp8_key != self._weights_key():
            self.refresh_fp8_cache()
        return self._fp8

    def fp8_weights_t(self):
        """The dgrad weights: (w1q^T, w1s^T, w2q^T, w2s^T), cached with the
        fp8 weights they come from."""
        w1q, w1s, w2q, w2s = self.fp8_weights()
        if self._fp8_t is None:
            self._fp8_t = ops.transpose_blockwise(w1q, w1s) + ops.transpose_blockwise(w2q, w2s)
        return self._fp8_t

    def gemm_weights(self):
        """(w1, w1s, w2, w2s) as the forward GEMMs take them: fp8_weights()
        with w1 / w2 packed where the packed kernel covers their shape."""
        self.fp8_weights()
        return self._gemm

    def gemm_weights_t(self):
        """The dgrad weights of fp8_weights_t() in the form the GEMM ops take
        (packed where covered), cached with them."""
        w1tq, w1ts, w2tq, w2ts = self.fp8_weights_t()
        if self._gemm_t is None:
            self._gemm_t = (self._for_gemm(w1tq), w1ts, self._for_gemm(w2tq), w2ts)
        return self._gemm_t

    def forward(self, x: torch.Tensor, logits: torch.Tensor | None = None,
                return_intermediates: bool = False):
        """x [T, H] bf16 -> y [T, H] bf16.  ``logits`` [T, E] f32 may be given
        directly (the benchmark configs specify router logits); otherwise
        they are x @ w_gate in fp32.  ``return_intermediates`` returns
        (y, intermediates) for a later ``backward_from`` without recording an
        autograd graph."""
        if return_intermediates:
            with torch.no_grad():
                if logits is None:
                    logits = x.float() @ self.w_gate
                    out, inter = self._forward_impl(x, logits, save=True)
                    inter["logits_from_gate"] = True
                    return out, inter
                return self._forward_impl(x, logits, save=True)
        if logits is None:
            logits = x.float() @ self.w_gate
        params = (x, logits, self.w1, self.w2)
        if torch.is_grad_enabled() and any(t.requires_grad for t in params):
            return _SimpleMoEFunction.apply(x, logits, self.w1, self.w2, self)
        with torch.no_grad():
            return self._forward_impl(x, logits, save=False)

    @torch.no_grad()
    def _forward_impl(self, x: torch.Tensor, logits: torch.Tensor, save: bool):
        x = x.detach().to(torch.bfloat16).contiguous()
        logits = logits.detach().float().contiguous()
        if x.shape[0] == 0:
            return self._empty_forward(x, logits, save)
        w1q, w1s, w2q, w2s = self.gemm_weights()
        # router and expert sort in three launches (the sort's histogram is
        # counted inside the router launch)
        idx, w, row_map, inv_map, counts, offsets = ops.route_topk_sort(logits, self.top_k,
                                                                        self.router_bias)
        xq, xs = ops.permute_quant_rows(x, inv_map, self.top_k)
        if save:
            # the backward pass needs c1 and bf16 h, so fc1 and SwiGLU run
            # as two kernels here
            c1 = ops.grouped_gemm_fp8(xq, xs, w1q, w1s, offsets)
            hq, hs, h = ops.swiglu_quant(c1, save_h=True)
        else:
            # inference: SwiGLU + requantisation run in the fc1 epilogue
            hq, hs = ops.grouped_gemm_fp8_swiglu(xq, xs, w1q, w1s, offsets)
        y = ops.grouped_gemm_fp8(hq, hs, w2q, w2s, offsets)
        out = ops.unpermute_combine(y, inv_map, w)
        if save:
            return out, dict(x=x, logits=logits, topk_idx=idx, topk_w=w, row_map=row_map,
                             inv_map=inv_map, counts=counts, offsets=offsets, xq=xq, xs=xs,
                             c1=c1, hq=hq, hs=hs, h=h, y=y)
        return out

    def _empty_forward(self, x: torch.Tensor, logits: torch.Tensor, save: bool):
        """An empty batch (T = 0): no kernel runs (the C ABI rejects T = 0);
        the outputs and intermediates are empty tensors of the usual shapes,
        with every expert's count 0."""
        dev, H, I = x.device, self.hidden, self.intermediate
        E, K = self.num_experts, self.top_k
        out = torch.empty((0, H), dtype=torch.bfloat16, device=dev)
        if not save:
            return out
        i32 = dict(dtype=torch.int32, device=dev)
        inter = dict(x=x, logits=logits, topk_idx=torch.empty((0, K), **i32),
                     topk_w=torch.empty((0, K), dtype=torch.float32, device=dev),
                     row_map=torch.empty(0, **i32), inv_map=torch.empty(0, **i32),
                     counts=torch.zeros(E, **i32), offsets=torch.zeros(E + 1, **i32),
                     xq=torch.empty((0, H), dtype=ops.FP8, device=dev),
                     xs=torch.empty((0, H // ops.GROUP), dtype=torch.float32, device=dev),
                     c1=torch.empty((0, 2 * I), dtype=torch.bfloat16, device=dev),
                     hq=torch.empty((0, I), dtype=ops.FP8, device=dev),
                     hs=torch.empty((0, I // ops.GROUP), dtype=torch.float32, device=dev),
                     h=torch.empty((0, I), dtype=torch.bfloat16, device=dev),
                     y=torch.empty((0, H), dtype=torch.bfloat16, device=dev))
        return out, inter

    def _empty_backward(self, inter: dict) -> dict:
        """Gradients of an empty batch: empty dx / dlogits / dtopk_w and zero
        weight gradients, with the keys ``backward_from`` returns."""
        dev, H, I = inter["x"].device, self.hidden, self.intermediate
        E, K = self.num_experts, self.top_k
        f32 = dict(dtype=torch.float32, device=dev)
        out = dict(dx=torch.empty((0, H), dtype=torch.bfloat16, device=dev),
                   dw1=torch.zeros((E, 2 * I, H), **f32), dw2=torch.zeros((E, H, I), **f32),
                   dtopk_w=torch.empty((0, K), **f32), dlogits=torch.empty((0, E), **f32),
                   dyq=torch.empty((0, H), dtype=ops.FP8, device=dev),
                   dys=torch.empty((0, H // ops.GROUP), **f32),
                   dh=torch.empty((0, I), dtype=torch.bfloat16, device=dev),
                   dxs=torch.empty((0, H), dtype=torch.bfloat16, device=dev))
        if inter.get("logits_from_gate"):
            out["dw_gate"] = torch.zeros((H, E), **f32)
        return out

    @torch.no_grad()
    def backward_from(self, inter: dict, dout: torch.Tensor) -> dict:
        """Backward of one forward call given its intermediates
        (``forward(..., return_intermediates=True)``) and dout [T,H] bf16.

        combine bwd fused with both quantisations of dy (1x128 rows, 128x1
        columns; dy never stored) ->
        fc2 dgrad (W2^T) and fc2 wgrad (128x1 dy, h) -> SwiGLU bwd fused with
        both quantisations of dc1 -> fc1 dgrad (W1^T) and fc1 wgrad (128x1
        dc1, sorted x) -> sum of the K replicas into dx.
        Returns dx [T,H] bf16, dw1 [E,2I,H] f32, dw2 [E,H,I] f32, the
        router-weight gradient dtopk_w [T,K] f32 and its continuation through
        the renormalisation and softmax, dlogits [T,E] f32 (plus dy's 1x128
        quantisation dyq, dys and the intermediates dh, dxs).  When the
        forward computed the logits itself (x @ w_gate), dx also holds the
        gating linear's contribution and dw_gate [H,E] f32 is returned.
        Every expert stage is a HIP kernel; the gating linear's two small
        fp32 matmuls are library GEMMs.  Nothing synchronises with the host."""
        if inter["x"].shape[0] == 0:
            return self._empty_backward(inter)
        w1tq, w1ts, w2tq, w2ts = self.gemm_weights_t()
        off, inv = inter["offsets"], inter["inv_map"]
        K = self.top_k
        # The weight gradients are off the dx critical path.  They run on a
        # second stream (default priority), so that a wgrad tile writing its
        # fp32 output shares the chip with dgrad tiles that are MFMA-bound.
        # Every side-stream segment starts by waiting for the main stream, and
        # the main stream waits for the side stream before returning.
        main = torch.cuda.current_stream()
        side = self._side_stream(main.device)
        ones = torch.ones_like(inter["topk_w"])
        # the returned weight gradients are allocated on the caller's stream,
        # so the caching allocator never hands their memory to side-stream
        # work while the caller still uses them
        E, H, I = self.num_experts, self.hidden, self.intermediate
        dw1 = torch.empty((E, 2 * I, H), dtype=torch.float32, device=dout.device)
        dw2 = torch.empty((E, H, I), dtype=torch.float32, device=dout.device)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            # the wgrad activation operands depend on the forward only: h, and
            # the sorted tokens x[row_map // K] gathered inside the quantiser
            hTq, hTs, _, _ = ops.quant_cols(inter["h"], off)
            xTq, xTs, _, _ = ops.quant_cols(inter["x"], off, gather=inter["row_map"], gather_div=K)
        # combine backward fused with both quantisations of dy (1x128 rows for
        # dgrad, 128x1 columns for wgrad); dy itself is never stored
        dyq, dys, dyTq, dyTs, pad, ld, dw = ops.unpermute_combine_bwd_quant(
            dout.contiguous(), inter["y"], inv, inter["row_map"], inter["topk_w"], off)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            ops.grouped_gemm_fp8_wgrad(dyTq, dyTs, hTq, hTs, pad, ld, out=dw2)
        dh = ops.grouped_gemm_fp8(dyq, dys, w2tq, w2ts, off)
        # SwiGLU backward fused with both quantisations of dc1 (dc1 itself is
        # never stored)
        dcq, dcs, dcTq, dcTs, _, _ = ops.swiglu_bwd_quant(inter["c1"], dh, off)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            ops.grouped_gemm_fp8_wgrad(dcTq, dcTs, xTq, xTs, pad, ld, out=dw1)
        dxs = ops.grouped_gemm_fp8(dcq, dcs, w1tq, w1ts, off)
        dx = ops.unpermute_combine(dxs, inv, ones)
        # router: renormalisation + softmax backward into the logits
        dlogits = ops.router_topk_bwd(inter["logits"], inter["topk_idx"], dw)
        out = dict(dx=dx, dw1=dw1, dw2=dw2, dtopk_w=dw, dlogits=dlogits, dyq=dyq, dys=dys,
                   dh=dh, dxs=dxs)
        if inter.get("logits_from_gate"):
            # logits = x @ w_gate in fp32: the gating linear's gradients
            x32 = inter["x"].float()
            out["dx"] = (dx.float() + dlogits @ self.w_gate.detach().t()).to(torch.bfloat16)
            out["dw_gate"] = x32.t() @ dlogits
        main.wait_stream(side)
        return out

    def _side_stream(self, device) -> torch.cuda.Stream:
        s = getattr(self, "_side", None)
        if s is None or s.device != device:
            s = torch.cuda.Stream(device=device)  # default priority
            self._side = s
        return s

