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


class SimpleMoE(nn.Module):
    """Dropless top-k MoE FFN with SwiGLU experts in blockwise fp8.

    Parameters follow the notes' naming: ``w1`` [E, 2I, H] holds the gate
    rows [0, I) and up rows [I, 2I) of fc1 in [N, K] layout; ``w2`` [E, H, I]
    is fc2.  ``w_gate`` [H, E] is the router's gating linear.
    Weights are quantised to fp8 with 128x128 block scales on first use and
    cached (``refresh_fp8_cache`` re-quantises after an update).
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

    @torch.no_grad()
    def reset_parameters(self, generator: torch.Generator | None = None, std: float = 0.02):
        for p in (self.w_gate, self.w1, self.w2):
            p.copy_(torch.randn(p.shape, generator=generator, dtype=torch.float32,
                                device=generator.device if generator is not None else p.device).to(p) * std)
        self._fp8 = None

    @torch.no_grad()
    def refresh_fp8_cache(self):
        w1q, w1s = ops.quantize_weight_blockwise(self.w1.detach().contiguous())
        w2q, w2s = ops.quantize_weight_blockwise(self.w2.detach().contiguous())
        self._fp8 = (w1q, w1s, w2q, w2s)
        return self._fp8

    def fp8_weights(self):
        return self._fp8 if self._fp8 is not None else self.refresh_fp8_cache()

    @torch.no_grad()
    def forward(self, x: torch.Tensor, logits: torch.Tensor | None = None,
                return_intermediates: bool = False):
        """x [T, H] bf16 -> y [T, H] bf16.  ``logits`` [T, E] f32 may be given
        directly (the benchmark configs specify router logits); otherwise
        they are x @ w_gate in fp32."""
        if logits is None:
            logits = x.float() @ self.w_gate
        w1q, w1s, w2q, w2s = self.fp8_weights()
        idx, w = ops.router_topk(logits.contiguous(), self.top_k, self.router_bias)
        xq, xs, row_map, inv_map, counts, offsets = ops.permute_quant(x, idx, self.num_experts)
        if return_intermediates:
            # the backward pass needs c1 and bf16 h, so fc1 and SwiGLU run
            # as two kernels here
            c1 = ops.grouped_gemm_fp8(xq, xs, w1q, w1s, offsets)
            hq, hs, h = ops.swiglu_quant(c1, save_h=True)
        else:
            # inference: SwiGLU + requantisation run in the fc1 epilogue
            hq, hs = ops.grouped_gemm_fp8_swiglu(xq, xs, w1q, w1s, offsets)
        y = ops.grouped_gemm_fp8(hq, hs, w2q, w2s, offsets)
        out = ops.unpermute_combine(y, inv_map, w)
        if return_intermediates:
            return out, dict(x=x, topk_idx=idx, topk_w=w, row_map=row_map, inv_map=inv_map,
                             counts=counts, offsets=offsets, xq=xq, xs=xs, c1=c1, hq=hq,
                             hs=hs, h=h, y=y)
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
        Returns dx [T,H] bf16, dw1 [E,2I,H] f32, dw2 [E,H,I] f32 and the
        router-weight gradient dtopk_w [T,K] f32 (plus dy's 1x128 quantisation dyq,
        dys and the intermediates dh, dxs).  Every stage is a HIP kernel;
        nothing synchronises with the host."""
        w1q, w1s, w2q, w2s = self.fp8_weights()
        if getattr(self, "_fp8_t", None) is None or self._fp8_t[0] is not w1q:
            self._fp8_t = (w1q,) + ops.transpose_blockwise(w1q, w1s) + ops.transpose_blockwise(w2q, w2s)
        _, w1tq, w1ts, w2tq, w2ts = self._fp8_t
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
        main.wait_stream(side)
        return dict(dx=dx, dw1=dw1, dw2=dw2, dtopk_w=dw, dyq=dyq, dys=dys, dh=dh, dxs=dxs)

    def _side_stream(self, device) -> torch.cuda.Stream:
        s = getattr(self, "_side", None)
        if s is None or s.device != device:
            s = torch.cuda.Stream(device=device)  # default priority
            self._side = s
        return s

