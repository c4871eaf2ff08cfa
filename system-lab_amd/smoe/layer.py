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


# Optimizer steps seen in this process.  Megatron-style optimizers write the
# stepped weights back through ``param.data.copy_()``, which does not advance
# a parameter's version counter; every torch optimizer step (Megatron's inner
# fp32 optimizer included) bumps this count instead, and the fp8 weight cache
# is keyed on it as well as on the parameters' storage and versions.
_OPT_STEPS = [0]
_OPT_HOOK = []


def _count_optimizer_step(optimizer, args, kwargs):
    _OPT_STEPS[0] += 1


def _install_optimizer_hook():
    if not _OPT_HOOK:
        from torch.optim.optimizer import register_optimizer_step_post_hook
        _OPT_HOOK.append(register_optimizer_step_post_hook(_count_optimizer_step))


class _SimpleMoEFunction(torch.autograd.Function):
    """Autograd node of one SimpleMoE forward.  The forward keeps the
    intermediates the fp8 backward needs as saved tensors, so autograd frees
    them after a backward (a second backward needs ``retain_graph=True``, as
    for any node, and otherwise raises PyTorch's own error) and checks that
    none was modified in place.  It also keeps the fp8 weights the forward
    used, so the dgrad runs on their transposes even if the weights are
    re-quantised before the backward.  The backward is
    ``SimpleMoE.backward_from`` (every stage a HIP kernel) plus the router
    backward into the logits.  The gating linear that produces the logits
    (x @ w_gate) sits outside this node, so autograd carries dlogits on into
    x and w_gate.  A parameter with a ``main_grad`` fp32 buffer (Megatron's
    gradient-accumulation convention) has its weight gradient added into it
    by the wgrad kernel itself (no separate fp32 gradient or add pass);
    otherwise the gradient is returned in the parameter's dtype."""

    @staticmethod
    def forward(ctx, x, logits, w1, w2, module):
        out, inter = module._forward_impl(x, logits, save=True)
        ctx.module = module
        ctx.keys = [k for k, v in inter.items() if isinstance(v, torch.Tensor)]
        ctx.extra = {k: v for k, v in inter.items() if not isinstance(v, torch.Tensor)}
        ctx.save_for_backward(*[inter[k] for k in ctx.keys])
        ctx.dtypes = (x.dtype, w1.dtype, w2.dtype)
        ctx.main_grads = (getattr(w1, "main_grad", None), getattr(w2, "main_grad", None))
        return out

    @staticmethod
    def backward(ctx, dout):
        inter = dict(zip(ctx.keys, ctx.saved_tensors))
        inter.update(ctx.extra)
        mg1, mg2 = ctx.main_grads
        # a weight gradient in the parameters' own dtype where that is bf16
        # (rounded once from the fp32 sums, as .to() would), else fp32
        wdt = torch.bfloat16 if ctx.dtypes[1] == ctx.dtypes[2] == torch.bfloat16 else torch.float32
        g = ctx.module.backward_from(inter, dout.to(torch.bfloat16).contiguous(),
                                     dw1_into=mg1, dw2_into=mg2, wgrad_dtype=wdt)
        grads = []
        for dw, mg, dt in zip((g["dw1"], g["dw2"]), ctx.main_grads, ctx.dtypes[1:]):
            grads.append(None if mg is not None else dw.to(dt))
        return g["dx"].to(ctx.dtypes[0]), g["dlogits"], grads[0], grads[1], None


class SimpleMoE(nn.Module):
    """Dropless top-k MoE FFN with SwiGLU experts in blockwise fp8.

    Parameters follow the notes' naming: ``w1`` [E, 2I, H] holds the gate
    rows [0, I) and up rows [I, 2I) of fc1 in [N, K] layout; ``w2`` [E, H, I]
    is fc2.  ``w_gate`` [H, E] is the router's gating linear.
    Weights are quantised to fp8 with 128x128 block scales on first use.
    The cache is keyed on the parameters' storage and version counters and
    on the number of torch optimizer steps taken in the process, so an
    in-place update (``p.copy_``, an optimizer step, or an optimizer that
    writes back through ``p.data`` after its inner step) re-quantises on the
    next call.  A write through ``p.data`` outside any optimizer step is
    invisible to both: call ``refresh_fp8_cache()`` after one.  Where a
    GEMM's K is a multiple of 512 the weights are cached packed in MFMA
    fragment order for the register-loaded kernel (``ops.pack_weight_fp8``;
    the same result, see ``ops.grouped_gemm_fp8``).  Footprint of the cache:
    the plain fp8 w1, w2 (E*(2I*H + H*I) bytes, the source of the dgrad
    transposes), their packed copies where packed, and the dgrad transposes
    once a backward ran (packed where covered, else plain; never both), plus
    the fp32 scales.

    ``wgrad_recipe`` chooses the 128x1 quantisation of the weight-gradient
    operands: "fp32" (the default) uses the activation rule s = amax/448;
    "e8m0" uses power-of-two scales (the least power of two >= amax/448, the
    scale format of the MXFP8 recipe) so that gfx950's scaled MFMA applies
    them in hardware and the wgrad does no per-output scale arithmetic.  The
    forward and the dgrad are the same in both.

    ``recipe`` chooses the scale rule of every quantisation: "blockwise" (the
    default: amax/448 for 1x128 activation and gradient rows and 128x128
    weight blocks) or "e8m0", which gives all of them, and the wgrad
    operands' 128x1 columns, power-of-two scales (E8M0 values, the MXFP8
    scale format at the blockwise granularity).  Its GEMMs then apply the
    scales in the scaled MFMA: the packed-weight GEMMs run
    ``smoe_grouped_gemm_fp8_packed_e8m0`` and the wgrad its E8M0 mode.

    Under autograd (grad mode on and an input or parameter requiring grad),
    ``forward`` records one graph node whose backward runs the fp8 backward
    (``loss.backward()`` fills w1.grad, w2.grad, w_gate.grad and x.grad).
    Without autograd it is the inference path: SwiGLU and its requantisation
    run in the fc1 epilogue and nothing is saved.
    """

    def __init__(self, hidden: int, intermediate: int, num_experts: int, top_k: int,
                 device=None, dtype=torch.bfloat16, router_bias: bool = False,
                 wgrad_recipe: str = "fp32", recipe: str = "blockwise"):
        super().__init__()
        if wgrad_recipe not in ("fp32", "e8m0"):
            raise ValueError("wgrad_recipe is 'fp32' (128x1 scales amax/448) or 'e8m0' "
                             "(power-of-two 128x1 scales applied by the scaled MFMA)")
        if recipe not in ("blockwise", "e8m0"):
            raise ValueError("recipe is 'blockwise' (scales amax/448) or 'e8m0' "
                             "(power-of-two scales for every quantisation)")
        self.wgrad_recipe = wgrad_recipe
        self.recipe = recipe
        self.hidden, self.intermediate = hidden, intermediate
        self.num_experts, self.top_k = num_experts, top_k
        kw = dict(device=device, dtype=dtype)
        self.w_gate = nn.Parameter(torch.empty(hidden, num_experts, device=device, dtype=torch.float32))
        self.w1 = nn.Parameter(torch.empty(num_experts, 2 * intermediate, hidden, **kw))
        self.w2 = nn.Parameter(torch.empty(num_experts, hidden, intermediate, **kw))
        self.register_buffer("router_bias", torch.zeros(num_experts, device=device) if router_bias else None)
        self._fp8 = None
        self._fp8_key = None
        self._gemm = None
        self._gemm_t = None
        _install_optimizer_hook()

    @torch.no_grad()
    def reset_parameters(self, generator: torch.Generator | None = None, std: float = 0.02):
        for p in (self.w_gate, self.w1, self.w2):
            p.copy_(torch.randn(p.shape, generator=generator, dtype=torch.float32,
                                device=generator.device if generator is not None else p.device).to(p) * std)

    @property
    def _pow2(self) -> bool:
        """Every quantisation takes power-of-two scales (recipe "e8m0")."""
        return self.recipe == "e8m0"

    @property
    def _row_scale(self) -> str:
        return "pow2" if self._pow2 else "amax"

    def _weights_key(self):
        return (_OPT_STEPS[0], self.recipe) + tuple((p.data_ptr(), p._version, tuple(p.shape))
                                        for p in (self.w1, self.w2))

    @torch.no_grad()
    def refresh_fp8_cache(self):
        rs = self._row_scale
        w1q, w1s = ops.quantize_weight_blockwise(self.w1.detach().to(torch.bfloat16).contiguous(), rs)
        w2q, w2s = ops.quantize_weight_blockwise(self.w2.detach().to(torch.bfloat16).contiguous(), rs)
        self._fp8 = (w1q, w1s, w2q, w2s)
        self._fp8_key = self._weights_key()
        self._gemm = (self._for_gemm(w1q), w1s, self._for_gemm(w2q), w2s)
        self._gemm_t = None
        return self._fp8

    def _for_gemm(self, wq):
        """The form the GEMM ops take: packed in MFMA fragment order where the
        register-loaded kernel covers the shape (K a multiple of 512, or for
        the E8M0 recipe of 128 from 512 up; the same bytes out, faster), else
        the plain [E, N, K] weights."""
        E, N, Kd = wq.shape
        ok = ops.packed_e8m0_ok if self._pow2 else ops.packed_gemm_ok
        return ops.pack_weight_fp8(wq) if ok(N, Kd) else wq

    def fp8_weights(self):
        """(w1q, w1s, w2q, w2s), re-quantised when w1 or w2 changed since the
        cache was filled (storage moved or version counter advanced)."""
        if self._fp8 is None or self._fp8_key != self._weights_key():
            self.refresh_fp8_cache()
        return self._fp8

    def fp8_weights_t(self):
        """The dgrad weights: (w1q^T, w1s^T, w2q^T, w2s^T) of the current fp8
        weights, computed on each call (the backward caches them in GEMM form,
        ``gemm_weights_t``)."""
        return self._transposed(self.fp8_weights())

    def _transposed(self, fp8):
        w1q, w1s, w2q, w2s = fp8
        return (ops.transpose_blockwise(w1q, w1s, k=self.hidden)
                + ops.transpose_blockwise(w2q, w2s, k=self.intermediate))

    def gemm_weights(self):
        """(w1, w1s, w2, w2s) as the forward GEMMs take them: fp8_weights()
        with w1 / w2 packed where the packed kernel covers their shape."""
        self.fp8_weights()
        return self._gemm

    def gemm_weights_t(self, fp8=None):
        """The dgrad weights in the form the GEMM ops take (packed where
        covered).  Those of the current fp8 weights are cached with them;
        ``fp8`` names other fp8 weights (a forward's, since re-quantised),
        whose transposes are computed and not cached."""
        cur = self.fp8_weights()
        if fp8 is not None and fp8 is not cur:
            w1tq, w1ts, w2tq, w2ts = self._transposed(fp8)
            return (self._for_gemm(w1tq), w1ts, self._for_gemm(w2tq), w2ts)
        if self._gemm_t is None:
            w1tq, w1ts, w2tq, w2ts = self._transposed(cur)
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
        fp8 = self.fp8_weights()
        w1q, w1s, w2q, w2s = self._gemm
        # router and expert sort in three launches (the sort's histogram is
        # counted inside the router launch)
        idx, w, row_map, inv_map, counts, offsets = ops.route_topk_sort(logits, self.top_k,
                                                                        self.router_bias)
        rs, e8 = self._row_scale, self._pow2
        xq, xs = ops.permute_quant_rows(x, inv_map, self.top_k, scale=rs)
        if save:
            # the backward pass needs c1 and bf16 h, so fc1 and SwiGLU run
            # as two kernels here
            c1 = ops.grouped_gemm_fp8(xq, xs, w1q, w1s, offsets, e8m0=e8)
            hq, hs, h = ops.swiglu_quant(c1, save_h=True, scale=rs)
        else:
            # inference: SwiGLU + requantisation run in the fc1 epilogue
            hq, hs = ops.grouped_gemm_fp8_swiglu(xq, xs, w1q, w1s, offsets, scale=rs)
        y = ops.grouped_gemm_fp8(hq, hs, w2q, w2s, offsets, e8m0=e8)
        out = ops.unpermute_combine(y, inv_map, w)
        if save:
            return out, dict(x=x, logits=logits, topk_idx=idx, topk_w=w, row_map=row_map,
                             inv_map=inv_map, counts=counts, offsets=offsets, xq=xq, xs=xs,
                             c1=c1, hq=hq, hs=hs, h=h, y=y, fp8=fp8)
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
                     xq=torch.empty((0, ops.pad128(H)), dtype=ops.FP8, device=dev),
                     xs=torch.empty((0, ops.nblocks(H)), dtype=torch.float32, device=dev),
                     c1=torch.empty((0, 2 * I), dtype=torch.bfloat16, device=dev),
                     hq=torch.empty((0, ops.pad128(I)), dtype=ops.FP8, device=dev),
                     hs=torch.empty((0, ops.nblocks(I)), dtype=torch.float32, device=dev),
                     h=torch.empty((0, I), dtype=torch.bfloat16, device=dev),
                     y=torch.empty((0, H), dtype=torch.bfloat16, device=dev))
        return out, inter

    def _empty_backward(self, inter: dict, wgrad_dtype=torch.float32) -> dict:
        """Gradients of an empty batch: empty dx / dlogits / dtopk_w and zero
        weight gradients, with the keys ``backward_from`` returns."""
        dev, H, I = inter["x"].device, self.hidden, self.intermediate
        E, K = self.num_experts, self.top_k
        f32 = dict(dtype=torch.float32, device=dev)
        wg = dict(dtype=wgrad_dtype, device=dev)
        out = dict(dx=torch.empty((0, H), dtype=torch.bfloat16, device=dev),
                   dw1=torch.zeros((E, 2 * I, H), **wg), dw2=torch.zeros((E, H, I), **wg),
                   dtopk_w=torch.empty((0, K), **f32), dlogits=torch.empty((0, E), **f32),
                   dyq=torch.empty((0, ops.pad128(H)), dtype=ops.FP8, device=dev),
                   dys=torch.empty((0, ops.nblocks(H)), **f32),
                   dh=torch.empty((0, I), dtype=torch.bfloat16, device=dev),
                   dxs=torch.empty((0, H), dtype=torch.bfloat16, device=dev))
        if inter.get("logits_from_gate"):
            out["dw_gate"] = torch.zeros((H, E), **f32)
        return out

    @torch.no_grad()
    def backward_from(self, inter: dict, dout: torch.Tensor, dw1_into: torch.Tensor | None = None,
                      dw2_into: torch.Tensor | None = None,
                      wgrad_dtype: torch.dtype = torch.float32) -> dict:
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
        fp32 matmuls are library GEMMs.  Nothing synchronises with the host.

        ``dw1_into`` / ``dw2_into`` (fp32 or bf16 [E,2I,H] / [E,H,I]) are
        gradient-accumulation buffers: the wgrad kernel adds the weight
        gradient into them in its epilogue and they are returned as dw1 /
        dw2.  Otherwise dw1 / dw2 are new tensors of ``wgrad_dtype`` (fp32 or
        bf16, rounded once from the fp32 sums).  The dgrad uses the
        transposes of the fp8 weights the forward ran with."""
        E, H, I = self.num_experts, self.hidden, self.intermediate
        for buf, shape, name in ((dw1_into, (E, 2 * I, H), "dw1_into"), (dw2_into, (E, H, I), "dw2_into")):
            if buf is not None and (tuple(buf.shape) != shape or buf.dtype not in (torch.float32, torch.bfloat16)
                                    or not buf.is_contiguous() or buf.device != dout.device):
                raise ValueError(f"{name} must be a contiguous fp32 or bf16 {list(shape)} tensor on {dout.device}")
        if inter["x"].shape[0] == 0:
            out = self._empty_backward(inter, wgrad_dtype)
            if dw1_into is not None:
                out["dw1"] = dw1_into
            if dw2_into is not None:
                out["dw2"] = dw2_into
            return out
        w1tq, w1ts, w2tq, w2ts = self.gemm_weights_t(inter.get("fp8"))
        off, inv = inter["offsets"], inter["inv_map"]
        K = self.top_k
        # The weight gradients are off the dx critical path.  They run on a
        # second stream (default priority), so that a wgrad tile writing its
        # fp32 output shares the chip with dgrad tiles that are MFMA-bound.
        # Every side-stream segment starts by waiting for the main stream, and
        # the main stream waits for the side stream before returning.
        main = torch.cuda.current_stream()
        side = self._side_stream(main.device)
        e8m0 = self.wgrad_recipe == "e8m0" or self._pow2
        cs = "pow2" if e8m0 else "fp32"
        rs, e8 = self._row_scale, self._pow2
        ones = torch.ones_like(inter["topk_w"])
        # the returned weight gradients are allocated on the caller's stream,
        # so the caching allocator never hands their memory to side-stream
        # work while the caller still uses them
        dw1 = dw1_into if dw1_into is not None else torch.empty((E, 2 * I, H), dtype=wgrad_dtype,
                                                                device=dout.device)
        dw2 = dw2_into if dw2_into is not None else torch.empty((E, H, I), dtype=wgrad_dtype,
                                                                device=dout.device)
        dout = dout.contiguous()
        side.wait_stream(main)
        with torch.cuda.stream(side):
            # the wgrad activation operands depend on the forward only: h, and
            # the sorted tokens x[row_map // K] gathered inside the quantiser
            hTq, hTs, _, _ = ops.quant_cols(inter["h"], off, col_scale=cs)
            xTq, xTs, _, _ = ops.quant_cols(inter["x"], off, gather=inter["row_map"], gather_div=K,
                                            col_scale=cs)
        # combine backward fused with dy's 1x128 row quantisation for the
        # dgrad; the 128x1 columns for the wgrad (rebuilt from dout, not from
        # the row pass) on the side stream; dy itself is never stored
        with torch.cuda.stream(side):
            dyTq, dyTs, pad, ld = ops.combine_bwd_quant_cols(dout, inter["row_map"],
                                                             inter["topk_w"], off, col_scale=cs)
            ops.grouped_gemm_fp8_wgrad(dyTq, dyTs, hTq, hTs, pad, ld, out=dw2,
                                       accumulate=dw2_into is not None, e8m0=e8m0)
        dyq, dys, _, _, _, _, dw = ops.unpermute_combine_bwd_quant(
            dout, inter["y"], inv, inter["row_map"], inter["topk_w"], off, col_scale=cs,
            row_scale=rs, cols=False)
        dh = ops.grouped_gemm_fp8(dyq, dys, w2tq, w2ts, off, e8m0=e8)
        # SwiGLU backward fused with both quantisations of dc1 (dc1 itself is
        # never stored)
        dcq, dcs, dcTq, dcTs, _, _ = ops.swiglu_bwd_quant(inter["c1"], dh, off, col_scale=cs,
                                                          row_scale=rs)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            ops.grouped_gemm_fp8_wgrad(dcTq, dcTs, xTq, xTs, pad, ld, out=dw1,
                                       accumulate=dw1_into is not None, e8m0=e8m0)
        dxs = ops.grouped_gemm_fp8(dcq, dcs, w1tq, w1ts, off, e8m0=e8)
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

