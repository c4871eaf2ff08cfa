"""Torch-facing ops of the SimpleMoE expert-layer hot path.

Each op validates its tensors, allocates outputs through torch's caching
allocator, and enqueues HIP kernels from libsmoe.so on the current stream.
No op synchronises with the host: routing counts and offsets stay on the
device.  There is no CPU or PyTorch fallback — a missing library raises.

Call shapes mirror the operators the reference's notes drive on MI355X:
``grouped_gemm_fp8(permuted, w, tokens_per_expert)``
(notes/2026-04/2026-04-21_gptoss_10_moe_fp8_grouped_gemm_diagnosis.md:39),
``Dispatcher.permute`` / ``unpermute`` (moe/MegatronCore_MoE_reading_notes.md:94-116),
with device-side ``offsets`` in place of a host ``tokens_per_expert`` list.
"""
from __future__ import annotations

import torch

from . import _C

FP8 = torch.float8_e4m3fn
GROUP = 128
# column-scale rules of the 128x1 (wgrad operand) quantisers, SMOE_COLSCALE_*
COL_SCALES = {"fp32": 0, "pow2": 1}
# scale rule of the row and weight quantisers (SMOE_SCALE_*): "amax" is
# s = amax/448, "pow2" the least power of two >= amax/448 (E8M0 values)
SCALES = {"amax": 0, "pow2": 1}
ROWSCALE_POW2 = 2  # SMOE_ROWSCALE_POW2: the row-scale bit of the fused quantisers


def pad128(d: int) -> int:
    """The fp8 row pitch of a dimension quantised in 128-wide groups.  A
    dimension that is not a multiple of 128 (it must be a multiple of 16) is
    quantised as if zero-padded to this size: the last group's scale comes
    from its valid elements and the padding bytes are 0."""
    return -(-d // GROUP) * GROUP


def nblocks(d: int) -> int:
    """128-wide groups (or weight blocks) along a dimension of size d."""
    return -(-d // GROUP)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(t: torch.Tensor, name: str, dtypes, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a GPU tensor (got {t.device}); the HIP kernels are the only path")
    if t.device.index != torch.cuda.current_device():
        # kernels launch on the current device's stream with raw pointers
        raise ValueError(f"{name} is on {t.device} but the current device is "
                         f"cuda:{torch.cuda.current_device()}")
    if t.dtype not in dtypes:
        raise TypeError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _scale(scale: str) -> int:
    if scale not in SCALES:
        raise ValueError(f"scale must be one of {sorted(SCALES)}, got {scale!r}")
    return SCALES[scale]


def _bytes(t: torch.Tensor) -> torch.Tensor:
    """fp8 tensors are accepted as float8_e4m3fn or raw uint8."""
    return t if t.dtype == torch.uint8 else t.view(torch.uint8)


# ------------------------------------------------------------------ router
def router_topk(logits: torch.Tensor, top_k: int, bias: torch.Tensor | None = None):
    """softmax(fp32 logits) [+ bias for selection] -> top-k ids (score desc,
    id asc) and renormalised weights.  logits [T,E] f32 -> (idx [T,K] i32,
    w [T,K] f32).  (moe/MoE_detailed_computation_dataflow.md:53-66)"""
    _check(logits, "logits", (torch.float32,), 2)
    T, E = logits.shape
    if bias is not None:
        _check(bias, "bias", (torch.float32,), 1)
        if bias.numel() != E:
            raise ValueError("bias must have E entries")
    idx = torch.empty((T, top_k), dtype=torch.int32, device=logits.device)
    w = torch.empty((T, top_k), dtype=torch.float32, device=logits.device)
    _C.call("smoe_router_topk", _ptr(logits), _ptr(bias), T, E, top_k, _ptr(idx), _ptr(w),
            _stream())
    return idx, w


def router_topk_bwd(logits: torch.Tensor, topk_idx: torch.Tensor, dtopk_w: torch.Tensor):
    """Backward of ``router_topk`` through the renormalisation and the
    softmax: dtopk_w [T,K] f32 -> dlogits [T,E] f32 (the selection bias has
    no gradient; ``topk_idx`` are the forward's picks)."""
    _check(logits, "logits", (torch.float32,), 2)
    _check(topk_idx, "topk_idx", (torch.int32,), 2)
    _check(dtopk_w, "dtopk_w", (torch.float32,), 2)
    T, E = logits.shape
    if topk_idx.shape[0] != T or dtopk_w.shape != topk_idx.shape:
        raise ValueError("topk_idx and dtopk_w must be [T, K] for logits [T, E]")
    K = topk_idx.shape[1]
    dl = torch.empty((T, E), dtype=torch.float32, device=logits.device)
    _C.call("smoe_router_topk_bwd", _ptr(logits), _ptr(topk_idx), _ptr(dtopk_w), T, E, K,
            _ptr(dl), _stream())
    return dl


# -------------------------------------------------------------------- sort
# Byte offset of the routing status word in the sort workspace
# (SMOE_ROUTE_STATUS_OFFSET): the number of pairs whose expert id was
# outside [0, E), rewritten by every sort.
ROUTE_STATUS_OFFSET = 0
_route_status: dict = {}


def _dev_key(device) -> torch.device:
    """A GPU device with its index filled in, so that 'cuda', 'cuda:0' and
    torch.device('cuda', 0) name the same status entry."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    if dev.type != "cuda":
        raise ValueError(f"routing status is kept per GPU, got {dev}")
    return torch.device("cuda", torch.cuda.current_device() if dev.index is None else dev.index)


def _sort_workspace(T: int, K: int, E: int, dev) -> torch.Tensor:
    nbytes = int(_C.lib().smoe_route_sort_workspace_size(T, K, E))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    # the status word of this call; check_route_status() reads it lazily
    _route_status[_dev_key(dev)] = ws[ROUTE_STATUS_OFFSET:ROUTE_STATUS_OFFSET + 4].view(torch.int32)
    return ws


def last_route_status(device=None) -> torch.Tensor:
    """Device int32 [1]: pairs dropped for an out-of-range expert id by the
    most recent sort on ``device`` (0 when every id was valid).  Reading it
    does not synchronise; converting it to a Python int does.  ``device``
    may omit the index ('cuda' is the current GPU)."""
    dev = _dev_key(device)
    if dev not in _route_status:
        raise RuntimeError(f"no routing sort has run on {dev}")
    st = _route_status[dev]
    # the allocation-free sort keeps its status word in library memory:
    # its count is recovered as T*K - offsets[E] (dropped pairs get no row)
    return st() if callable(st) else st


def check_route_status(device=None) -> None:
    """Synchronise and raise if the most recent sort on ``device`` met
    expert ids outside [0, E): those pairs got no row (inv_map = -1) and
    contribute nothing to the combine."""
    n = int(last_route_status(device).item())
    if n:
        raise ValueError(f"routing: {n} (token, slot) pairs had an expert id outside [0, E) "
                         "and were dropped")


def route_sort_noalloc(topk_idx: torch.Tensor, row_map: torch.Tensor, inv_map: torch.Tensor,
                       counts: torch.Tensor, offsets: torch.Tensor) -> None:
    """``route_sort`` into caller-provided outputs through the allocation-free
    entry point (smoe_route_sort_noalloc: the sort's workspace is a static
    array inside the library, so nothing is allocated and the call can be
    captured in a HIP graph).  The routing status of this call is readable
    through ``last_route_status`` / ``check_route_status`` like any sort's.
    Calls that overlap on one GPU share the library's array and race."""
    _check(topk_idx, "topk_idx", (torch.int32,), 2)
    T, K = topk_idx.shape
    R = T * K
    E = counts.numel()
    for t, n, name in ((row_map, R, "row_map"), (inv_map, R, "inv_map"), (counts, E, "counts"),
                       (offsets, E + 1, "offsets")):
        _check(t, name, (torch.int32,), 1)
        if t.numel() != n:
            raise ValueError(f"{name} must have {n} entries")
    _C.call("smoe_route_sort_noalloc", _ptr(topk_idx), T, K, E, _ptr(row_map), _ptr(inv_map),
            _ptr(counts), _ptr(offsets), _stream())
    _route_status[_dev_key(topk_idx.device)] = lambda: (R - offsets[E:]).to(torch.int32)


def route_sort(topk_idx: torch.Tensor, num_experts: int):
    """Stable expert sort of the T*K pairs.  -> (row_map [R], inv_map [R],
    counts [E], offsets [E+1]), all int32 on the device.  Ids outside
    [0, E) get no row (inv_map = -1); ``check_route_status`` reports them."""
    _check(topk_idx, "topk_idx", (torch.int32,), 2)
    T, K = topk_idx.shape
    dev = topk_idx.device
    R = T * K
    row_map = torch.empty(R, dtype=torch.int32, device=dev)
    inv_map = torch.empty(R, dtype=torch.int32, device=dev)
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    ws = _sort_workspace(T, K, num_experts, dev)
    _C.call("smoe_route_sort", _ptr(topk_idx), T, K, num_experts, _ptr(row_map), _ptr(inv_map),
            _ptr(counts), _ptr(offsets), _ptr(ws), ws.numel(), _stream())
    return row_map, inv_map, counts, offsets


def route_topk_sort(logits: torch.Tensor, top_k: int, bias: torch.Tensor | None = None):
    """Router fused with the expert sort (the sort's histogram is counted in
    the router launch): the outputs of ``router_topk`` then ``route_sort``,
    byte for byte.  -> (topk_idx, topk_w, row_map, inv_map, counts, offsets)."""
    _check(logits, "logits", (torch.float32,), 2)
    T, E = logits.shape
    if bias is not None:
        _check(bias, "bias", (torch.float32,), 1)
        if bias.numel() != E:
            raise ValueError("bias must have E entries")
    dev = logits.device
    R = T * top_k
    idx = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    w = torch.empty((T, top_k), dtype=torch.float32, device=dev)
    row_map = torch.empty(R, dtype=torch.int32, device=dev)
    inv_map = torch.empty(R, dtype=torch.int32, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    ws = _sort_workspace(T, top_k, E, dev)
    _C.call("smoe_route_topk_sort", _ptr(logits), _ptr(bias), T, E, top_k, _ptr(idx), _ptr(w),
            _ptr(row_map), _ptr(inv_map), _ptr(counts), _ptr(offsets), _ptr(ws), ws.numel(),
            _stream())
    return idx, w, row_map, inv_map, counts, offsets


# ---------------------------------------------------------------- dispatch
def permute_quant_rows(x: torch.Tensor, inv_map: torch.Tensor, top_k: int, scale: str = "amax"):
    """Quantise each token row of x [T,H] bf16 once (1x128 groups) and write it
    to the rows inv_map[t*K+k].  -> (xq [T*K,pad128(H)] fp8,
    xs [T*K,pad128(H)/128] f32).  H need only be a multiple of 16 (see
    ``pad128``).  ``scale``: "amax" (s = amax/448) or "pow2" (power-of-two
    scales, the E8M0 recipe)."""
    mode = _scale(scale)
    _check(x, "x", (torch.bfloat16,), 2)
    _check(inv_map, "inv_map", (torch.int32,))
    T, H = x.shape
    if inv_map.numel() != T * top_k:
        raise ValueError("inv_map must have T*K entries")
    R = T * top_k
    xq = torch.empty((R, pad128(H)), dtype=FP8, device=x.device)
    xs = torch.empty((R, nblocks(H)), dtype=torch.float32, device=x.device)
    _C.call("smoe_permute_quant_ex", _ptr(x), _ptr(inv_map), T, H, top_k, _ptr(xq), _ptr(xs),
            mode, _stream())
    return xq, xs


def permute_quant(x: torch.Tensor, topk_idx: torch.Tensor, num_experts: int,
                  scale: str = "amax"):
    """Dispatcher.permute fused with 1x128 fp8 quantisation
    (moe/MegatronCore_MoE_reading_notes.md:94-99, 498-501).
    -> (xq, xs, row_map, inv_map, counts, offsets).  ``scale`` as for
    ``permute_quant_rows``."""
    if _scale(scale) != SCALES["amax"]:
        row_map, inv_map, counts, offsets = route_sort(topk_idx, num_experts)
        xq, xs = permute_quant_rows(x, inv_map, topk_idx.shape[1], scale)
        return xq, xs, row_map, inv_map, counts, offsets
    _check(x, "x", (torch.bfloat16,), 2)
    _check(topk_idx, "topk_idx", (torch.int32,), 2)
    T, H = x.shape
    if topk_idx.shape[0] != T:
        raise ValueError("topk_idx must have T rows")
    K = topk_idx.shape[1]
    dev = x.device
    R = T * K
    row_map = torch.empty(R, dtype=torch.int32, device=dev)
    inv_map = torch.empty(R, dtype=torch.int32, device=dev)
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    xq = torch.empty((R, pad128(H)), dtype=FP8, device=dev)
    xs = torch.empty((R, nblocks(H)), dtype=torch.float32, device=dev)
    ws = _sort_workspace(T, K, num_experts, dev)
    _C.call("smoe_dispatch_quant", _ptr(x), _ptr(topk_idx), T, H, K, num_experts,
            _ptr(row_map), _ptr(inv_map), _ptr(counts), _ptr(offsets), _ptr(xq), _ptr(xs),
            _ptr(ws), ws.numel(), _stream())
    return xq, xs, row_map, inv_map, counts, offsets


# ----------------------------------------------------------------- weights
def quantize_weight_blockwise(w: torch.Tensor, scale: str = "amax"):
    """128x128 blockwise fp8 weights.  w [E,N,K] bf16 ("NK" layout,
    summary/fp8_expert_gemm_optimization.md:137) -> (wq [E,N,pad128(K)] fp8,
    ws [E,ceil(N/128),pad128(K)/128] f32).  N and K that are not multiples
    of 128 (multiples of 16) end in partial blocks, quantised as the
    zero-padded block; wq's padding columns are 0.  ``scale`` as for
    ``permute_quant_rows``."""
    mode = _scale(scale)
    _check(w, "w", (torch.bfloat16,), 3)
    E, N, Kd = w.shape
    wq = torch.empty((E, N, pad128(Kd)), dtype=FP8, device=w.device)
    ws = torch.empty((E, nblocks(N), nblocks(Kd)), dtype=torch.float32, device=w.device)
    _C.call("smoe_quantize_weight_blockwise_ex", _ptr(w), E, N, Kd, _ptr(wq), _ptr(ws), mode,
            _stream())
    return wq, ws


# -------------------------------------------------------------------- GEMM
class PackedWeight:
    """fp8 expert weights rearranged in MFMA fragment order for the
    register-loaded grouped GEMM (``pack_weight_fp8``).  ``data`` holds the
    same E*N*K bytes as the [E, N, K] weights, in the packed order; the
    128x128 scales are unchanged and passed alongside as before.  The GEMM ops
    take a PackedWeight wherever they take wq and then run the packed kernel
    (the same output; see grouped_gemm_fp8)."""

    __slots__ = ("data",)

    def __init__(self, data: torch.Tensor):
        self.data = data

    @property
    def shape(self):
        return self.data.shape

    @property
    def device(self):
        return self.data.device


PACKED_MAX_K = 65536  # the packed kernel keeps a tile's weight-scale column in LDS


def packed_gemm_ok(N: int, Kd: int) -> bool:
    """Whether the packed GEMM covers a weight of N rows and K = Kd: it needs
    K a multiple of 512 and at most 65536, and N*K < 2^32 (the same checks
    as smoe_grouped_gemm_fp8_packed; other weights use the plain kernel)."""
    return (Kd % (4 * GROUP) == 0 and 0 < Kd <= PACKED_MAX_K and N % 16 == 0
            and N * Kd < (1 << 32))


def packed_e8m0_ok(N: int, Kd: int) -> bool:
    """Whether the E8M0 GEMM (smoe_grouped_gemm_fp8_packed_e8m0) covers a
    packed weight of N rows and K = Kd: K a multiple of 128 from 512 to
    65536, N % 16 == 0 and N*K < 2^32 (the C entry point's checks)."""
    return (Kd % GROUP == 0 and 4 * GROUP <= Kd <= PACKED_MAX_K and N % 16 == 0
            and N * Kd < (1 << 32))


def pack_weight_fp8(wq: torch.Tensor) -> PackedWeight:
    """[E, N, K] fp8 weights -> PackedWeight (smoe_pack_weight_fp8).  Raises
    unless ``packed_gemm_ok(N, K)`` or ``packed_e8m0_ok(N, K)`` (a weight only
    the E8M0 GEMM covers can only be used with ``e8m0=True``)."""
    _check(wq, "wq", (FP8, torch.uint8), 3)
    E, N, Kd = wq.shape
    if not (packed_gemm_ok(N, Kd) or packed_e8m0_ok(N, Kd)):
        raise ValueError(f"packed weights need K % 128 == 0, 512 <= K <= {PACKED_MAX_K}, "
                         f"N % 16 == 0 and N*K < 2^32 (N={N}, K={Kd})")
    wp = torch.empty((E, N, Kd), dtype=torch.uint8, device=wq.device)
    _C.call("smoe_pack_weight_fp8", _ptr(_bytes(wq)), E, N, Kd, _ptr(wp), _stream())
    return PackedWeight(wp)


def _weight(wq, name):
    """(tensor, packed?) of a GEMM weight argument."""
    if isinstance(wq, PackedWeight):
        _check(wq.data, name, (torch.uint8,), 3)
        return wq.data, True
    _check(wq, name, (FP8, torch.uint8))
    return wq, False


def grouped_gemm_fp8(xq: torch.Tensor, xs: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor,
                     offsets: torch.Tensor, out: torch.Tensor | None = None,
                     e8m0: bool = False) -> torch.Tensor:
    """Dropless fp8 grouped GEMM: rows [offsets[e], offsets[e+1]) of xq times
    W[e]^T with 1x128 / 128x128 scales -> bf16 [R, N].  Rows outside
    [offsets[0], offsets[E]) are not written.  ``wq`` is [E, N, K] fp8, or a
    PackedWeight (``pack_weight_fp8``) for the register-loaded kernel.  That
    kernel orders each 128-wide K block's products differently inside the
    MFMA: the bytes are the same whenever those products sum exactly in fp32
    (every benchmark and layer workload), else they can differ in the last
    bf16 bit, within the GEMM tolerance.  ``e8m0``: every scale is a power
    of two (the "pow2" quantisers); a PackedWeight then runs the kernel that
    applies the scales in the MFMA (smoe_grouped_gemm_fp8_packed_e8m0),
    whose sums can differ from the packed kernel's in the last bf16 bit.
    Plain weights run the plain kernel either way (its arithmetic is exact
    for any scale)."""
    _check(xq, "xq", (FP8, torch.uint8))
    wt, packed = _weight(wq, "wq")
    _check(xs, "xs", (torch.float32,), 2)
    _check(ws, "ws", (torch.float32,), 3)
    _check(offsets, "offsets", (torch.int32,), 1)
    R, Kd = xq.shape
    E, N, Kw = wt.shape
    if Kw != Kd:
        raise ValueError(f"K mismatch: xq has {Kd}, wq has {Kw}")
    if packed and not (packed_e8m0_ok(N, Kd) if e8m0 else packed_gemm_ok(N, Kd)):
        raise ValueError(f"packed weights need K % 512 == 0 (K % 128 == 0 and K >= 512 with "
                         f"e8m0), K <= {PACKED_MAX_K} and N*K < 2^32 (N={N}, K={Kd})")
    if offsets.numel() != E + 1:
        raise ValueError("offsets must have E+1 entries")
    if Kd % GROUP:
        raise ValueError(f"xq's K ({Kd}) must be its 128-padded pitch")
    if xs.shape != (R, Kd // GROUP) or ws.shape != (E, nblocks(N), Kd // GROUP):
        raise ValueError("scale shapes do not match the operands")
    if out is None:
        out = torch.empty((R, N), dtype=torch.bfloat16, device=xq.device)
    else:
        _check(out, "out", (torch.bfloat16,), 2)
        if out.shape != (R, N):
            raise ValueError("out must be [R, N]")
    if packed:
        fn = "smoe_grouped_gemm_fp8_packed_e8m0" if e8m0 else "smoe_grouped_gemm_fp8_packed"
        _C.call(fn, _ptr(_bytes(xq)), _ptr(xs), _ptr(wt), _ptr(ws), _ptr(offsets), E, R, N, Kd,
                _ptr(out), _stream())
    else:
        _C.call("smoe_grouped_gemm_fp8", _ptr(_bytes(xq)), _ptr(xs), _ptr(_bytes(wt)), _ptr(ws),
                _ptr(offsets), E, R, N, Kd, _ptr(out), None, 0, _stream())
    return out


def grouped_gemm_fp8_swiglu(xq: torch.Tensor, xs: torch.Tensor, w1q: torch.Tensor,
                            w1s: torch.Tensor, offsets: torch.Tensor, save_c1: bool = False,
                            scale: str = "amax"):
    """fc1 GEMM with SwiGLU + 1x128 requantisation fused into the epilogue.
    Same bytes as ``swiglu_quant(grouped_gemm_fp8(xq, xs, w1q, w1s, offsets))``;
    returns (hq [R,I] fp8, hs [R,I/128] f32), plus c1 [R,2I] bf16 when
    ``save_c1``.  Rows outside [offsets[0], offsets[E]) are not written.
    ``w1q`` may be a PackedWeight (see grouped_gemm_fp8).  ``scale="pow2"``
    (the E8M0 recipe: power-of-two operand scales in, power-of-two hs out)
    gives the bytes of ``swiglu_quant(grouped_gemm_fp8(..., e8m0=True),
    scale="pow2")``: fused (smoe_grouped_gemm_fp8_packed_e8m0_swiglu) for a
    packed W1 with I % 128 == 0, else those two calls."""
    pow2 = _scale(scale) != SCALES["amax"]
    _check(xq, "xq", (FP8, torch.uint8))
    wt, packed = _weight(w1q, "w1q")
    if pow2 and not (packed and wt.shape[1] % (2 * GROUP) == 0):
        c1 = grouped_gemm_fp8(xq, xs, w1q, w1s, offsets, e8m0=True)
        hq, hs = swiglu_quant(c1, scale=scale)
        return (hq, hs, c1) if save_c1 else (hq, hs)
    _check(xs, "xs", (torch.float32,), 2)
    _check(w1s, "w1s", (torch.float32,), 3)
    _check(offsets, "offsets", (torch.int32,), 1)
    R, Kd = xq.shape
    E, N, Kw = wt.shape
    if Kw != Kd:
        raise ValueError(f"K mismatch: xq has {Kd}, w1q has {Kw}")
    if packed and not (packed_e8m0_ok(N, Kd) if pow2 else packed_gemm_ok(N, Kd)):
        raise ValueError(f"packed weights need K % 512 == 0 (K % 128 == 0 and K >= 512 with "
                         f"scale='pow2'), K <= {PACKED_MAX_K} and N*K < 2^32 (N={N}, K={Kd})")
    if N % 2 == 0 and (N // 2) % GROUP and (N // 2) % 16 == 0:
        # I not a multiple of 128: the fused epilogue pairs 128-column gate
        # and up blocks, which such an I does not have; the same bytes come
        # from the GEMM followed by the SwiGLU kernel
        c1 = grouped_gemm_fp8(xq, xs, w1q, w1s, offsets)
        hq, hs = swiglu_quant(c1)
        return (hq, hs, c1) if save_c1 else (hq, hs)
    if N % (2 * GROUP):
        raise ValueError("w1q rows must be gate | up halves, each a multiple of 16")
    if offsets.numel() != E + 1:
        raise ValueError("offsets must have E+1 entries")
    if xs.shape != (R, Kd // GROUP) or w1s.shape != (E, N // GROUP, Kd // GROUP):
        raise ValueError("scale shapes do not match the operands")
    I = N // 2
    hq = torch.empty((R, I), dtype=FP8, device=xq.device)
    hs = torch.empty((R, I // GROUP), dtype=torch.float32, device=xq.device)
    c1 = torch.empty((R, N), dtype=torch.bfloat16, device=xq.device) if save_c1 else None
    if pow2:
        fn = "smoe_grouped_gemm_fp8_packed_e8m0_swiglu"
    else:
        fn = "smoe_grouped_gemm_fp8_packed_swiglu" if packed else "smoe_grouped_gemm_fp8_swiglu"
    _C.call(fn, _ptr(_bytes(xq)), _ptr(xs), _ptr(wt if packed else _bytes(wt)), _ptr(w1s),
            _ptr(offsets), E, R, I, Kd, _ptr(hq), _ptr(hs), _ptr(c1), _stream())
    return (hq, hs, c1) if save_c1 else (hq, hs)


# ------------------------------------------------------------------ SwiGLU
def swiglu_quant(c1: torch.Tensor, save_h: bool = False, scale: str = "amax"):
    """h = silu(gate)*up (gate = columns [0,I), up = [I,2I)) requantised 1x128.
    c1 [R,2I] bf16 -> (hq [R,pad128(I)] fp8, hs [R,pad128(I)/128] f32), plus
    h as bf16 [R,I] when ``save_h`` (the fc2 wgrad operand for the backward
    pass).  ``scale`` as for ``permute_quant_rows``."""
    mode = _scale(scale)
    _check(c1, "c1", (torch.bfloat16,), 2)
    R, I2 = c1.shape
    if I2 % 2:
        raise ValueError("c1 must have an even number of columns (gate | up)")
    I = I2 // 2
    hq = torch.empty((R, pad128(I)), dtype=FP8, device=c1.device)
    hs = torch.empty((R, nblocks(I)), dtype=torch.float32, device=c1.device)
    h = torch.empty((R, I), dtype=torch.bfloat16, device=c1.device) if save_h else None
    _C.call("smoe_swiglu_quant_ex", _ptr(c1), R, I, _ptr(hq), _ptr(hs), _ptr(h), mode, _stream())
    return (hq, hs, h) if save_h else (hq, hs)


# ----------------------------------------------------------------- combine
def unpermute_combine(y: torch.Tensor, inv_map: torch.Tensor, topk_w: torch.Tensor,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """out[t] = sum_k w[t,k] * y[inv_map[t*K+k]] in fp32 -> bf16 [T, H]
    (moe/MoE_detailed_computation_dataflow.md:195)."""
    _check(y, "y", (torch.bfloat16,), 2)
    _check(inv_map, "inv_map", (torch.int32,))
    _check(topk_w, "topk_w", (torch.float32,), 2)
    T, K = topk_w.shape
    R, H = y.shape
    if R != T * K or inv_map.numel() != R:
        raise ValueError("y / inv_map must have T*K rows")
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=y.device)
    else:
        _check(out, "out", (torch.bfloat16,), 2)
        if tuple(out.shape) != (T, H):
            raise ValueError(f"out must be [{T}, {H}] bf16")
    _C.call("smoe_unpermute_combine", _ptr(y), _ptr(inv_map), _ptr(topk_w), T, K, H, _ptr(out),
            _stream())
    return out


# ---------------------------------------------------------------- backward
def quant_rows(x: torch.Tensor, scale: str = "amax"):
    """1x128 row quantisation without permutation: x [M,C] bf16 ->
    (q [M,pad128(C)] fp8, s [M,pad128(C)/128] f32).  ``scale`` as for
    ``permute_quant_rows``."""
    mode = _scale(scale)
    _check(x, "x", (torch.bfloat16,), 2)
    M, C = x.shape
    q = torch.empty((M, pad128(C)), dtype=FP8, device=x.device)
    s = torch.empty((M, nblocks(C)), dtype=torch.float32, device=x.device)
    _C.call("smoe_quant_rows_1x128_ex", _ptr(x), M, C, _ptr(q), _ptr(s), mode, _stream())
    return q, s


def transpose_blockwise(wq: torch.Tensor, ws: torch.Tensor, k: int | None = None):
    """[E,N,Kp] fp8 + [E,NB,KB] -> [E,K,pad128(N)] + [E,KB,NB] (dgrad
    weights; blockwise quantisation commutes with the transpose).  ``k`` is
    the true K when wq's pitch Kp = pad128(K) holds padding (default Kp);
    the result's padding columns past N are 0."""
    _check(wq, "wq", (FP8, torch.uint8), 3)
    _check(ws, "ws", (torch.float32,), 3)
    E, N, Kp = wq.shape
    Kd = Kp if k is None else int(k)
    if N % 16 or Kd % 16 or Kp % GROUP or pad128(Kd) != Kp:
        raise ValueError(f"wq [{E}, {N}, {Kp}] is not the padded form of a K = {Kd} weight")
    if tuple(ws.shape) != (E, nblocks(N), Kp // GROUP):
        raise ValueError(f"ws must be [{E}, {nblocks(N)}, {Kp // GROUP}] for wq {tuple(wq.shape)}")
    wqT = torch.empty((E, Kd, pad128(N)), dtype=FP8, device=wq.device)
    wsT = torch.empty((E, Kp // GROUP, nblocks(N)), dtype=torch.float32, device=wq.device)
    _C.call("smoe_transpose_blockwise_fp8", _ptr(_bytes(wq)), _ptr(ws), E, N, Kd,
            _ptr(wqT), _ptr(wsT), _stream())
    return wqT, wsT


def _col_scale(col_scale: str) -> int:
    if col_scale not in COL_SCALES:
        raise ValueError(f"col_scale must be one of {sorted(COL_SCALES)}, got {col_scale!r}")
    return COL_SCALES[col_scale]


def quant_cols(x: torch.Tensor, offsets: torch.Tensor, gather: torch.Tensor | None = None,
               gather_div: int = 1, col_scale: str = "fp32"):
    """Transposed 128x1 quantisation over the expert row segments ``offsets``
    (E+1) of x [R,C] bf16, or, with ``gather`` [R] i32, of the rows
    x[gather[r] // gather_div].  -> (xTq [C, ld] fp8, xTs [C, ld/128] f32,
    pad [E+1] i32, ld) where pad are the 128-aligned segment starts.
    ``col_scale`` "fp32" is the s = amax/448 rule; "pow2" the least power of
    two >= amax/448 (the E8M0 recipe the wgrad's ``e8m0`` mode applies in
    hardware)."""
    _check(x, "x", (torch.bfloat16,), 2)
    _check(offsets, "offsets", (torch.int32,), 1)
    C = x.shape[1]
    if gather is not None:
        _check(gather, "gather", (torch.int32,), 1)
        R = gather.numel()
        if gather_div < 1:
            raise ValueError("gather_div must be >= 1")
        # the kernel reads x row gather[r] // gather_div with gather[r] < R
        if x.shape[0] * gather_div < R:
            raise ValueError(f"x has {x.shape[0]} rows; gather of {R} rows / {gather_div} "
                             f"needs at least {-(-R // gather_div)}")
    else:
        R = x.shape[0]
    E = offsets.numel() - 1
    ld = int(_C.lib().smoe_quant_cols_ld(R, E))
    xTq = torch.empty((C, ld), dtype=FP8, device=x.device)
    xTs = torch.empty((C, ld // GROUP), dtype=torch.float32, device=x.device)
    pad = torch.empty(E + 1, dtype=torch.int32, device=x.device)
    _C.call("smoe_quant_cols_128x1", _ptr(x), _ptr(gather), gather_div, R, C, _ptr(offsets), E,
            ld, _ptr(xTq), _ptr(xTs), _ptr(pad), _col_scale(col_scale), _stream())
    return xTq, xTs, pad, ld


def _fused_scale(col_scale: str, row_scale: str) -> int:
    return _col_scale(col_scale) | (ROWSCALE_POW2 if _scale(row_scale) else 0)


def quant_rows_cols(x: torch.Tensor, offsets: torch.Tensor, col_scale: str = "fp32",
                    row_scale: str = "amax"):
    """Both quantisations of x [R,C] bf16 from one read: the 1x128 rows of
    ``quant_rows`` and the transposed 128x1 columns of ``quant_cols`` over
    the expert segments ``offsets`` (which must cover all R rows).
    -> (xq [R,pad128(C)] fp8, xs [R,pad128(C)/128], xTq [C,ld] fp8,
    xTs [C,ld/128], pad, ld).  ``col_scale`` ("fp32" | "pow2") rules the
    column scales, ``row_scale`` ("amax" | "pow2") the row scales."""
    mode = _fused_scale(col_scale, row_scale)
    _check(x, "x", (torch.bfloat16,), 2)
    _check(offsets, "offsets", (torch.int32,), 1)
    R, C = x.shape
    E = offsets.numel() - 1
    ld = int(_C.lib().smoe_quant_cols_ld(R, E))
    xq = torch.empty((R, pad128(C)), dtype=FP8, device=x.device)
    xs = torch.empty((R, nblocks(C)), dtype=torch.float32, device=x.device)
    xTq = torch.empty((C, ld), dtype=FP8, device=x.device)
    xTs = torch.empty((C, ld // GROUP), dtype=torch.float32, device=x.device)
    pad = torch.empty(E + 1, dtype=torch.int32, device=x.device)
    _C.call("smoe_quant_rows_cols", _ptr(x), R, C, _ptr(offsets), E, ld, _ptr(xq), _ptr(xs),
            _ptr(xTq), _ptr(xTs), _ptr(pad), mode, _stream())
    return xq, xs, xTq, xTs, pad, ld


def swiglu_bwd_quant(c1: torch.Tensor, dh: torch.Tensor, offsets: torch.Tensor,
                     save_dc1: bool = False, col_scale: str = "fp32", row_scale: str = "amax"):
    """SwiGLU backward fused with both quantisations of its output: the
    bytes of ``quant_rows_cols(swiglu_bwd(c1, dh), offsets)`` without
    storing dc1 (returned as the last element when ``save_dc1``).
    c1 [R,2I], dh [R,I] bf16 -> (dcq [R,2I] fp8, dcs, dcTq [2I,ld] fp8, dcTs,
    pad, ld[, dc1]).  Scale rules as for ``quant_rows_cols``."""
    mode = _fused_scale(col_scale, row_scale)
    _check(c1, "c1", (torch.bfloat16,), 2)
    _check(dh, "dh", (torch.bfloat16,), 2)
    _check(offsets, "offsets", (torch.int32,), 1)
    R, N = c1.shape
    I = N // 2
    if dh.shape != (R, I) or N != 2 * I:
        raise ValueError("dh must be [R, I] for c1 [R, 2I]")
    E = offsets.numel() - 1
    ld = int(_C.lib().smoe_quant_cols_ld(R, E))
    dev = c1.device
    if I % GROUP:
        # dc1's 1x128 row groups straddle the dg | du boundary when I is not
        # a multiple of 128, which the fused kernel's column slabs assume: the
        # same bytes from the SwiGLU backward kernel and the one-read quantiser
        dc1 = swiglu_bwd(c1, dh)
        out = quant_rows_cols(dc1, offsets, col_scale=col_scale, row_scale=row_scale)
        return out + (dc1,) if save_dc1 else out
    dcq = torch.empty((R, N), dtype=FP8, device=dev)
    dcs = torch.empty((R, N // GROUP), dtype=torch.float32, device=dev)
    dcTq = torch.empty((N, ld), dtype=FP8, device=dev)
    dcTs = torch.empty((N, ld // GROUP), dtype=torch.float32, device=dev)
    pad = torch.empty(E + 1, dtype=torch.int32, device=dev)
    dc1 = torch.empty((R, N), dtype=torch.bfloat16, device=dev) if save_dc1 else None
    _C.call("smoe_swiglu_bwd_quant", _ptr(c1), _ptr(dh), R, I, _ptr(offsets), E, ld, _ptr(dcq),
            _ptr(dcs), _ptr(dcTq), _ptr(dcTs), _ptr(pad), _ptr(dc1), mode, _stream())
    out = (dcq, dcs, dcTq, dcTs, pad, ld)
    return out + (dc1,) if save_dc1 else out


WGRAD_MODES = {(torch.float32, False): 0, (torch.float32, True): 1,
               (torch.bfloat16, False): 2, (torch.bfloat16, True): 3}
WGRAD_E8M0 = 4  # SMOE_WGRAD_E8M0


def grouped_gemm_fp8_wgrad(aTq, aTs, bTq, bTs, pad, ld: int, out: torch.Tensor | None = None,
                           accumulate: bool = False, dtype=torch.float32,
                           e8m0: bool = False) -> torch.Tensor:
    """dW[e] = A_e^T B_e over each expert's rows from quant_cols operands:
    aT [N, ld], bT [K, ld] -> [E, N, K] (into ``out`` when given, else a new
    tensor of ``dtype``, fp32 or bf16).  With ``accumulate`` the gradient is
    added into ``out`` (fp32: one fp32 addition per value; bf16: the fp32 sum
    rounded once), as a gradient-accumulation buffer (``main_grad``) needs;
    experts without rows leave ``out`` untouched.  ``e8m0``: the operands
    come from the ``col_scale="pow2"`` quantisers, whose power-of-two scales
    the scaled MFMA applies in hardware (scales that are not powers of two
    would be read by their exponent only)."""
    _check(aTq, "aTq", (FP8, torch.uint8), 2)
    _check(bTq, "bTq", (FP8, torch.uint8), 2)
    _check(aTs, "aTs", (torch.float32,), 2)
    _check(bTs, "bTs", (torch.float32,), 2)
    _check(pad, "pad", (torch.int32,), 1)
    N, K, E = aTq.shape[0], bTq.shape[0], pad.numel() - 1
    if aTq.shape[1] != ld or bTq.shape[1] != ld or ld % GROUP:
        raise ValueError("operands must share the padded row length ld (a multiple of 128)")
    if tuple(aTs.shape) != (N, ld // GROUP) or tuple(bTs.shape) != (K, ld // GROUP):
        raise ValueError(f"scales must be [{N}, {ld // GROUP}] and [{K}, {ld // GROUP}]")
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs the buffer to add into (out)")
        if dtype not in (torch.float32, torch.bfloat16):
            raise TypeError("the weight gradient is fp32 or bf16")
        dW = torch.empty((E, N, K), dtype=dtype, device=aTq.device)
    else:
        _check(out, "out", (torch.float32, torch.bfloat16), 3)
        if tuple(out.shape) != (E, N, K):
            raise ValueError(f"out must be [{E}, {N}, {K}]")
        dW = out
    _C.call("smoe_grouped_gemm_fp8_wgrad_ex", _ptr(_bytes(aTq)), _ptr(aTs), _ptr(_bytes(bTq)),
            _ptr(bTs), _ptr(pad), E, N, K, ld, _ptr(dW),
            WGRAD_MODES[(dW.dtype, bool(accumulate))] | (WGRAD_E8M0 if e8m0 else 0), _stream())
    return dW


def swiglu_bwd(c1: torch.Tensor, dh: torch.Tensor) -> torch.Tensor:
    """c1 [R,2I] (gate | up), dh [R,I] bf16 -> dc1 [R,2I] bf16 = [dg | du]."""
    _check(c1, "c1", (torch.bfloat16,), 2)
    _check(dh, "dh", (torch.bfloat16,), 2)
    R, I2 = c1.shape
    if dh.shape != (R, I2 // 2):
        raise ValueError("dh must be [R, I]")
    dc1 = torch.empty_like(c1)
    _C.call("smoe_swiglu_bwd", _ptr(c1), _ptr(dh), R, I2 // 2, _ptr(dc1), _stream())
    return dc1


def unpermute_combine_bwd(dout: torch.Tensor, y: torch.Tensor, inv_map: torch.Tensor,
                          topk_w: torch.Tensor):
    """Backward of unpermute_combine: -> (dy [T*K,H] bf16, dw [T,K] f32)."""
    _check(dout, "dout", (torch.bfloat16,), 2)
    _check(y, "y", (torch.bfloat16,), 2)
    _check(inv_map, "inv_map", (torch.int32,))
    _check(topk_w, "topk_w", (torch.float32,), 2)
    T, K = topk_w.shape
    H = dout.shape[1]
    if dout.shape[0] != T or tuple(y.shape) != (T * K, H) or inv_map.numel() != T * K:
        raise ValueError("dout must be [T, H], y [T*K, H] and inv_map T*K for topk_w [T, K]")
    dy = torch.empty((T * K, H), dtype=torch.bfloat16, device=dout.device)
    dw = torch.empty((T, K), dtype=torch.float32, device=dout.device)
    _C.call("smoe_unpermute_combine_bwd", _ptr(dout), _ptr(y), _ptr(inv_map), _ptr(topk_w), T, K,
            H, _ptr(dy), _ptr(dw), _stream())
    return dy, dw


def unpermute_combine_bwd_quant(dout: torch.Tensor, y: torch.Tensor, inv_map: torch.Tensor,
                                row_map: torch.Tensor, topk_w: torch.Tensor,
                                offsets: torch.Tensor, col_scale: str = "fp32",
                                row_scale: str = "amax", cols: bool = True):
    """Combine backward fused with both quantisations of dy: the bytes of
    ``quant_rows_cols(unpermute_combine_bwd(...)[0], offsets, col_scale,
    row_scale)`` and dw, without storing dy.  -> (dyq [T*K,pad128(H)] fp8,
    dys, dyTq [H,ld] fp8, dyTs, pad, ld, dw [T,K] f32).  ``cols=False``
    skips the column pass (dyTq, dyTs are None); ``combine_bwd_quant_cols``
    gives it on its own."""
    mode = _fused_scale(col_scale, row_scale)
    _check(dout, "dout", (torch.bfloat16,), 2)
    _check(y, "y", (torch.bfloat16,), 2)
    _check(inv_map, "inv_map", (torch.int32,))
    _check(row_map, "row_map", (torch.int32,))
    _check(topk_w, "topk_w", (torch.float32,), 2)
    _check(offsets, "offsets", (torch.int32,), 1)
    T, K = topk_w.shape
    H = dout.shape[1]
    R = T * K
    if dout.shape[0] != T or y.shape != (R, H):
        raise ValueError("dout must be [T, H] and y [T*K, H] for topk_w [T, K]")
    if inv_map.numel() != R or row_map.numel() != R:
        raise ValueError("inv_map and row_map must hold T*K entries")
    E = offsets.numel() - 1
    ld = int(_C.lib().smoe_quant_cols_ld(R, E))
    dev = dout.device
    dyq = torch.empty((R, pad128(H)), dtype=FP8, device=dev)
    dys = torch.empty((R, nblocks(H)), dtype=torch.float32, device=dev)
    dyTq = torch.empty((H, ld), dtype=FP8, device=dev) if cols else None
    dyTs = torch.empty((H, ld // GROUP), dtype=torch.float32, device=dev) if cols else None
    pad = torch.empty(E + 1, dtype=torch.int32, device=dev)
    dw = torch.empty((T, K), dtype=torch.float32, device=dev)
    _C.call("smoe_unpermute_combine_bwd_quant", _ptr(dout), _ptr(y), _ptr(inv_map),
            _ptr(row_map), _ptr(topk_w), T, K, H, _ptr(offsets), E, ld, _ptr(dyq), _ptr(dys),
            _ptr(dyTq), _ptr(dyTs), _ptr(pad), _ptr(dw), mode, _stream())
    return dyq, dys, dyTq, dyTs, pad, ld, dw


def combine_bwd_quant_cols(dout: torch.Tensor, row_map: torch.Tensor, topk_w: torch.Tensor,
                           offsets: torch.Tensor, col_scale: str = "fp32"):
    """The column pass of ``unpermute_combine_bwd_quant`` alone (dy's 128x1
    columns rebuilt from dout, row_map and topk_w; y is not read):
    -> (dyTq [H,ld] fp8, dyTs, pad, ld), the same bytes."""
    mode = _col_scale(col_scale)
    _check(dout, "dout", (torch.bfloat16,), 2)
    _check(row_map, "row_map", (torch.int32,))
    _check(topk_w, "topk_w", (torch.float32,), 2)
    _check(offsets, "offsets", (torch.int32,), 1)
    T, K = topk_w.shape
    H = dout.shape[1]
    R = T * K
    if dout.shape[0] != T:
        raise ValueError("dout must be [T, H] for topk_w [T, K]")
    if row_map.numel() != R:
        raise ValueError("row_map must hold T*K entries")
    E = offsets.numel() - 1
    ld = int(_C.lib().smoe_quant_cols_ld(R, E))
    dev = dout.device
    dyTq = torch.empty((H, ld), dtype=FP8, device=dev)
    dyTs = torch.empty((H, ld // GROUP), dtype=torch.float32, device=dev)
    pad = torch.empty(E + 1, dtype=torch.int32, device=dev)
    _C.call("smoe_combine_bwd_quant_cols", _ptr(dout), _ptr(row_map), _ptr(topk_w), T, K, H,
            _ptr(offsets), E, ld, _ptr(dyTq), _ptr(dyTs), _ptr(pad), mode, _stream())
    return dyTq, dyTs, pad, ld
