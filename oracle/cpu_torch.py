"""PyTorch-CPU restatements of the hot path — TEST INFRASTRUCTURE ONLY.

The CPU baselines that bench.py times next to the GPU path, written with
vectorised torch CPU ops so that they run multi-threaded on the host's cores:
  * ``dispatch_quant``: route sort + permute + 1x128 quantisation (C2, C3);
  * ``grouped_gemm_fp8``: the blockwise-scaled grouped GEMM (C5) as fp32
    dequantise + matmul per expert.
Only ``tests/`` and bench.py's CPU baseline legs use them; the product path
never does.

Parity: ``tests/test_oracle.py`` holds ``dispatch_quant`` byte-for-byte to
the numpy oracle (``smoe_oracle.route_sort`` + ``smoe_oracle.permute_quant``)
and ``grouped_gemm_fp8`` to the float64 oracle within the GEMM tolerance.
The e4m3 encode is torch's own ``float8_e4m3fn`` cast after the +-448 clamp,
which is the cast the oracle's software encoder is pinned against.
"""
import torch

GROUP = 128
E4M3_MAX = 448.0


def dispatch_quant(x: torch.Tensor, topk_idx: torch.Tensor, num_experts: int):
    """x [T,H] bf16, topk_idx [T,K] int -> (xq [T*K,H] uint8, xs [T*K,H/128]
    f32, row_map, inv_map, counts, offsets), all on the CPU.

    C2 (notes/2026-04/2026-04-10_monolithmoe_layout_c_pack_optimization.md:56,80,120):
    pairs p = t*K + k sorted stably by expert id, row_map[r] = p,
    inv_map[p] = r.  C3 (moe/MegatronCore_MoE_reading_notes.md:498-501): per
    1x128 group s = amax/448 (1 when amax == 0), q = e4m3(clamp(x/s, +-448)),
    computed once per token and copied to its K sorted rows."""
    T, H = x.shape
    K = topk_idx.shape[1]
    flat = topk_idx.reshape(-1).to(torch.int64)
    row_map = torch.sort(flat, stable=True).indices
    inv_map = torch.empty_like(row_map)
    inv_map[row_map] = torch.arange(flat.numel(), dtype=torch.int64)
    counts = torch.bincount(flat, minlength=num_experts)
    offsets = torch.zeros(num_experts + 1, dtype=torch.int64)
    offsets[1:] = torch.cumsum(counts, 0)
    g = x.to(torch.float32).view(T, H // GROUP, GROUP)
    amax = g.abs().amax(dim=2)
    s = torch.where(amax == 0, torch.ones_like(amax), amax / E4M3_MAX)
    q = (g / s.unsqueeze(2)).clamp_(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    q = q.view(torch.uint8).view(T, H)
    tok = row_map // K
    return (q[tok], s[tok], row_map.to(torch.int32), inv_map.to(torch.int32),
            counts.to(torch.int32), offsets.to(torch.int32))


def grouped_gemm_fp8(xq: torch.Tensor, xs: torch.Tensor, wq: torch.Tensor, ws: torch.Tensor,
                     offsets) -> torch.Tensor:
    """C5 on the CPU: xq [R,K] u8 (e4m3 bytes), xs [R,K/128] f32, wq [E,N,K] u8,
    ws [E,N/128,K/128] f32, offsets [E+1] -> fp32 [R,N].  Each operand is
    dequantised to fp32 (value * its block scale) and expert e's rows
    [offsets[e], offsets[e+1]) are multiplied by W[e]^T with torch.matmul
    (summary/fp8_expert_gemm_optimization.md:89-95: fp8 dot -> fp32 acc ->
    dequant; the scales are applied before the product here, which is the
    same sum up to fp32 rounding)."""
    R, Kd = xq.shape
    E, N, _ = wq.shape
    a = xq.view(torch.float8_e4m3fn).to(torch.float32).view(R, Kd // GROUP, GROUP)
    a = (a * xs.unsqueeze(2)).view(R, Kd)
    out = torch.zeros((R, N), dtype=torch.float32)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi <= lo:
            continue
        w = wq[e].view(torch.float8_e4m3fn).to(torch.float32).view(N // GROUP, GROUP, Kd // GROUP, GROUP)
        w = (w * ws[e][:, None, :, None]).view(N, Kd)
        out[lo:hi] = a[lo:hi] @ w.T
    return out
