"""PyTorch-CPU restatement of the dispatch step — TEST INFRASTRUCTURE ONLY.

The CPU baseline that bench.py times next to the GPU path: the same route
sort + permute + 1x128 quantisation semantics as ``smoe_oracle`` (C2, C3),
written with vectorised torch CPU ops so that it runs multi-threaded on the
host's cores.  Only ``tests/`` and bench.py's ``cpu_baseline`` leg use it;
the product path never does.

Parity: ``tests/test_oracle.py`` holds it byte-for-byte to the numpy oracle
(``smoe_oracle.route_sort`` + ``smoe_oracle.permute_quant``).  The e4m3
encode is torch's own ``float8_e4m3fn`` cast after the +-448 clamp, which is
the cast the oracle's software encoder is pinned against.
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
