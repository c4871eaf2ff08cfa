"""smoe — MI355X-native (gfx950) SimpleMoE expert-layer hot path.

Python host code over a C-ABI library of hand-written HIP kernels
(libsmoe.so, built in-tree by ``python -m smoe.build``).
"""
from . import _C, ops, workloads  # noqa: F401
from .layer import SimpleMoE  # noqa: F401
from .ops import (  # noqa: F401
    router_topk,
    router_topk_bwd,
    last_route_status,
    check_route_status,
    route_sort,
    route_topk_sort,
    permute_quant_rows,
    permute_quant,
    quantize_weight_blockwise,
    grouped_gemm_fp8,
    grouped_gemm_fp8_swiglu,
    swiglu_quant,
    unpermute_combine,
    quant_rows,
    transpose_blockwise,
    quant_cols,
    quant_rows_cols,
    swiglu_bwd_quant,
    grouped_gemm_fp8_wgrad,
    swiglu_bwd,
    unpermute_combine_bwd,
    unpermute_combine_bwd_quant,
)

__all__ = ["SimpleMoE", "workloads",
           "router_topk",
           "router_topk_bwd",
           "last_route_status",
           "check_route_status",
           "route_sort",
           "route_topk_sort",
           "permute_quant_rows",
           "permute_quant",
           "quantize_weight_blockwise",
           "grouped_gemm_fp8",
           "grouped_gemm_fp8_swiglu",
           "swiglu_quant",
           "unpermute_combine",
           "quant_rows",
           "transpose_blockwise",
           "quant_cols",
           "quant_rows_cols",
           "swiglu_bwd_quant",
           "grouped_gemm_fp8_wgrad",
           "swiglu_bwd",
           "unpermute_combine_bwd",
           "unpermute_combine_bwd_quant",
           ]
