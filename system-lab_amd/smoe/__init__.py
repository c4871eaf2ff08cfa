"""smoe — MI355X-native (gfx950) SimpleMoE expert-layer hot path.

Python host code over a C-ABI library of hand-written HIP kernels
(libsmoe.so, built in-tree by ``python -m smoe.build``).
"""
from . import _C, ops, workloads  # noqa: F401
from .layer import SimpleMoE  # noqa: F401
from .ops import (grouped_gemm_fp8, permute_quant, permute_quant_rows,  # noqa: F401
                  quantize_weight_blockwise, route_sort, router_topk, swiglu_quant,
                  unpermute_combine)

__all__ = ["SimpleMoE", "router_topk", "route_sort", "permute_quant", "permute_quant_rows",
           "quantize_weight_blockwise", "grouped_gemm_fp8", "swiglu_quant",
           "unpermute_combine", "workloads"]
