"""ctypes binding of libsmoe.so, the C-ABI library of gfx950 HIP kernels.

The library is loaded from this package directory only (built in-tree by
``smoe.build``).  There is no fallback: if the library is missing, every op
raises ``SmoeLibraryMissing``.  Signatures mirror ``include/smoe.h``.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libsmoe.so")

c_int, c_size_t, c_void_p, c_char_p = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
P = c_void_p  # every device pointer travels as an untyped address

# name -> (restype, argtypes); the complete export list of include/smoe.h
SIGNATURES = {
    "smoe_strerror": (c_char_p, [c_int]),
    "smoe_version": (c_char_p, []),
    "smoe_router_topk": (c_int, [P, P, c_int, c_int, c_int, P, P, P]),
    "smoe_router_topk_bwd": (c_int, [P, P, P, c_int, c_int, c_int, P, P]),
    "smoe_route_sort_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "smoe_route_sort": (c_int, [P, c_int, c_int, c_int, P, P, P, P, P, c_size_t, P]),
    "smoe_route_sort_noalloc_max_bytes": (c_size_t, []),
    "smoe_route_sort_noalloc": (c_int, [P, c_int, c_int, c_int, P, P, P, P, P]),
    "smoe_route_topk_sort": (c_int, [P, P, c_int, c_int, c_int, P, P, P, P, P, P, P, c_size_t,
                                     P]),
    "smoe_permute_quant": (c_int, [P, P, c_int, c_int, c_int, P, P, P]),
    "smoe_permute_quant_ex": (c_int, [P, P, c_int, c_int, c_int, P, P, c_int, P]),
    "smoe_dispatch_quant": (c_int, [P, P, c_int, c_int, c_int, c_int, P, P, P, P, P, P, P,
                                    c_size_t, P]),
    "smoe_selftest_quant": (c_int, [P, P]),
    "smoe_selftest_recip": (c_int, [P, P]),
    "smoe_quantize_weight_blockwise": (c_int, [P, c_int, c_int, c_int, P, P, P]),
    "smoe_quantize_weight_blockwise_ex": (c_int, [P, c_int, c_int, c_int, P, P, c_int, P]),
    "smoe_grouped_gemm_fp8_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "smoe_grouped_gemm_fp8": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, P, P,
                                      c_size_t, P]),
    "smoe_grouped_gemm_fp8_swiglu": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, P, P,
                                             P, P]),
    "smoe_pack_weight_fp8": (c_int, [P, c_int, c_int, c_int, P, P]),
    "smoe_grouped_gemm_fp8_packed": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, P, P]),
    "smoe_grouped_gemm_fp8_packed_e8m0": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, P, P]),
    "smoe_grouped_gemm_fp8_packed_e8m0_swiglu": (c_int, [P, P, P, P, P, c_int, c_int, c_int,
                                                         c_int, P, P, P, P]),
    "smoe_grouped_gemm_fp8_packed_swiglu": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int,
                                                    P, P, P, P]),
    "smoe_swiglu_quant": (c_int, [P, c_int, c_int, P, P, P]),
    "smoe_swiglu_quant_h": (c_int, [P, c_int, c_int, P, P, P, P]),
    "smoe_swiglu_quant_ex": (c_int, [P, c_int, c_int, P, P, P, c_int, P]),
    "smoe_unpermute_combine": (c_int, [P, P, P, c_int, c_int, c_int, P, P]),
    "smoe_quant_rows_1x128": (c_int, [P, c_int, c_int, P, P, P]),
    "smoe_quant_rows_1x128_ex": (c_int, [P, c_int, c_int, P, P, c_int, P]),
    "smoe_transpose_blockwise_fp8": (c_int, [P, P, c_int, c_int, c_int, P, P, P]),
    "smoe_quant_cols_ld": (c_int, [c_int, c_int]),
    "smoe_quant_cols_128x1": (c_int, [P, P, c_int, c_int, c_int, P, c_int, c_int, P, P, P, c_int,
                                      P]),
    "smoe_quant_rows_cols": (c_int, [P, c_int, c_int, P, c_int, c_int, P, P, P, P, P, c_int, P]),
    "smoe_swiglu_bwd_quant": (c_int, [P, P, c_int, c_int, P, c_int, c_int, P, P, P, P, P, P, c_int,
                                      P]),
    "smoe_grouped_gemm_fp8_wgrad": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, P, P]),
    "smoe_grouped_gemm_fp8_wgrad_ex": (c_int, [P, P, P, P, P, c_int, c_int, c_int, c_int, P,
                                               c_int, P]),
    "smoe_swiglu_bwd": (c_int, [P, P, c_int, c_int, P, P]),
    "smoe_unpermute_combine_bwd": (c_int, [P, P, P, P, c_int, c_int, c_int, P, P, P]),
    "smoe_unpermute_combine_bwd_quant": (c_int, [P, P, P, P, P, c_int, c_int, c_int, P, c_int,
                                                 c_int, P, P, P, P, P, P, c_int, P]),
    "smoe_combine_bwd_quant_cols": (c_int, [P, P, P, c_int, c_int, c_int, P, c_int, c_int, P, P,
                                            P, c_int, P]),
}


# libsmoe_probe.so: the benchmark's HBM traffic-mix probe, kept out of the
# product library (csrc/bench/smoe_bw_probe.hip)
PROBE_PATH = os.path.join(_HERE, "libsmoe_probe.so")
PROBE_SIGNATURES = {"smoe_bw_probe": (c_int, [P, c_int, c_int, c_int, P, c_size_t, P, P])}


class SmoeLibraryMissing(RuntimeError):
    pass


class SmoeError(RuntimeError):
    def __init__(self, fn: str, status: int, text: str):
        super().__init__(f"{fn} failed with status {status}: {text}")
        self.status = status


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libsmoe.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise SmoeLibraryMissing(
                        f"{LIB_PATH} not found: build it with `python -m smoe.build` "
                        "(the HIP library is the only implementation; there is no fallback)")
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise SmoeError on failure."""
    st = getattr(lib(), name)(*args)
    if st != 0:
        raise SmoeError(name, st, lib().smoe_strerror(st).decode())


_probe = None


def probe_call(name: str, *args) -> None:
    """Call an entry point of the benchmark's probe library
    (libsmoe_probe.so, built next to libsmoe.so) and raise on failure."""
    global _probe
    with _lock:
        if _probe is None:
            if not os.path.exists(PROBE_PATH):
                raise SmoeLibraryMissing(f"{PROBE_PATH} not found: build it with `python -m smoe.build`")
            handle = ctypes.CDLL(PROBE_PATH)
            for n, (res, a) in PROBE_SIGNATURES.items():
                getattr(handle, n).restype = res
                getattr(handle, n).argtypes = a
            _probe = handle
    st = getattr(_probe, name)(*args)
    if st != 0:
        raise SmoeError(name, st, lib().smoe_strerror(st).decode())
