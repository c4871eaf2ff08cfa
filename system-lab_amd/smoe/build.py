"""Build libsmoe.so (the C-ABI library of HIP kernels for gfx950) in-tree.

    python -m smoe.build            # from system-lab_amd/

Every HIP source is compiled by hipcc for gfx950 only, with IEEE-exact fp32
division, no multiply-add contraction (the quantisation and combine kernels
are bit-exact against a CPU restatement of the same operations) and packed
fp32 instructions disabled.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(PKG), "csrc")
LIB = os.path.join(PKG, "libsmoe.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["smoe_api.cpp", "smoe_route.hip", "smoe_quant.hip", "smoe_gemm.hip",
           "smoe_gemm_wgrad.hip", "smoe_gemm_packed.hip", "smoe_gemm_e8m0.hip", "smoe_combine.hip", "smoe_backward.hip"]
# the benchmark's HBM probe: its own library, not part of libsmoe.so
PROBE_SOURCES = ["bench/smoe_bw_probe.hip"]
PROBE_LIB = os.path.join(PKG, "libsmoe_probe.so")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]


def _compile(src: str) -> str:
    obj = os.path.join(PKG, "_obj", os.path.splitext(os.path.basename(src))[0] + ".o")
    os.makedirs(os.path.dirname(obj), exist_ok=True)
    path = os.path.join(CSRC, src)
    if src.endswith(".hip"):
        cmd = [HIPCC, *HIP_FLAGS, "-c", path, "-o", obj]
    else:
        cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def _link(objs, lib: str) -> None:
    tmp = lib + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    srcs = SOURCES + PROBE_SOURCES
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(objs[:len(SOURCES)], LIB)
    _link(objs[len(SOURCES):], PROBE_LIB)
    if verbose:
        print("built", LIB, "and", PROBE_LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
