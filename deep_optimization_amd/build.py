"""Builds libdopt.so (the gfx950 HIP kernels + C ABI of include/dopt.h) in-tree.

Usage: ``python -m deep_optimization_amd.build`` or ``deep_optimization_amd.build.build()``.
Every call recompiles all sources (hipcc cross-compiles for gfx950 without a GPU).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ_DIR = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libdopt.so")

SOURCES = [
    "dopt_abi.hip",
    "quant_pack_f32.hip",
    "quant_pack_f16.hip",
    "quant_pack_bf16.hip",
    "dequant_unpack.hip",
    "pack_codes.hip",
    "fp8_gemm.hip",
    "fp8_pack.hip",
    "act_fused.hip",
    "bn_fused.hip",
    "dw_gemm.hip",
    "graph_tools.hip",
    "alam.hip",
]

ARCH = "gfx950"

# -ffp-contract=off: the quantizer's fp32 ops are rounded one by one (bit-exact contract);
# correctly rounded fp32 divide for step = range/QMAX and inv = 1/step;
# packed-fp32 VALU ops disabled (ordinary scalar fp32 code only).
HIPFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-rdc",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libdopt.so)")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *HIPFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile every source for gfx950 and link libdopt.so next to this file; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-fno-gpu-rdc", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
