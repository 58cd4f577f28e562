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


TORCH_LIB = os.path.join(PKG, "libdopt_torch.so")
INCLUDE = os.path.join(os.path.dirname(PKG), "include")


def build_torch_ops(verbose: bool = False) -> str:
    """The native act_lib operator kernels (csrc/torch_ops.cpp, host C++ against torch's headers and
    libdopt.so) -> libdopt_torch.so next to libdopt.so."""
    import torch
    import torch.utils.cpp_extension as ce

    cxx = shutil.which("g++") or "c++"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [f"-I{p}" for p in ce.include_paths(device_type="cuda")] + [f"-I{INCLUDE}"]
    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    tmp = TORCH_LIB + ".tmp"
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DUSE_ROCM=1",
           "-D__HIP_PLATFORM_AMD__=1", *incs, os.path.join(CSRC, "torch_ops.cpp"), f"-L{PKG}", "-ldopt",
           f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}", "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"torch_ops.cpp failed to build:\n{proc.stderr[-4000:]}")
    os.replace(tmp, TORCH_LIB)
    if verbose:
        print(f"built {TORCH_LIB}")
    return TORCH_LIB


def build(jobs: int | None = None, verbose: bool = False) -> str:
    """Compile every source for gfx950, link libdopt.so next to this file and build the native
    operator library on it; returns libdopt.so's path."""
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
    build_torch_ops(verbose)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
