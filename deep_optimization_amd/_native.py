"""The native operator library (libdopt_torch.so, csrc/torch_ops.cpp): C++ CUDA (HIP) kernels of
the act_lib operators the compressed layers call most often, registered with the dispatcher.

``load()`` runs before act_lib.py and bn_lib.py define their operators: the dispatcher takes a
kernel for an operator whose schema is defined later. For the operators in ``OPS`` the Python
modules then register only the schema and the fake kernel; every other operator keeps its Python
implementation. When the library is not built the Python implementations serve all operators
(they call the same C ABI, through ctypes).
"""
from __future__ import annotations

import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdopt_torch.so")
OPS = frozenset({"quant_pack", "quant_pack_tiles", "dequant_unpack", "dequant_unpack_tiles", "quant_pack_triton",
                 "dequant_unpack_triton", "relu_fwd_fused_pack", "relu_bwd_fused_unpack", "bn_train_fwd",
                 "bn_train_bwd"})

_loaded = None


def load() -> bool:
    """Loads the library once; returns whether its kernels are registered."""
    global _loaded
    if _loaded is None:
        _loaded = False
        if os.path.exists(LIB_PATH):
            torch.ops.load_library(LIB_PATH)
            _loaded = True
    return _loaded


def native(name: str) -> bool:
    """Whether operator ``name``'s CUDA kernel comes from the native library."""
    return name in OPS and load()


__all__ = ["load", "native", "OPS", "LIB_PATH"]
