"""Measurement probes of the benchmark and the tests, kept out of the product library.

``libdopt_probe.so`` (``stream_probe.hip``, declared in ``dopt_probe.h``) holds two families of
diagnostic kernels: ``dopt_stream_probe``, the memory system's ceiling for the quant-pack kernel's
byte mix, and ``dopt_valu_probe``, instruction and MFMA-stream issue costs plus the exhaustive
check of the quantizer's exact-division helpers. ``modes`` holds bench.py's probe modes.

``build()`` compiles the library for gfx950 next to this file; ``lib()`` loads it.
"""
from __future__ import annotations

import ctypes
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libdopt_probe.so")
CSRC = os.path.join(os.path.dirname(HERE), "deep_optimization_amd", "csrc")
SYMBOLS = ("dopt_probe_last_error", "dopt_stream_probe", "dopt_valu_probe")

_lib = None


def build(verbose: bool = False) -> str:
    """hipcc for gfx950 with the product library's flags; returns the library's path."""
    from deep_optimization_amd.build import HIPFLAGS

    hipcc = next(c for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc"))
                 if c and os.path.exists(c))
    tmp = LIB + ".tmp"
    cmd = [hipcc, *HIPFLAGS, "-shared", "-I", HERE, "-I", CSRC, os.path.join(HERE, "stream_probe.hip"), "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for stream_probe.hip:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            raise RuntimeError(f"{LIB} is not built: run `python -c 'import probes; probes.build()'`")
        L = ctypes.CDLL(LIB)
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        L.dopt_probe_last_error.restype = ctypes.c_char_p
        L.dopt_probe_last_error.argtypes = []
        L.dopt_stream_probe.argtypes = [vp, vp, vp, vp, i64, i32, vp]
        L.dopt_stream_probe.restype = i32
        L.dopt_valu_probe.argtypes = [i32, vp, i64, vp]
        L.dopt_valu_probe.restype = i32
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: {lib().dopt_probe_last_error().decode()} (status {rc})")


__all__ = ["build", "lib", "check", "SYMBOLS", "LIB"]
