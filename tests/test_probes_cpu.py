"""The probe library (libdopt_probe.so) on the CPU: it exports what probes/dopt_probe.h declares,
the product library exports none of it, and the argument checks fail before any HIP call."""
import ctypes
import os
import re

import pytest

import probes
from deep_optimization_amd import _lib

HEADER = os.path.join(os.path.dirname(probes.__file__), "dopt_probe.h")
needs_probe_lib = pytest.mark.skipif(not os.path.exists(probes.LIB), reason="libdopt_probe.so not built")
EINVAL = -2


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(dopt_\w+)\s*\(", text, re.M)))


def test_header_declares_the_loader_symbols():
    assert header_functions() == sorted(probes.SYMBOLS)


@needs_probe_lib
def test_probe_library_exports_and_product_library_does_not():
    P = ctypes.CDLL(probes.LIB)
    for name in header_functions():
        assert hasattr(P, name), name
    if os.path.exists(_lib.LIB_PATH):
        D = ctypes.CDLL(_lib.LIB_PATH)
        for name in ("dopt_stream_probe", "dopt_valu_probe"):
            assert not hasattr(D, name), name


@needs_probe_lib
def test_valu_probe_argument_checks():
    L = probes.lib()
    assert L.dopt_valu_probe(9, 16, 8, None) == EINVAL  # unknown kind
    assert L.dopt_valu_probe(-1, 16, 8, None) == EINVAL
    assert L.dopt_valu_probe(0, 16, 0, None) == EINVAL  # no blocks
    assert L.dopt_valu_probe(0, 16, 65537, None) == EINVAL
    assert L.dopt_valu_probe(0, None, 8, None) == EINVAL
    assert L.dopt_valu_probe(0, 18, 8, None) == EINVAL  # unaligned
    assert b"kind" in L.dopt_probe_last_error() or b"pointer" in L.dopt_probe_last_error()


@needs_probe_lib
def test_stream_probe_argument_checks():
    L = probes.lib()
    assert L.dopt_stream_probe(16, None, 16, 16, 4, 3, None) == EINVAL  # bits
    assert L.dopt_stream_probe(20, None, 16, 16, 4, 2, None) == EINVAL  # unaligned x
    assert L.dopt_stream_probe(16, None, 16, 16, -1, 2, None) == EINVAL
    assert L.dopt_stream_probe(16, None, 16, 16, 0, 2, None) == 0  # nothing to do
