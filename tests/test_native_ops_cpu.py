"""The native operator library (libdopt_torch.so, csrc/torch_ops.cpp) on the CPU: it loads, and
the dispatcher holds its CUDA kernels for exactly the operators _native.OPS names, beside the
Python fake kernels; the other operators keep their Python CUDA kernels."""
import os

import pytest
import torch

import deep_optimization_amd  # noqa: F401
from deep_optimization_amd import _native

needs_native = pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="libdopt_torch.so not built")


@needs_native
def test_native_kernels_are_registered():
    assert _native.load()
    for name in sorted(_native.OPS):
        dump = torch._C._dispatch_dump(f"act_lib::{name}")
        cuda = [line for line in dump.splitlines() if line.startswith("CUDA:")]
        assert cuda and "torch_ops.cpp" in cuda[0], (name, dump)
        assert any(line.startswith("Meta:") for line in dump.splitlines()), name
    for name in ("pack_triton", "unpack_triton", "gelu_fwd_fused_quan_pack", "dw_gemm", "bn_fwd_reduce"):
        cuda = [line for line in torch._C._dispatch_dump(f"act_lib::{name}").splitlines() if line.startswith("CUDA:")]
        assert cuda and ".py" in cuda[0], name


@needs_native
def test_native_ops_trace_under_fake_tensors():
    """The fake kernels still serve shape propagation for the native operators."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        x = torch.empty((4, 6, 256), dtype=torch.bfloat16, device="cuda")
        p, s, m = torch.ops.act_lib.quant_pack(x, 2, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
        assert p.shape == (24, 16) and s.shape == (4, 6) and s.dtype == torch.float32
        y = torch.ops.act_lib.dequant_unpack_triton(p, s.to(torch.bfloat16), m.to(torch.bfloat16), 2, 256, False, 0)
        assert y.shape == (4, 6, 256) and y.dtype == torch.bfloat16
        X = torch.empty((8, 16, 32, 32), dtype=torch.bfloat16, device="cuda")
        w = torch.empty(16, device="cuda")
        out = torch.ops.act_lib.bn_train_fwd(X, w, w, w, w, 0.1, 512, 2, 2)
        assert out[0].shape == (8, 16, 1024) and out[1].shape == (16, 8 * 1024 * 2 // 32)
