"""The native operators (libdopt_torch.so, csrc/torch_ops.cpp) against the Python implementations
they replace in the dispatcher (act_lib.py, bn_lib.py, which call the same C ABI through ctypes):
every output bit for bit on the same inputs, the in-place running statistics included, and the
same error classes (ValueError for bad bits, RuntimeError for mismatched sizes). The operators'
numerics are pinned against the CPU oracle by the other GPU tests, which now run through these
kernels."""
import os

import pytest
import torch

import deep_optimization_amd  # noqa: F401
from deep_optimization_amd import _lib, _native, act_lib, bn_lib

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(_native.LIB_PATH), reason="libdopt_torch.so not built")]
DEV = "cuda"
ops = torch.ops.act_lib


def same(a, b):
    if isinstance(a, torch.Tensor):
        assert a.dtype == b.dtype and a.shape == b.shape, (a.dtype, b.dtype, a.shape, b.shape)
        assert torch.equal(a.view(torch.uint8) if a.is_floating_point() else a,
                           b.view(torch.uint8) if b.is_floating_point() else b)
    elif isinstance(a, (tuple, list)):
        assert len(a) == len(b)
        for x, y in zip(a, b):
            same(x, y)
    else:
        assert a == b, (a, b)


def rnd(shape, seed, dtype=torch.bfloat16, scale=2.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(dtype)


@pytest.mark.parametrize("rounding", [0, 1, 2])
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_quant_pack_and_dequant(bits, rounding):
    x = rnd((3, 40, 256), bits + 10 * rounding)
    noise = torch.rand((3, 40, 256), generator=torch.Generator(device=DEV).manual_seed(1), device=DEV)
    args = (bits, 256, True, 2.5, True, rounding, noise if rounding == 1 else None, 7, 3, torch.float32)
    got, want = ops.quant_pack(x, *args), act_lib._quant_pack(x, *args)
    same(got, want)
    for dt in (torch.bfloat16, torch.float32):
        same(ops.dequant_unpack(*got, bits, 256, dt), act_lib._dequant_unpack(*got, bits, 256, dt))


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_tile_ops(bits):
    x = rnd((2, 8, 32, 48), bits, dtype=torch.float32)
    args = (bits, 256, False, 0.0, False, 0, None, 0, 0, torch.bfloat16)
    got, want = ops.quant_pack_tiles(x, *args), act_lib._quant_pack_tiles(x, *args)
    same(got, want)
    same(ops.dequant_unpack_tiles(*got, bits, 256, 2, 8, 32, 48, torch.bfloat16),
         act_lib._dequant_unpack_tiles(*got, bits, 256, 2, 8, 32, 48, torch.bfloat16))


@pytest.mark.parametrize("avg_alam,alam_bits", [(False, 0), (True, 2), (True, 4)])
def test_reference_schema_ops(avg_alam, alam_bits):
    x = rnd((4, 12, 256), alam_bits + 3)
    got = ops.quant_pack_triton(x, 2, 256, avg_alam, alam_bits, True, 3.0)
    want = act_lib._quant_pack_triton(x, 2, 256, avg_alam, alam_bits, True, 3.0)
    same(got, want)
    same(ops.dequant_unpack_triton(*got, 2, 256, avg_alam, alam_bits),
         act_lib._dequant_unpack_triton(*got, 2, 256, avg_alam, alam_bits))


@pytest.mark.parametrize("relu6", [False, True])
@pytest.mark.parametrize("bits", [1, 2])
def test_relu_ops(bits, relu6):
    x = rnd((4, 16, 14, 14), bits + 2 * relu6, scale=4.0)
    got = ops.relu_fwd_fused_pack(x, not relu6, relu6, bits, 64)
    want = act_lib._relu_fwd_fused_pack(x, not relu6, relu6, bits, 64)
    same(got, want)
    dy = rnd(x.shape, 9, dtype=torch.float32)
    same(ops.relu_bwd_fused_unpack(got[1], dy, bits, got[2], got[3], 64),
         act_lib._relu_bwd_fused_unpack(got[1], dy, bits, got[2], got[3], 64))


@pytest.mark.parametrize("kind", [_lib.BN_QUANT, _lib.BN_RELU_QUANT, _lib.BN_RELU6_QUANT])
@pytest.mark.parametrize("stats", ["f32", "none", "bf16"])
def test_batchnorm_layer_ops(kind, stats):
    N, C, H, W = 8, 32, 28, 28
    x = rnd((N, C, H, W), kind, scale=1.5)
    w = torch.rand(C, device=DEV) + 0.5
    b = torch.randn(C, device=DEV)
    if stats == "none":
        rm_a = rv_a = rm_b = rv_b = torch.empty(0, device=DEV)
    else:
        dt = torch.float32 if stats == "f32" else torch.bfloat16
        rm_a, rv_a = torch.randn(C, device=DEV).to(dt), (torch.rand(C, device=DEV) + 0.5).to(dt)
        rm_b, rv_b = rm_a.clone(), rv_a.clone()
    got = ops.bn_train_fwd(x, w, b, rm_a, rv_a, 0.1, 256, 2, kind)
    want = bn_lib._bn_train_fwd(x, w, b, rm_b, rv_b, 0.1, 256, 2, kind)
    same(got, want)
    same((rm_a, rv_a), (rm_b, rv_b))
    y, packed, rp, scale, xmin, mean, var = got
    dy = rnd(y.shape, 5)
    relu_packed = rp if kind != _lib.BN_QUANT else None
    same(ops.bn_train_bwd(packed, relu_packed, dy, scale, xmin, w, var, 256, 2, kind),
         bn_lib._bn_train_bwd(packed, relu_packed, dy, scale, xmin, w, var, 256, 2, kind))


def test_error_classes():
    x = torch.zeros(1, 1, 256, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        ops.quant_pack(x, 3, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
    with pytest.raises(ValueError):
        ops.quant_pack_triton(x, 5, 256, False, 0, False, 0.0)
    with pytest.raises(RuntimeError, match="shape"):
        ops.quant_pack(x, 2, 128, False, 0.0, False, 0, None, 0, 0, torch.float32)
    with pytest.raises(RuntimeError, match="noise"):
        ops.quant_pack(x, 2, 256, False, 0.0, False, 1, None, 0, 0, torch.float32)
    with pytest.raises(RuntimeError, match="alam_bits"):
        ops.quant_pack_triton(x, 2, 256, True, 3, False, 0.0)
    p, s, m = ops.quant_pack(x, 2, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
    with pytest.raises(RuntimeError, match="packed holds"):
        ops.dequant_unpack(p[:, :8], s, m, 2, 256, torch.bfloat16)
    with pytest.raises(RuntimeError, match="one per channel"):
        X = torch.zeros(2, 4, 8, 8, device=DEV)
        ops.bn_train_fwd(X, torch.ones(3, device=DEV), torch.zeros(4, device=DEV), torch.empty(0, device=DEV),
                         torch.empty(0, device=DEV), 0.1, 128, 2, _lib.BN_QUANT)
    with pytest.raises(RuntimeError, match="relu"):
        ops.relu_fwd_fused_pack(torch.zeros(2, 64, device=DEV), False, False, 1, 64)
