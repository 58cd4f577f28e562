"""Randomised parity sweep: the GPU operators against the oracle, bit for bit, over random draws of
input dtype, bits, group size, rounding (nearest, a noise tensor with the 1 - 2^-24 edge value,
Philox with 40-bit seeds and offsets), clamp, scale/min dtype, output dtype, flat and spatial-tile
layouts, ragged shapes, and inputs with NaN, +-inf and signed zeros; also the host plumbing
(unified_quantize -> unified_dequantize without the squash, against the CPU grouping + the
oracle, 2-D / 3-D / 4-D, with and without act_padding), the ReLU mask pack / unpack, the PACT clamp
and code pack / unpack; and the BatchNorm normalize + quant-pack and its backward (ReLU, ReLU6
and squashed modes, random N, C, H, W with N*HW a multiple of the group) to the bar of
tests/test_gpu_bn.py: sums within an fp32 summation bound, everything downstream of them bit for
bit, the squashed mode's codes within one step and different only at near-ties of the float64
code argument; and the fused GELU / SiLU forward and backward on continuous data to the bar of
tests/test_gpu_act.py; and the weight-gradient GEMM (bf16 and packed operands, ragged K) to the bar of
tests/test_gpu_dw.py; and the FP8 GEMM (random shapes, padded strides, a sentinel around C) to the bar
of tests/test_gpu_parity.py; and the ALAM quantizer and its dequantization. Fixed seeds; each case
that differs is reported by its parameters.
"""
import random

import numpy as np
import pytest
import torch

import deep_optimization_amd  # noqa: F401
import oracle
from deep_optimization_amd import _lib
from deep_optimization_amd.modules import module_utils as mu
from deep_optimization_amd.modules import tensor_act_reshape_utils as tr
from tests.test_gpu_act import _check_act_quant
from tests.test_gpu_bn import as_f32, check_stats, geo, npv, squash_codes_close, sums_close
from tests.test_gpu_dw import check_close as dw_check_close
from tests.test_gpu_dw import operands as dw_operands
from tests.test_gpu_parity import ROUNDINGS, assert_quant_equal, np_view

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
rng = random.Random(0)
_big = [1]


def big():
    return _big[0]


def rand_x(shape, dtype):
    gen = torch.Generator().manual_seed(rng.randrange(1 << 30))
    x = torch.randn(shape, generator=gen)
    k = rng.random()
    if k < 0.15:
        x = x * 1e-3
    elif k < 0.25:
        x = x * 300
    elif k < 0.35:
        x = torch.round(x * 4) / 4
    elif k < 0.40:
        x = torch.full(shape, 1.5)
    elif k < 0.50:
        x = x * torch.exp(torch.randn(shape[:-1] + (1,), generator=gen) * 3)
    if rng.random() < 0.15:
        flat = x.view(-1)
        for v in (float("nan"), float("inf"), -float("inf"), -0.0, 0.0):
            flat[rng.randrange(flat.numel())] = v
    return x.to(dtype)


def rounding_args(ng, g):
    r = rng.choice(["nearest", "noise", "philox"])
    noise = torch.rand(ng * g, generator=torch.Generator().manual_seed(rng.randrange(1 << 30))) if r == "noise" else None
    if noise is not None and rng.random() < 0.2:
        noise[rng.randrange(noise.numel())] = 1.0 - 2.0 ** -24
    seed = rng.randrange(1 << 40) if r == "philox" else 0
    offset = rng.randrange(1 << 40) if r == "philox" else 0
    return r, noise, seed, offset


def case_flat():
    dt = rng.choice(DTYPES)
    bits = rng.choice([1, 2, 4, 8])
    g = rng.choice([64, 128, 256, 512, 1024])
    N, G = rng.randint(1, 5), rng.randint(1, 40 * big())
    x = rand_x((N, G, g), dt)
    r, noise, seed, offset = rounding_args(N * G, g)
    clamp = rng.random() < 0.3
    alpha = rng.choice([0.5, 3.0, 1e-3]) if clamp else 0.0
    sdt = rng.choice([torch.float32, torch.bfloat16])
    name = f"flat {dt} b{bits} g{g} N{N} G{G} {r} clamp{clamp}/{alpha} {sdt}"
    p, s, m = torch.ops.act_lib.quant_pack(x.to(DEV), bits, g, clamp, alpha, False, ROUNDINGS[r],
                                           None if noise is None else noise.to(DEV), seed, offset, sdt)
    ref = oracle.quant_pack(np_view(x).reshape(-1, g), g, bits, rounding=ROUNDINGS[r],
                            noise=None if noise is None else noise.numpy(), seed=seed, offset=offset,
                            flags=oracle.FLAG_CLAMP if clamp else 0, clamp_alpha=alpha,
                            meta_dtype=oracle.F32 if sdt == torch.float32 else oracle.BF16)
    assert_quant_equal((p, s, m), ref, name)
    ydt = rng.choice([torch.float32, torch.bfloat16])
    y = torch.ops.act_lib.dequant_unpack(p, s, m, bits, g, ydt)
    yo = oracle.dequant_unpack(*ref, g, bits, y_dtype=oracle.F32 if ydt == torch.float32 else oracle.BF16)
    np.testing.assert_array_equal(np_view(y).reshape(yo.shape), yo, err_msg=f"dequant {name} {ydt}")
    return name


def case_tile():
    dt = rng.choice([torch.float32, torch.bfloat16, torch.float16])
    bits = rng.choice([1, 2, 4, 8])
    g = rng.choice([64, 256, 1024])
    s_ = int(round(g ** 0.5))
    shape = (rng.randint(1, 3), rng.randint(1, 6 * big()), s_ * rng.randint(1, 4), s_ * rng.randint(1, 4))
    x = rand_x(shape, dt)
    ng = shape[0] * shape[1] * (shape[2] // s_) * (shape[3] // s_)
    r, noise, seed, offset = rounding_args(ng, g)
    sdt = rng.choice([torch.float32, torch.bfloat16])
    name = f"tile {dt} b{bits} g{g} {shape} {r} {sdt}"
    p, s, m = torch.ops.act_lib.quant_pack_tiles(x.to(DEV), bits, g, False, 0.0, False, ROUNDINGS[r],
                                                 None if noise is None else noise.to(DEV), seed, offset, sdt)
    ref = oracle.quant_pack(np_view(x), g, bits, tile_nchw=shape, rounding=ROUNDINGS[r],
                            noise=None if noise is None else noise.numpy(), seed=seed, offset=offset,
                            meta_dtype=oracle.F32 if sdt == torch.float32 else oracle.BF16)
    assert_quant_equal((p, s, m), ref, name)
    ydt = rng.choice([torch.float32, torch.bfloat16])
    y = torch.ops.act_lib.dequant_unpack_tiles(p, s, m, bits, g, *shape, ydt)
    yo = oracle.dequant_unpack(*ref, g, bits, tile_nchw=shape, y_dtype=oracle.F32 if ydt == torch.float32 else oracle.BF16)
    np.testing.assert_array_equal(np_view(y), yo, err_msg=f"dequant {name}")
    return name


def case_module():
    """unified_quantize -> unified_dequantize (no squash) against the host grouping on the CPU +
    the oracle, for 2-D / 3-D / 4-D shapes with and without act_padding."""
    bits = rng.choice([1, 2, 4, 8])
    g = rng.choice([64, 128, 256, 512, 1024])
    pad = rng.random() < 0.5
    kind = rng.choice(["2d", "3d", "4d_tile", "4d_flat"])
    if kind == "2d":
        shape = (rng.randint(1, 6), g * rng.randint(1, 5) if not pad else rng.randint(1, 3000))
    elif kind == "3d":
        shape = (rng.randint(1, 4), rng.randint(1, 50), g if not pad else rng.randint(1, 800))
        if not pad:
            shape = (shape[0], shape[1], g * rng.randint(1, 3))
    elif kind == "4d_tile":
        g = rng.choice([64, 256, 1024])
        s_ = int(round(g ** 0.5))
        shape = (rng.randint(1, 3), rng.randint(1, 5), s_ * rng.randint(1, 3), s_ * rng.randint(1, 3))
    else:
        shape = (rng.randint(1, 3), rng.randint(1, 8), 7, 9) if pad else (rng.randint(1, 3), g // 64 * 4, 4, 4)
    x = rand_x(shape, torch.bfloat16)
    meta = {"L": {"bits": bits, "pack_only": False, "group_size": g, "act_padding": pad, "N": shape[0],
                  "AVG_ALAM": False, "ALAM_BITS": 0, "squash": False}}
    clamp = rng.random() < 0.5
    name = f"module {kind} {shape} b{bits} g{g} pad{pad} clamp{clamp}"
    try:
        groups, N, G, nh, nw, ori, pe, re_, cm = tr.spatical_aware_act_tensor_reshape(x, g, pad, False)
    except RuntimeError:
        return name + " (layout rejected on the CPU too)"
    q, qm, _ = mu.unified_quantize(x.to(DEV), None, "L", meta, clamp, 3.0)
    y = mu.unified_dequantize(q, qm, None)
    ref = oracle.quant_pack(np_view(groups.contiguous()).reshape(-1, g), g, bits,
                            flags=oracle.FLAG_CLAMP if clamp else 0, clamp_alpha=3.0, meta_dtype=oracle.BF16)
    yo = oracle.dequant_unpack(*ref, g, bits, y_dtype=oracle.BF16)
    yo_t = torch.from_numpy(yo.view(np.int16)).view(torch.bfloat16).reshape(groups.shape)
    back = tr.spatical_aware_act_tensor_reshape_back(yo_t, ori, g, nh, nw, pad, pe, re_, cm)
    np.testing.assert_array_equal(np_view(y), np_view(back), err_msg=name)
    return name


def case_relu():
    dt = rng.choice([torch.float32, torch.bfloat16])
    bits = rng.choice([1, 2, 4, 8])
    n = 64 * rng.randint(1, 3000 * big())
    relu6 = rng.random() < 0.3
    x = rand_x((n,), dt)
    g = 64
    y, packed, N, G = torch.ops.act_lib.relu_fwd_fused_pack(x.to(DEV).view(1, -1, g), not relu6, relu6, bits, g)
    ry, rp = oracle.relu_pack(np_view(x), bits, relu6)
    name = f"relu {dt} b{bits} n{n} relu6{relu6}"
    np.testing.assert_array_equal(np_view(y).reshape(-1), ry, err_msg=name)
    np.testing.assert_array_equal(np_view(packed).reshape(-1), rp, err_msg=name)
    dyt = rng.choice(DTYPES)
    dy = rand_x((n,), dyt)
    dx = torch.ops.act_lib.relu_bwd_fused_unpack(packed, dy.to(DEV).view(1, -1, g), bits, N, G, g)
    np.testing.assert_array_equal(np_view(dx).reshape(-1), oracle.relu_unpack(rp, np_view(dy), bits), err_msg=name)
    return name


def case_pact():
    dt = rng.choice(DTYPES)
    n = rng.randint(1, 100000 * big())
    alpha = rng.choice([0.25, 1.0, 3.0, 1e-3, float("inf")])
    x = rand_x((n,), dt)
    y, mask = torch.ops.act_lib.group_pact_clamp_fwd(x.to(DEV), alpha)
    ry, rm = oracle.pact_clamp_fwd(np_view(x), alpha)
    name = f"pact {dt} n{n} a{alpha}"
    np.testing.assert_array_equal(np_view(y), ry, err_msg=name)
    np.testing.assert_array_equal(mask.cpu().numpy(), rm, err_msg=name)
    dy = rand_x((n,), rng.choice(DTYPES))
    dx = torch.ops.act_lib.group_pact_clamp_bwd(mask, alpha, dy.to(DEV))
    np.testing.assert_array_equal(np_view(dx), oracle.pact_clamp_bwd(rm, np_view(dy)), err_msg=name)
    return name


def case_codes():
    bits = rng.choice([1, 2, 4, 8])
    g = rng.choice([64, 128, 256, 512, 1024])
    ng = rng.randint(1, 500)
    codes = torch.randint(0, 1 << bits, (1, ng, g), generator=torch.Generator().manual_seed(rng.randrange(1 << 30)),
                          dtype=torch.int8) if bits < 8 else \
        torch.randint(0, 128, (1, ng, g), generator=torch.Generator().manual_seed(rng.randrange(1 << 30)), dtype=torch.int8)
    p = torch.ops.act_lib.pack_triton(codes.to(DEV), bits, g)
    name = f"codes b{bits} g{g} ng{ng}"
    np.testing.assert_array_equal(np_view(p), oracle.pack_codes(codes.numpy(), g, bits), err_msg=name)
    back = torch.ops.act_lib.unpack_triton(p, bits, 1, ng, g)
    assert torch.equal(back.cpu(), codes), name
    return name


def case_bn():
    dt = rng.choice(DTYPES)
    bits = rng.choice([1, 2, 4, 8])
    BLOCK = rng.choice([64, 128, 256, 512, 1024])
    grp = BLOCK // 2
    M = grp * rng.randint(1, 6)
    HW = rng.choice([d for d in range(1, min(M, 1024) + 1) if M % d == 0])
    H = rng.choice([d for d in range(1, HW + 1) if HW % d == 0])
    shape = (M // HW, rng.randint(1, 8 * big()), H, HW // H)
    N, C = shape[0], shape[1]
    mode = rng.choice(["relu", "relu6", "squash"])
    gen = torch.Generator().manual_seed(rng.randrange(1 << 30))
    x = (torch.randn(shape, generator=gen) * rng.choice([0.01, 1.7, 50.0]) + rng.choice([0.0, 0.5, -3.0])).to(dt)
    w = torch.rand(C, generator=gen) + 0.5
    b = torch.randn(C, generator=gen) * 0.3
    name = f"bn {dt} {shape} BLOCK{BLOCK} b{bits} {mode}"
    g = geo(x)
    ops = torch.ops.act_lib
    x3 = x.to(DEV).view(N, C, -1)
    wd, bd = w.to(DEV), b.to(DEV)
    s, q = ops.bn_fwd_reduce(x3, **g, BLOCK_M=BLOCK, num_warps=8, num_stages=5)
    if mode == "squash":
        y, packed, scale, xmin, mean, var = ops.bn_fwd_norm_quant_pack_fused(
            x3, s, q, wd, bd, None, None, **g, BLOCK_M=BLOCK, bits=bits, sync=False, avg_alam=False, alam_bits=0,
            num_warps=8, num_stages=5)
        rp, omode = None, oracle.BN_QUANT
    else:
        y, packed, rp, scale, xmin, mean, var = ops.bn_relu_fwd_norm_fused_quant_pack(
            x3, s, q, wd, bd, None, None, **g, relu=mode == "relu", relu6=mode == "relu6", BLOCK_SIZE=BLOCK,
            BITS=bits, sync=False)
        omode = oracle.BN_RELU_QUANT if mode == "relu" else oracle.BN_RELU6_QUANT
    torch.cuda.synchronize()
    check_stats(x, s, q)
    ref = oracle.bn_norm_quant(npv(x), w.numpy(), b.numpy(), mode=omode, group_size=grp, bits=bits, eps=1e-5,
                               sum=npv(s), sumsq=npv(q))
    for what, got, want in (("mean", mean, ref["mean"]), ("var", var, ref["var"]), ("y", y, ref["y"])):
        np.testing.assert_array_equal(npv(got).reshape(-1), want.reshape(-1), err_msg=f"{what} {name}")
    if rp is not None:
        np.testing.assert_array_equal(npv(rp), ref["relu_packed"], err_msg=name)
    if mode == "squash":
        ok, msg = squash_codes_close(x, mean, var, npv(packed), ref["packed"], bits, grp)
        assert ok, f"{name}: {msg}"
        for a, r in ((npv(scale), ref["scale"]), (npv(xmin), ref["min"])):
            assert np.abs(a.astype(np.int64) - r.astype(np.int64)).max() <= 1, name
    else:
        for what, got, want in (("packed", packed, ref["packed"]), ("scale", scale, ref["scale"]),
                                ("min", xmin, ref["min"])):
            np.testing.assert_array_equal(npv(got), want, err_msg=f"{what} {name}")
    dy = torch.randn(shape, generator=gen).to(dt)
    dy3 = dy.to(DEV).view(N, C, -1)
    if mode == "squash":
        dw, db = ops.bn_bwd_reduce_dequant_unpack_fused(packed, dy3, scale, xmin, **g, BLOCK_M=BLOCK, bits=bits,
                                                        avg_alam=False, alam_bits=0)
        dx = ops.bn_bwd_dx_dequant_unpack_fused(packed, dy3, scale, xmin, dw, db, wd, var, **g, BLOCK_M=BLOCK,
                                                bits=bits, sync=False, avg_alam=False, alam_bits=0)
        eps = 1e-7
    else:
        dw, db = ops.bn_relu_bwd_reduce_fused_dequant_unpack(packed, rp, dy3, scale, xmin, **g, BLOCK_SIZE=BLOCK,
                                                             BITS=bits)
        dx = ops.bn_relu_bwd_dx_fused_dequant_unpack(packed, rp, dy3, dw, db, wd, var, scale, xmin, **g,
                                                     BLOCK_SIZE=BLOCK, BITS=bits)
        eps = 1e-5
    torch.cuda.synchronize()
    kw = dict(mode=omode, packed=npv(packed), relu_packed=None if rp is None else npv(rp), scale=npv(scale),
              min=npv(xmin), group_size=grp, bits=bits)
    rdw, rdb = oracle.bn_bwd_reduce(npv(dy), **kw)
    dyf = np.abs(as_f32(npv(dy))).astype(np.float64)
    assert sums_close(npv(db), rdb, dyf.sum(axis=(0, 2, 3))), f"db {name}"
    assert sums_close(npv(dw), rdw, 8.0 * dyf.sum(axis=(0, 2, 3))), f"dw {name}"
    rdx = oracle.bn_bwd_dx(npv(dy), npv(dw), npv(db), w.numpy(), npv(var), eps=eps, **kw)
    np.testing.assert_array_equal(npv(dx).reshape(-1), rdx.reshape(-1), err_msg=f"dx {name}")
    return name


def case_act():
    """Fused GELU / SiLU forward (y and the squashed derivative's codes) on continuous data of at least
    32k elements, to the bar of tests/test_gpu_act.py (values within one bf16 ulp, codes within one
    step on under 1% of the elements: the derivative goes through exp); the backward on the GPU's own
    codes bit for bit. SiLU also in the spatial-tile layout."""
    act = rng.choice(["gelu", "silu"])
    bits = rng.choice([1, 2, 4, 8])
    g = rng.choice([64, 128, 256])
    dt = rng.choice([torch.bfloat16, torch.float32])
    s_ = int(round(g ** 0.5))
    tiles = act == "silu" and s_ * s_ == g and rng.random() < 0.5
    if tiles:
        shape = (rng.randint(2, 4), rng.randint(4, 16), s_ * rng.randint(2, 6), s_ * rng.randint(2, 6))
    else:
        shape = (rng.randint(1, 4), rng.randint(64, 256), g * rng.randint(1, 8))
    while int(np.prod(shape)) < 32768:
        shape = (shape[0] * 2,) + shape[1:]
    gen = torch.Generator().manual_seed(rng.randrange(1 << 30))
    x = (torch.randn(shape, generator=gen) * rng.uniform(0.5, 4.0)).to(dt)
    name = f"{act} {dt} {shape} b{bits} g{g}"
    if act == "gelu":
        y, packed, scale, xmin, N, G = torch.ops.act_lib.gelu_fwd_fused_quan_pack(x.to(DEV), bits, g)
        tile = None
    else:
        y, packed, scale, xmin, N, G, nh, nw, pe, re_ = torch.ops.act_lib.silu_fwd_quan_pack(
            x.to(DEV), bits, g, False, 0, False)
        tile = shape if re_ else None
        assert bool(re_) == tiles, name
    torch.cuda.synchronize()
    xin = np_view(x) if tile else np_view(x).reshape(-1, g)
    ry, rp, rs, rm = oracle.act_quant_pack(xin, oracle.ACT_GELU if act == "gelu" else oracle.ACT_SILU, g, bits,
                                           tile_nchw=tile)
    _check_act_quant((y, packed, scale, xmin), (ry.reshape(-1), rp, rs, rm), g, bits)
    dy = torch.randn(shape, generator=gen).to(rng.choice([torch.bfloat16, torch.float32]))
    if act == "gelu":
        dx = torch.ops.act_lib.gelu_bwd_fused_dequan_unpack(packed, dy.to(DEV), scale, xmin, bits, N, G, g)
    else:
        dx = torch.ops.act_lib.silu_bwd_fused_dequan_unpack(packed, dy.to(DEV), scale, xmin, bits, N, G, g, False,
                                                            nh, nw, pe, re_, False, 0)
    dyn = np_view(dy) if tile else np_view(dy).reshape(-1, g)
    want = oracle.act_dequant_mul(np_view(packed), np_view(scale), np_view(xmin), g, bits, dyn, tile_nchw=tile)
    np.testing.assert_array_equal(np_view(dx).reshape(-1), want.reshape(-1), err_msg=name)
    return name


def case_dw():
    """The weight-gradient GEMM on random M, N (multiples of 256) and ragged K, to the bar of
    tests/test_gpu_dw.py: dW and db within 1e-4 of the sum of the terms' magnitudes of float64
    products, the bf16 output the rounding of the fp32 one, and the packed-code path bit for bit
    equal to the bf16 path fed with the dequantized activation."""
    M, N = 256 * rng.randint(1, 8), 256 * rng.randint(1, 8)
    K = rng.randint(1, 20000)
    bits = rng.choice([1, 2, 4, 8])
    g = rng.choice([g_ for g_ in (64, 128, 256, 512, 1024) if (K * N) % g_ == 0])
    name = f"dw M{M} N{N} K{K} b{bits} g{g}"
    dy, x = dw_operands(K, M, N, rng.randrange(1 << 30))
    ops = torch.ops.act_lib
    packed, scale, xmin = ops.quant_pack_triton(x.reshape(1, -1, g), bits, g, False, 0, True, 3.0)
    x_hat = ops.dequant_unpack_triton(packed, scale, xmin, bits, g, False, 0).reshape(K, N)
    want, wdb = ops.dw_gemm(dy, x_hat, None, None, None, N, 0, 0, True, torch.float32)
    got, gdb = ops.dw_gemm(dy, None, packed, scale, xmin, N, bits, g, True, torch.float32)
    w16, _ = ops.dw_gemm(dy, x_hat, None, None, None, N, 0, 0, False, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(got, want), name
    assert torch.equal(w16, want.to(torch.bfloat16)), name
    dw_check_close(want, dy, x_hat)
    mag = dy.double().abs().sum(0)
    for d in (wdb, gdb):
        assert bool(((d.double() - dy.double().sum(0)).abs() <= 1e-4 * mag + 1e-6).all()), f"db {name}"
    return name


def case_fp8():
    """The FP8 e4m3 GEMM through the C ABI on random M, N, K (K a multiple of 16, a quarter of the
    cases from 8192 up, the 16x16x128 kernel) with padded row strides holding NaN encodings and a
    sentinel around C, to the bar of tests/test_gpu_parity.py: within bf16 rounding (plus 1e-3 of
    the largest magnitude) of the fp32 product of the same e4m3 operands, nothing written outside
    M x N."""
    big_k = rng.random() < 0.25
    M, N = (rng.randint(1, 600), rng.randint(1, 600)) if big_k else (rng.randint(1, 3000), rng.randint(1, 3000))
    K = 16 * (rng.randint(512, 560) if big_k else rng.randint(1, 300))
    lda, ldb, ldc = K + 16 * rng.randint(0, 3), K + 16 * rng.randint(0, 3), N + rng.randint(0, 9)
    gen = torch.Generator(device=DEV).manual_seed(rng.randrange(1 << 30))
    a8 = (torch.randn(M, lda, generator=gen, device=DEV) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    b8 = (torch.randn(N, ldb, generator=gen, device=DEV) * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    a8.view(torch.uint8)[:, K:] = 0x7F
    b8.view(torch.uint8)[:, K:] = 0xFF
    c = torch.full((M + 1, ldc), 77.0, dtype=torch.bfloat16, device=DEV)
    name = f"fp8 M{M} N{N} K{K} lda{lda} ldb{ldb} ldc{ldc}"
    rc = _lib.lib().dopt_fp8_gemm_nt(a8.data_ptr(), b8.data_ptr(), M, N, K, lda, ldb, 1.0 / 1600.0, c.data_ptr(),
                                     ldc, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "fp8_gemm_nt")
    ref = (a8[:, :K].float() @ b8[:, :K].float().t()) / 1600.0
    got = c[:M, :N].float()
    assert bool(torch.isfinite(got).all()), name
    assert bool(((got - ref).abs() <= ref.abs() * 2 ** -7 + 1e-3 * ref.abs().max()).all()), name
    assert bool((c[:M, N:] == 77.0).all()) and bool((c[M:] == 77.0).all()), f"{name}: written outside C"
    return name


def case_alam():
    """The ALAM (avg_alam) quantizer through the C ABI without the squash: codes, scale and min bit
    for bit (runs of alam_bits code arguments summed left to right); its dequantization within one
    bf16 ulp plus 1e-5 of the group's step per element (the Box-Muller noise's log / cos are the C
    library's in the oracle, a few fp32 ulps from the GPU's, which matters where the result cancels
    to near zero)."""
    dt = rng.choice(DTYPES)
    g = rng.choice([64, 128, 256, 512, 1024])
    bits, alam = rng.choice([(b_, a_) for b_ in (1, 2, 4, 8) for a_ in (1, 2, 4, 8) if (g * b_ // 32) % a_ == 0])
    ng = rng.randint(1, 60 * big())
    clamp = rng.random() < 0.3
    x = rand_x((ng, g), dt)
    name = f"alam {dt} g{g} b{bits} A{alam} ng{ng} clamp{clamp}"
    L, st = _lib.lib(), torch.cuda.current_stream().cuda_stream
    xd = x.to(DEV)
    p = torch.empty((ng, g * bits // 32 // alam), dtype=torch.int32, device=DEV)
    s_ = torch.empty(ng, dtype=torch.bfloat16, device=DEV)
    m = torch.empty(ng, dtype=torch.bfloat16, device=DEV)
    code = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}[dt]
    flags = oracle.FLAG_CLAMP if clamp else 0
    rc = L.dopt_alam_quant_pack(xd.data_ptr(), code, ng, g, bits, alam, flags, 2.5, p.data_ptr(), s_.data_ptr(),
                                m.data_ptr(), st)
    assert rc == 0, L.dopt_last_error()
    y = torch.empty((ng, g), dtype=torch.bfloat16, device=DEV)
    rc = L.dopt_alam_dequant_unpack(p.data_ptr(), s_.data_ptr(), m.data_ptr(), ng, g, bits, alam, oracle.ALAM_SEED,
                                    y.data_ptr(), st)
    assert rc == 0, L.dopt_last_error()
    torch.cuda.synchronize()
    rp, rs, rm = oracle.alam_quant_pack(np_view(x), g, bits, alam, flags=flags, clamp_alpha=2.5)
    np.testing.assert_array_equal(np_view(p).view(np.uint32).reshape(rp.shape), rp, err_msg=name)
    np.testing.assert_array_equal(np_view(s_), rs, err_msg=name)
    np.testing.assert_array_equal(np_view(m), rm, err_msg=name)
    yo = oracle.alam_dequant_unpack(rp, rs, rm, g, bits, alam)
    yg = oracle.bf16_bits_to_f32(np_view(y).reshape(-1)).astype(np.float64)
    yr = oracle.bf16_bits_to_f32(yo.reshape(-1)).astype(np.float64)
    step = np.repeat(oracle.bf16_bits_to_f32(rs).astype(np.float64), g)
    # one bf16 ulp, plus the noise's fp32 error (a few ulps of |n| <= ~5, times the step) where
    # q + n - 1/2 and min nearly cancel
    tol = 2.0 ** -7 * np.maximum(np.abs(yg), np.abs(yr)) + 1e-5 * step
    with np.errstate(invalid="ignore"):  # inf - inf where a group's range is infinite
        ok = (yg == yr) | (np.abs(yg - yr) <= tol) | (np.isnan(yg) & np.isnan(yr))
    assert ok.all(), f"{name}: dequant {int((~ok).sum())} values beyond one bf16 ulp + 1e-5 step"
    return name


CASES = [case_flat] * 4 + [case_tile] * 3 + [case_module] * 3 + [case_relu, case_pact, case_codes] + [case_bn] * 2 + [case_act] * 2 + [case_dw, case_fp8, case_alam]


@pytest.mark.parametrize("seed,n,scale", [(101, 3000, 1), (102, 3000, 1), (103, 600, 8)])
def test_random_sweep(seed, n, scale):
    rng.seed(seed)
    _big[0] = scale
    fails = []
    for _ in range(n):
        fn = rng.choice(CASES)
        try:
            fn()
        except AssertionError as e:
            fails.append(f"{fn.__name__}: {str(e)[:400]}")
    assert not fails, f"{len(fails)} of {n} cases differ; first: " + " | ".join(fails[:3])
