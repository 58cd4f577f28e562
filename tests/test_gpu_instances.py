"""GPU parity of the kernel instances the other GPU test files leave unlaunched, through the
operators and the C ABI, against the CPU oracle:

* the quantizer's spatial-tile layout at every (input dtype, bits, square group size, rounding),
  with the unpack to bf16 and to fp32;
* the reference's clamp + squash pre-transform at every (input dtype, bits, group size, rounding),
  flat and tiled;
* the fused GELU / SiLU forward on fp32 and bf16 inputs, flat and tiled, with fp32 and bf16 scale
  and min, and their backward with fp32 and bf16 dy;
* the unfused activation forward (ReLU, ReLU6, GELU, SiLU) on fp32, fp16 and bf16 inputs;
* the packed-operand weight gradient without the bias gradient.

Bars as in the files these extend: bit-exact where the arithmetic is the reference's; the tanh
squash and the GELU / SiLU values are checked against float64 with the tolerances stated at each
check (tests/restate.py, tests/test_gpu_act.py).
"""
import ctypes

import numpy as np
import pytest
import torch

import deep_optimization_amd  # noqa: F401
import oracle
from deep_optimization_amd import _lib
from tests.restate import squash_inputs, squash_mismatch
from tests.test_gpu_act import bf16_close
from tests.test_gpu_parity import (TORCH_TO_ORACLE, assert_quant_equal, gpu_quant, make_input, np_view,
                                   oracle_quant, quant_np)

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = [torch.bfloat16, torch.float32, torch.float16]
DTYPE_IDS = ["bf16", "f32", "f16"]
# per square group size: an [N, C, H, W] whose s x s tiles number a few dozen groups
TILE_SHAPES = {64: (2, 3, 16, 24), 256: (2, 3, 32, 48), 1024: (1, 2, 64, 32)}


def groups_to_nchw(xg, shape, g):
    """The [N, C, H, W] tensor whose tile gather (group (n, c, th, tw) holds x[n, c, th s + i,
    tw s + j] at element i s + j) gives the rows of xg in order."""
    n, c, h, w = shape
    s = int(round(g ** 0.5))
    return xg.reshape(n, c, h // s, w // s, s, s).permute(0, 1, 2, 4, 3, 5).reshape(n, c, h, w).contiguous()


# ----------------------------------------------------------------------------- tile layout
@pytest.mark.parametrize("rounding", ["nearest", "noise", "philox"])
@pytest.mark.parametrize("g", sorted(TILE_SHAPES))
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_tiles_every_instance(dtype, bits, g, rounding):
    shape = TILE_SHAPES[g]
    x = make_input(shape, dtype, seed=bits * 31 + g)
    n_groups = shape[0] * shape[1] * (shape[2] * shape[3] // g)
    noise = torch.rand(n_groups * g, generator=torch.Generator().manual_seed(bits)) if rounding == "noise" else None
    gpu = gpu_quant(x, bits, g, rounding, noise, seed=9, offset=4, tile=True)
    ref = oracle_quant(x, bits, g, rounding, noise, seed=9, offset=4, tile=shape)
    assert_quant_equal(gpu, ref, f"tiles {dtype} b{bits} g{g} {rounding}")
    for out in (torch.bfloat16, torch.float32):
        y = torch.ops.act_lib.dequant_unpack_tiles(*gpu, bits, g, *shape, out)
        yo = oracle.dequant_unpack(*ref, g, bits, tile_nchw=shape, y_dtype=TORCH_TO_ORACLE[out])
        np.testing.assert_array_equal(np_view(y), yo)


# ----------------------------------------------------------------------------- clamp + squash
PRE_CASES = [(g, "flat") for g in (64, 128, 256, 512, 1024)] + [(g, "tiles") for g in sorted(TILE_SHAPES)]
# tile shapes holding the 120 groups of 256 of squash_inputs at each square group size
PRE_TILE_SHAPES = {64: (2, 3, 64, 80), 256: (2, 3, 64, 80), 1024: (2, 3, 32, 160)}


@pytest.mark.parametrize("rounding", ["nearest", "noise", "philox"])
@pytest.mark.parametrize("g,layout", PRE_CASES)
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_pretransform_every_instance(dtype, bits, g, layout, rounding):
    """clamp(x, -3, 3) then tanh(2x)/2 before the quantizer (the reference's live path), against
    the float64 restatement: min within 2 fp32 ulps, scale within what that gives, codes equal
    away from 4-ulp bands around the rounding boundaries (squash_mismatch)."""
    xg = squash_inputs(bits * 7 + g).reshape(-1, g)
    xt = torch.from_numpy(xg).to(dtype)
    xr = xt.float().numpy()  # the values the kernel reads, in group order
    ng = xg.shape[0]
    u = None
    noise = None
    if rounding == "noise":
        u = torch.rand(xg.shape, generator=torch.Generator().manual_seed(g)).numpy()
        noise = torch.from_numpy(u)
    elif rounding == "philox":
        u = oracle.philox_noise(0, ng * g, 21, 6).reshape(ng, g)
    if layout == "tiles":
        x_in = groups_to_nchw(xt, PRE_TILE_SHAPES[g], g)
        noise = None if noise is None else noise.reshape(-1)
    else:
        x_in = xt.view(1, ng, g)
        noise = None if noise is None else noise.view(1, ng, g)
    got = gpu_quant(x_in, bits, g, rounding, noise, seed=21, offset=6, clamp=True, alpha=3.0, squash=True,
                    tile=layout == "tiles")
    assert squash_mismatch(quant_np(got), xr, bits, 3.0, u=u) == []


# ----------------------------------------------------------------------------- fused GELU / SiLU
def act_quant_pack_abi(x, act, g, bits, tile, meta):
    """dopt_act_quant_pack on x (flat groups of g, or the [N, C, H, W] tile layout)."""
    L = _lib.lib()
    ng = x.numel() // g
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=DEV)
    packed = torch.empty((ng, g * bits // 32), dtype=torch.int32, device=DEV)
    scale = torch.empty(ng, dtype=meta, device=DEV)
    xmin = torch.empty(ng, dtype=meta, device=DEV)
    tile_arr = None if tile is None else (ctypes.c_int64 * 4)(*tile)
    code = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
    rc = L.dopt_act_quant_pack(x.data_ptr(), code[x.dtype], act, ng, g, bits, tile_arr, y.data_ptr(),
                               packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), code[meta],
                               torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "act_quant_pack")
    torch.cuda.synchronize()
    return y, packed, scale, xmin


ACT_CASES = [(g, None) for g in (64, 128, 256, 512, 1024)] + [(g, TILE_SHAPES[g]) for g in sorted(TILE_SHAPES)]


@pytest.mark.parametrize("g,tile", ACT_CASES, ids=lambda c: str(c))
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("act", ["gelu", "silu"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_fused_activation_every_instance(dtype, act, bits, g, tile):
    """y within one bf16 ulp (+1e-6) of the oracle; scale and min within 2^-7 relative (+1e-6), the
    bf16 ulp, whether stored as bf16 or fp32 (the derivative they come from goes through the GPU's
    and the C library's exp, which differ by fp32 ulps before the derivative's cancellation); codes
    within one step on under 1% of the elements; the backward with fp32 and bf16 dy on the GPU's own
    codes bit for bit."""
    a = oracle.ACT_GELU if act == "gelu" else oracle.ACT_SILU
    shape = tile if tile is not None else (3, 5, 2 * g)
    x = (torch.randn(shape, generator=torch.Generator().manual_seed(bits + g)) * 2.5).to(dtype)
    meta = torch.float32 if bits % 4 == 0 else torch.bfloat16  # both meta types over the bit widths
    y, packed, scale, xmin = act_quant_pack_abi(x.to(DEV), a, g, bits, tile, meta)
    xin = np_view(x) if tile is not None else np_view(x).reshape(-1, g)
    mo = oracle.F32 if meta == torch.float32 else oracle.BF16
    ry, rp, rs, rm = oracle.act_quant_pack(xin, a, g, bits, tile_nchw=tile, meta_dtype=mo)
    assert bf16_close(np_view(y).reshape(-1), ry.reshape(-1)).all()
    if meta == torch.bfloat16:
        assert bf16_close(np_view(scale), rs).all() and bf16_close(np_view(xmin), rm).all()
    else:
        for got, want in ((np_view(scale), rs), (np_view(xmin), rm)):
            a, b = got.astype(np.float64), want.astype(np.float64)
            assert (np.abs(a - b) <= 2.0 ** -7 * np.maximum(np.abs(a), np.abs(b)) + 1e-6).all()
    cg = oracle.unpack_codes(np_view(packed), g, bits).view(np.uint8).astype(int)
    cr = oracle.unpack_codes(rp, g, bits).view(np.uint8).astype(int)
    assert np.max(np.abs(cg - cr)) <= 1 and np.mean(cg != cr) < 0.01
    for dyt in (torch.float32, torch.bfloat16):
        dy = torch.randn(shape, generator=torch.Generator().manual_seed(3)).to(dyt)
        dx = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
        dyd = dy.to(DEV)
        tile_arr = None if tile is None else (ctypes.c_int64 * 4)(*tile)
        code = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
        rc = _lib.lib().dopt_act_dequant_mul(packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), code[meta],
                                             x.numel() // g, g, bits, tile_arr, dyd.data_ptr(), code[dyt],
                                             dx.data_ptr(), torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "act_dequant_mul")
        torch.cuda.synchronize()
        dyn = np_view(dy) if tile is not None else np_view(dy).reshape(-1, g)
        want = oracle.act_dequant_mul(np_view(packed), np_view(scale), np_view(xmin), g, bits, dyn, tile_nchw=tile)
        np.testing.assert_array_equal(np_view(dx).reshape(-1), want.reshape(-1))


# ----------------------------------------------------------------------------- unfused forward
@pytest.mark.parametrize("act", ["relu", "relu6", "gelu", "silu"])
@pytest.mark.parametrize("dtype", DTYPES, ids=DTYPE_IDS)
def test_unfused_activation_every_dtype(dtype, act):
    """relu_triton / gelu_triton / silu_triton on every input dtype: ReLU(6) values and masks bit
    for bit; GELU / SiLU values and derivatives within one bf16 ulp (+1e-6) of the oracle."""
    x = (torch.randn(4099, generator=torch.Generator().manual_seed(17)) * 4).to(dtype)
    xn = np_view(x)
    if act in ("relu", "relu6"):
        y, mask = torch.ops.act_lib.relu_triton(x.to(DEV), act == "relu", act == "relu6")
        ry, rmask = oracle.act_forward(xn, oracle.ACT_RELU if act == "relu" else oracle.ACT_RELU6)
        np.testing.assert_array_equal(np_view(y), ry)
        np.testing.assert_array_equal(mask.cpu().numpy(), rmask)
    else:
        op = torch.ops.act_lib.gelu_triton if act == "gelu" else torch.ops.act_lib.silu_triton
        y, d = op(x.to(DEV))
        ry, rd = oracle.act_forward(xn, oracle.ACT_GELU if act == "gelu" else oracle.ACT_SILU)
        assert bf16_close(np_view(y), ry).all() and bf16_close(np_view(d), rd).all()


# ----------------------------------------------------------------------------- weight gradient
@pytest.mark.parametrize("bits,g", [(1, 64), (2, 256), (4, 128), (8, 512)])
@pytest.mark.parametrize("M,N", [(768, 768), (2304, 768)], ids=["128-row tiles", "256-row tiles"])
@pytest.mark.parametrize("K", [2048, 2000])
def test_packed_dw_without_bias_gradient(bits, g, M, N, K):
    """dw_gemm on packed codes without the bias gradient equals the same call with it, bit for
    bit (the two are separate kernel instances; 8-bit codes, and K not a multiple of 32, take the
    register-decoding kernel)."""
    gen = torch.Generator().manual_seed(bits + M)
    dy = (torch.randn((K, M), generator=gen) * 0.1).to(torch.bfloat16).to(DEV)
    x = torch.randn((K, N), generator=gen).to(torch.bfloat16).to(DEV)
    ops = torch.ops.act_lib
    packed, scale, xmin = ops.quant_pack_triton(x.reshape(1, -1, g), bits, g, False, 0, True, 3.0)
    want, wdb = ops.dw_gemm(dy, None, packed, scale, xmin, N, bits, g, True, torch.float32)
    got, none = ops.dw_gemm(dy, None, packed, scale, xmin, N, bits, g, False, torch.float32)
    torch.cuda.synchronize()
    assert none is None and wdb is not None
    assert torch.equal(got, want)
