"""GPU parity of the BatchNorm kernels (statistics, normalize + quant-pack, backward reduce and
input gradient) against the CPU oracle, through the act_lib operators -> the C ABI.

Bar:
  * sums (forward statistics, backward dweight / dbias): fp32 reductions in a fixed order, within
    1e-5 of the sum of the terms' magnitudes (a bound of fp32 summation error) of the float64
    oracle sums;
  * everything downstream of the sums, given the GPU's sums: bit-exact (mean, var, y, x_hat,
    ReLU mask, codes, scale, min, dx), except the squashed mode's codes, which go through tanh
    (libdevice in the reference, ocml here, the C library in the oracle): within one code, and
    different only at elements whose float64 code argument lies within the two tanh evaluations'
    error of a rounding boundary (squash_codes_close); scale and min within one bf16 ulp.
Shapes cover every access width of the kernels (8 elements per access at HW = 256, 784; 4 at
HW = 196; 2 at HW = 50; 1 at HW = 49 and for a misaligned input view), group sizes 32..512
(BLOCK_M 64..1024), bits 1/2/4/8, bf16 / fp32 / fp16 inputs, the sync path, and the squashed
operators' avg_alam mode (runs of 1..64 elements per code, the reduce's tl.rand noise).
"""
import numpy as np
import pytest
import torch

import deep_optimization_amd  # noqa: F401
import oracle
from deep_optimization_amd.fusion import DOBatchNormReLU2d
from deep_optimization_amd.modules.normalization import DOBatchNorm2d

pytestmark = pytest.mark.gpu
DEV = "cuda"
ops = torch.ops.act_lib


def npv(t):
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16,):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float16:
        return t.numpy()
    if t.dtype == torch.int32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def make(shape, dtype, seed, shift=0.5, scale=1.7):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=g) * scale + shift).to(dtype)
    C = shape[1]
    w = torch.rand(C, generator=g) + 0.5
    b = torch.randn(C, generator=g) * 0.3
    return x, w, b


def geo(x):
    N, C = x.shape[0], x.shape[1]
    HW = x.numel() // (N * C)
    return dict(M=N * HW, HW=HW, stride_n=C * HW, stride_c=HW)


def codes_of(packed, bits):
    """codes of a little-endian code bitstream (numpy.unpackbits)"""
    b = np.unpackbits(np.ascontiguousarray(packed).reshape(-1).view(np.uint8), bitorder="little")
    return (b.reshape(-1, bits).astype(np.int64) << np.arange(bits)).sum(axis=1)


def as_f32(a):
    """a numpy view from npv as float32 (bf16 bit patterns widened)"""
    return oracle.bf16_bits_to_f32(a) if a.dtype == np.uint16 else a.astype(np.float32)


def squash_codes_close(x, mean, var, gpu_packed, ref_packed, bits, grp, eps=1e-5):
    """Squashed-mode codes against the oracle's: within one step everywhere, and different only
    where the element's code argument, worked out in float64 from the kernels' fp32
    x_hat = (x - mean) * (1 / sqrt(var + eps)), lies within the two squash evaluations' error of a
    rounding boundary. Each evaluation of 2 tanh(x/2) is within 2e-7 of the exact value (ocml here,
    the C library's tanhf in the oracle; libdevice in the reference), so elements closer than that
    to a boundary may round either way; data with few distinct values can stack many elements on
    one exact tie (the argument at k + 1/2 steps). Returns (ok, message)."""
    cg, cr = codes_of(gpu_packed, bits), codes_of(ref_packed, bits)
    d = np.abs(cg - cr)
    if d.max(initial=0) > 1:
        return False, f"codes {d.max()} apart"
    idx = np.flatnonzero(d)
    if idx.size == 0:
        return True, ""
    xs = np.asarray(as_f32(npv(x)), dtype=np.float32)
    N, C = xs.shape[0], xs.shape[1]
    x3 = xs.reshape(N, C, -1)
    HW = x3.shape[2]
    M = N * HW
    mean32, var32 = as_f32(npv(mean)), as_f32(npv(var))
    inv32 = np.float32(1.0) / np.sqrt(var32 + np.float32(eps))
    qmax = (1 << bits) - 1
    for k in idx:
        c, e = divmod(int(k), M)
        r = e // grp
        es = np.arange(r * grp, (r + 1) * grp)
        xh = ((x3[es // HW, c, es % HW] - mean32[c]) * inv32[c]).astype(np.float64)
        t = 2.0 * np.tanh(np.clip(xh, -3.0, 3.0) / 2.0)
        mn, mx = t.min(), t.max()
        step = (mx - mn) / qmax if mx > mn else 1.0
        arg = (t[e - r * grp] - mn) / step + 0.5
        tol = 6e-7 / step + 1e-4
        if abs(arg - round(arg)) > tol:
            return False, f"code {k} (channel {c}, element {e}) differs {abs(arg - round(arg)):.3g} from a boundary"
    return True, ""


def sums_close(got, want_f64, mag):
    return np.all(np.abs(got.astype(np.float64) - want_f64) <= 1e-5 * mag + 1e-30)


def check_stats(x, s, q):
    rs, rq = oracle.bn_reduce(npv(x))
    xa = np.abs(npv(x).astype(np.float32) if x.dtype != torch.bfloat16 else oracle.bf16_bits_to_f32(npv(x)))
    mag = xa.astype(np.float64).sum(axis=tuple(i for i in range(xa.ndim) if i != 1))
    mag2 = (xa.astype(np.float64) ** 2).sum(axis=tuple(i for i in range(xa.ndim) if i != 1))
    assert sums_close(npv(s), rs, mag)
    assert sums_close(npv(q), rq, mag2)


SHAPES = [(4, 16, 16, 16), (8, 32, 14, 14), (16, 8, 7, 7), (32, 16, 28, 28), (8, 16, 5, 10)]
DTYPES = [torch.bfloat16, torch.float32, torch.float16]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f32", "f16"])
def test_reduce_and_plain_normalize(shape, dtype):
    x, w, b = make(shape, dtype, 1)
    xd = x.to(DEV)
    g = geo(x)
    s, q = ops.bn_fwd_reduce(xd.view(shape[0], shape[1], -1), **g, BLOCK_M=256, num_warps=8, num_stages=5)
    torch.cuda.synchronize()
    check_stats(x, s, q)
    y, xh, mean, var = ops.bn_fwd_norm(xd.view(shape[0], shape[1], -1), s, q, w.to(DEV), b.to(DEV), None, None, **g,
                                       BLOCK_M=256, sync=False, num_warps=8, num_stages=5)
    ref = oracle.bn_norm_quant(npv(x), w.numpy(), b.numpy(), mode=oracle.BN_NORM, eps=1e-7, sum=npv(s),
                               sumsq=npv(q))
    np.testing.assert_array_equal(npv(mean), ref["mean"])
    np.testing.assert_array_equal(npv(var), ref["var"])
    np.testing.assert_array_equal(npv(y).reshape(-1), ref["y"].reshape(-1))
    np.testing.assert_array_equal(npv(xh).reshape(-1), ref["x_hat"].reshape(-1))
    # the plain mode's backward on the saved x_hat, dy in the input's dtype
    dy = torch.randn(shape, generator=torch.Generator().manual_seed(5)).to(dtype)
    dy3 = dy.to(DEV).view(shape[0], shape[1], -1)
    dg, dbt = ops.bn_bwd_reduce(xh, dy3, **g, BLOCK_M=256, num_warps=8, num_stages=5)
    dx = ops.bn_bwd_dx(xh, dy3, var, w.to(DEV), dbt, dg, **g, BLOCK_M=256, sync=False, num_warps=8, num_stages=5)
    torch.cuda.synchronize()
    rdg, rdb = oracle.bn_bwd_reduce(npv(dy), mode=oracle.BN_NORM, x_hat=npv(xh))
    dyf = np.abs(as_f32(npv(dy))).astype(np.float64)
    assert sums_close(npv(dbt), rdb, dyf.sum(axis=(0, 2, 3)))
    xhf = np.abs(as_f32(npv(xh))).astype(np.float64).reshape(dyf.shape)
    assert sums_close(npv(dg), rdg, (dyf * xhf).sum(axis=(0, 2, 3)))
    rdx = oracle.bn_bwd_dx(npv(dy), npv(dg), npv(dbt), w.numpy(), npv(var), mode=oracle.BN_NORM, eps=1e-7,
                           x_hat=npv(xh))
    np.testing.assert_array_equal(npv(dx).reshape(-1), rdx.reshape(-1))


# (shape, BLOCK_M): M = N*HW is a multiple of the group BLOCK_M // 2
QCASES = [((4, 16, 16, 16), 64), ((4, 16, 16, 16), 1024), ((8, 32, 14, 14), 64), ((16, 32, 14, 14), 128),
          ((32, 16, 28, 28), 512), ((32, 8, 7, 7), 64), ((32, 8, 5, 10), 64)]


@pytest.mark.parametrize("case", QCASES, ids=lambda c: "x".join(map(str, c[0])) + f"-B{c[1]}")
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("mode", ["relu", "relu6", "squash"])
@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f32", "f16"])
def test_fused_forward_and_backward(case, bits, mode, dtype):
    """x and dy in one dtype: every (dtype, mode, bits, access width) instance of the four kernels."""
    shape, BLOCK = case
    x, w, b = make(shape, dtype, 100 + bits)
    N, C = shape[0], shape[1]
    g = geo(x)
    x3 = x.to(DEV).view(N, C, -1)
    wd, bd = w.to(DEV), b.to(DEV)
    s, q = ops.bn_fwd_reduce(x3, **g, BLOCK_M=BLOCK, num_warps=8, num_stages=5)
    if mode == "squash":
        y, packed, scale, xmin, mean, var = ops.bn_fwd_norm_quant_pack_fused(
            x3, s, q, wd, bd, None, None, **g, BLOCK_M=BLOCK, bits=bits, sync=False, avg_alam=False, alam_bits=0,
            num_warps=8, num_stages=5)
        rp = None
        omode = oracle.BN_QUANT
    else:
        y, packed, rp, scale, xmin, mean, var = ops.bn_relu_fwd_norm_fused_quant_pack(
            x3, s, q, wd, bd, None, None, **g, relu=mode == "relu", relu6=mode == "relu6", BLOCK_SIZE=BLOCK,
            BITS=bits, sync=False)
        omode = oracle.BN_RELU_QUANT if mode == "relu" else oracle.BN_RELU6_QUANT
    torch.cuda.synchronize()
    check_stats(x, s, q)
    grp = BLOCK // 2
    ref = oracle.bn_norm_quant(npv(x), w.numpy(), b.numpy(), mode=omode, group_size=grp, bits=bits, eps=1e-5,
                               sum=npv(s), sumsq=npv(q))
    np.testing.assert_array_equal(npv(mean), ref["mean"])
    np.testing.assert_array_equal(npv(var), ref["var"])
    np.testing.assert_array_equal(npv(y).reshape(-1), ref["y"].reshape(-1))
    if rp is not None:
        np.testing.assert_array_equal(npv(rp), ref["relu_packed"])
    if mode == "squash":
        ok, msg = squash_codes_close(x, mean, var, npv(packed), ref["packed"], bits, grp)
        assert ok, msg
        for a, r in ((npv(scale), ref["scale"]), (npv(xmin), ref["min"])):
            assert np.abs(a.astype(np.int64) - r.astype(np.int64)).max() <= 1
    else:
        np.testing.assert_array_equal(npv(packed), ref["packed"])
        np.testing.assert_array_equal(npv(scale), ref["scale"])
        np.testing.assert_array_equal(npv(xmin), ref["min"])

    # backward on the GPU's own saved tensors
    gdy = torch.Generator().manual_seed(7)
    dy = torch.randn(shape, generator=gdy).to(dtype)
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
    assert sums_close(npv(db), rdb, dyf.sum(axis=(0, 2, 3)))
    assert sums_close(npv(dw), rdw, 8.0 * dyf.sum(axis=(0, 2, 3)))  # |x_hat'| < 8 for this data
    rdx = oracle.bn_bwd_dx(npv(dy), npv(dw), npv(db), w.numpy(), npv(var), eps=eps, **kw)
    np.testing.assert_array_equal(npv(dx).reshape(-1), rdx.reshape(-1))


@pytest.mark.parametrize("mode", ["plain", "squash", "relu"])
def test_sync_path_bit_exact(mode):
    shape = (8, 16, 14, 14)
    x, w, b = make(shape, torch.bfloat16, 9)
    N, C = shape[0], shape[1]
    g = geo(x)
    gen = torch.Generator().manual_seed(3)
    mean = torch.randn(C, generator=gen) * 0.3
    inv = torch.rand(C, generator=gen) + 0.5
    x3 = x.to(DEV).view(N, C, -1)
    args = (x3, None, None, w.to(DEV), b.to(DEV), mean.to(DEV), inv.to(DEV))
    if mode == "plain":
        y, xh, mo, vo = ops.bn_fwd_norm(*args, **g, BLOCK_M=64, sync=True, num_warps=8, num_stages=5)
        assert mo is None and vo is None
        ref = oracle.bn_norm_quant(npv(x), w.numpy(), b.numpy(), mode=oracle.BN_NORM, mean=mean.numpy(),
                                   invstd=inv.numpy())
        np.testing.assert_array_equal(npv(xh).reshape(-1), ref["x_hat"].reshape(-1))
        # backward with the inverse std in place of the variance
        dy = torch.randn(shape, generator=gen).to(torch.bfloat16)
        dy3 = dy.to(DEV).view(N, C, -1)
        dg, dbt = ops.bn_bwd_reduce(xh, dy3, **g, BLOCK_M=64, num_warps=8, num_stages=5)
        dx = ops.bn_bwd_dx(xh, dy3, inv.to(DEV), w.to(DEV), dbt, dg, **g, BLOCK_M=64, sync=True, num_warps=8,
                           num_stages=5)
        rdx = oracle.bn_bwd_dx(npv(dy), npv(dg), npv(dbt), w.numpy(), inv.numpy(), mode=oracle.BN_NORM,
                               var_is_invstd=True, x_hat=npv(xh))
        np.testing.assert_array_equal(npv(dx).reshape(-1), rdx.reshape(-1))
    elif mode == "squash":
        y, packed, scale, xmin, mo, vo = ops.bn_fwd_norm_quant_pack_fused(
            *args, **g, BLOCK_M=64, bits=2, sync=True, avg_alam=False, alam_bits=0, num_warps=8, num_stages=5)
        ref = oracle.bn_norm_quant(npv(x), w.numpy(), b.numpy(), mode=oracle.BN_QUANT, group_size=32, bits=2,
                                   mean=mean.numpy(), invstd=inv.numpy())
    else:
        y, packed, rp, scale, xmin, mo, vo = ops.bn_relu_fwd_norm_fused_quant_pack(
            *args, **g, relu=True, relu6=False, BLOCK_SIZE=64, BITS=2, sync=True)
        ref = oracle.bn_norm_quant(npv(x), w.numpy(), b.numpy(), mode=oracle.BN_RELU_QUANT, group_size=32, bits=2,
                                   mean=mean.numpy(), invstd=inv.numpy())
        np.testing.assert_array_equal(npv(packed), ref["packed"])
        np.testing.assert_array_equal(npv(rp), ref["relu_packed"])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(npv(y).reshape(-1), ref["y"].reshape(-1))


def test_errors():
    x = torch.randn(2, 4, 10, 10, device=DEV).to(torch.bfloat16)
    x3 = x.view(2, 4, 100)
    g = geo(x)
    s, q = ops.bn_fwd_reduce(x3, **g, BLOCK_M=64, num_warps=8, num_stages=5)
    w = torch.ones(4, device=DEV)
    with pytest.raises(RuntimeError, match="group_size == 0"):  # M = 200 is not a multiple of 32
        ops.bn_fwd_norm_quant_pack_fused(x3, s, q, w, w, None, None, **g, BLOCK_M=64, bits=2, sync=False,
                                         avg_alam=False, alam_bits=0, num_warps=8, num_stages=5)
    with pytest.raises(ValueError):
        ops.bn_relu_fwd_norm_fused_quant_pack(x3, s, q, w, w, None, None, **g, relu=True, relu6=False, BLOCK_SIZE=64,
                                              BITS=3, sync=False)
    with pytest.raises(RuntimeError, match="alam_bits"):  # 2-bit groups of 32 have 2 code words: 4 runs cannot fill them
        ops.bn_fwd_norm_quant_pack_fused(x3, s, q, w, w, None, None, **g, BLOCK_M=64, bits=2, sync=False,
                                         avg_alam=True, alam_bits=4, num_warps=8, num_stages=5)


# ----------------------------------------------------------------------------- avg_alam
# (shape, BLOCK_M, bits, alam_bits): run lengths dividing the group's code words (1: the plain
# codes, noise in the reduce only; 16 and 64: runs spanning 2 and 8 lanes), every access width
# (8 at 16x16 / 28x28, 4 at 14x14, 2 at 5x10, 1 at 7x7), groups of 32..256, and channels whose last
# wave of 512 elements lies partly past M (7x7: M = 1568); each in bf16, fp32 and fp16
ACASES = [((4, 16, 16, 16), 64, 2, 2), ((4, 16, 16, 16), 64, 8, 8), ((16, 8, 14, 14), 128, 1, 2),
          ((16, 32, 14, 14), 128, 4, 4), ((32, 16, 28, 28), 512, 2, 16), ((32, 16, 28, 28), 512, 8, 64),
          ((32, 8, 7, 7), 64, 4, 4), ((32, 8, 5, 10), 64, 2, 1), ((32, 8, 5, 10), 64, 4, 2),
          ((16, 16, 28, 28), 256, 1, 4)]


@pytest.mark.parametrize("case", ACASES, ids=lambda c: "x".join(map(str, c[0])) + f"-B{c[1]}-b{c[2]}-A{c[3]}")
@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "f32", "f16"])
def test_alam_forward_and_backward(case, dtype):
    """avg_alam=True through the reference's three squashed operators against the oracle, x and dy
    in one dtype: y, mean and var bit for bit; codes (runs' truncated means of tanh-squashed
    arguments) within one step on under 1% of the runs, scale / min within one bf16 ulp; the reduce
    (codes plus tl.rand noise) within the fp32 summation bound; dx on the GPU's codes bit for bit."""
    shape, BLOCK, bits, alam = case
    x, w, b = make(shape, dtype, 300 + bits + alam)
    N, C = shape[0], shape[1]
    g = geo(x)
    x3 = x.to(DEV).view(N, C, -1)
    wd, bd = w.to(DEV), b.to(DEV)
    s, q = ops.bn_fwd_reduce(x3, **g, BLOCK_M=BLOCK, num_warps=8, num_stages=5)
    y, packed, scale, xmin, mean, var = ops.bn_fwd_norm_quant_pack_fused(
        x3, s, q, wd, bd, None, None, **g, BLOCK_M=BLOCK, bits=bits, sync=False, avg_alam=True, alam_bits=alam,
        num_warps=8, num_stages=5)
    torch.cuda.synchronize()
    grp = BLOCK // 2
    M = g["M"]
    assert tuple(packed.shape) == (C, M * bits // 32 // alam)
    ref = oracle.bn_norm_quant(npv(x), w.numpy(), b.numpy(), mode=oracle.BN_QUANT, group_size=grp, bits=bits,
                               eps=1e-5, sum=npv(s), sumsq=npv(q), alam_bits=alam)
    np.testing.assert_array_equal(npv(mean), ref["mean"])
    np.testing.assert_array_equal(npv(var), ref["var"])
    np.testing.assert_array_equal(npv(y).reshape(-1), ref["y"].reshape(-1))
    d = np.abs(codes_of(npv(packed), bits) - codes_of(ref["packed"], bits))
    assert d.max() <= 1 and (d > 0).mean() < 0.01
    for a, r in ((npv(scale), ref["scale"]), (npv(xmin), ref["min"])):
        assert np.abs(a.astype(np.int64) - r.astype(np.int64)).max() <= 1

    dy = torch.randn(shape, generator=torch.Generator().manual_seed(8)).to(dtype)
    dy3 = dy.to(DEV).view(N, C, -1)
    dw, db = ops.bn_bwd_reduce_dequant_unpack_fused(packed, dy3, scale, xmin, **g, BLOCK_M=BLOCK, bits=bits,
                                                    avg_alam=True, alam_bits=alam)
    dx = ops.bn_bwd_dx_dequant_unpack_fused(packed, dy3, scale, xmin, dw, db, wd, var, **g, BLOCK_M=BLOCK,
                                            bits=bits, sync=False, avg_alam=True, alam_bits=alam)
    torch.cuda.synchronize()
    kw = dict(mode=oracle.BN_QUANT, packed=npv(packed), scale=npv(scale), min=npv(xmin), group_size=grp, bits=bits,
              alam_bits=alam)
    rdw, rdb = oracle.bn_bwd_reduce(npv(dy), **kw)
    dyf = np.abs(as_f32(npv(dy))).astype(np.float64)
    assert sums_close(npv(db), rdb, dyf.sum(axis=(0, 2, 3)))
    assert sums_close(npv(dw), rdw, 8.0 * dyf.sum(axis=(0, 2, 3)))  # |x_hat'| < 8 for this data
    rdx = oracle.bn_bwd_dx(npv(dy), npv(dw), npv(db), w.numpy(), npv(var), eps=1e-7, **kw)
    np.testing.assert_array_equal(npv(dx).reshape(-1), rdx.reshape(-1))


# ----------------------------------------------------------------------------- layers
def _layer_case(layer_cls, shape, BLOCK, act_padding=False, **kw):
    torch.manual_seed(11)
    C = shape[1]
    meta = {"bn": {"group_size": BLOCK, "bits": 2, "act_padding": act_padding, "AVG_ALAM": False, "ALAM_BITS": 0,
                   "pack_only": False, "N": C, "DIVISION": None}}
    layer = layer_cls(C, target_name="bn", meta=meta, **kw).to(DEV).train()
    ref = torch.nn.BatchNorm2d(C).to(DEV).train()
    with torch.no_grad():
        layer.weight.uniform_(0.5, 1.5)
        layer.bias.uniform_(-0.5, 0.5)
        ref.load_state_dict(layer.state_dict())
    x = (torch.randn(shape, device=DEV) * 1.5 + 0.3).requires_grad_(True)
    return layer, ref, x, meta


@pytest.mark.parametrize("act_padding", [False, True])
def test_do_batchnorm2d_layer(act_padding):
    shape = (8, 16, 28, 28)
    layer, ref, x, meta = _layer_case(DOBatchNorm2d, shape, 256, act_padding)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = layer(x)
    yr = ref(x.detach().float().requires_grad_(True))
    assert y.dtype == torch.bfloat16
    torch.testing.assert_close(y.float(), yr, rtol=2 ** -7, atol=2e-2)
    # running statistics: the reference's update with the biased batch variance
    xd = x.detach().double()
    var_b = xd.var(dim=(0, 2, 3), unbiased=False)
    torch.testing.assert_close(layer.running_mean.double(), 0.1 * xd.mean(dim=(0, 2, 3)), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(layer.running_var.double(), 0.9 + 0.1 * var_b, rtol=1e-5, atol=1e-6)
    assert int(layer.num_batches_tracked) == 1
    dy = torch.randn_like(y)
    y.backward(dy)
    assert layer.weight.grad.dtype == torch.float32 and torch.isfinite(x.grad).all()
    # the gradient follows the saved, squashed and quantized x_hat: close to exact BN's in direction
    xr = x.detach().float().requires_grad_(True)
    ref.zero_grad()
    ref(xr).backward(dy.float())
    cos = torch.nn.functional.cosine_similarity(x.grad.float().flatten(), xr.grad.flatten(), dim=0)
    assert cos > 0.9, float(cos)
    torch.testing.assert_close(layer.bias.grad, ref.bias.grad, rtol=1e-3, atol=1e-3)


def test_do_batchnorm2d_layer_avg_alam():
    """The layer with the per-layer meta AVG_ALAM (the Controller sets it from its config for
    BatchNorm layers, controller.py:179-187): the reference's operator path with runs of 2."""
    shape = (8, 16, 28, 28)
    layer, ref, x, meta = _layer_case(DOBatchNorm2d, shape, 256)
    meta["bn"].update({"AVG_ALAM": True, "ALAM_BITS": 2})
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = layer(x)
    yr = ref(x.detach().float().requires_grad_(True))
    torch.testing.assert_close(y.float(), yr, rtol=2 ** -7, atol=2e-2)
    torch.testing.assert_close(layer.running_mean, ref.running_mean, rtol=1e-5, atol=1e-6)
    dy = torch.randn_like(y)
    y.backward(dy)
    assert torch.isfinite(x.grad).all() and torch.isfinite(layer.weight.grad).all()
    xr = x.detach().float().requires_grad_(True)
    ref.zero_grad()
    ref(xr).backward(dy.float())
    cos = torch.nn.functional.cosine_similarity(x.grad.float().flatten(), xr.grad.flatten(), dim=0)
    assert cos > 0.9, float(cos)
    torch.testing.assert_close(layer.bias.grad, ref.bias.grad, rtol=1e-3, atol=1e-3)


def test_do_batchnorm_relu_layer():
    shape = (8, 16, 28, 28)
    layer, ref, x, meta = _layer_case(DOBatchNormReLU2d, shape, 256)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = layer(x)
    yr = torch.relu(ref(x.detach().float()))
    torch.testing.assert_close(y.float(), yr, rtol=2 ** -7, atol=2e-2)
    dy = torch.randn_like(y)
    y.backward(dy)
    xr = x.detach().float().requires_grad_(True)
    ref.zero_grad()
    torch.relu(ref(xr)).backward(dy.float())
    cos = torch.nn.functional.cosine_similarity(x.grad.float().flatten(), xr.grad.flatten(), dim=0)
    assert cos > 0.9, float(cos)
    # dbias = sum(dy * mask) exactly as autograd's (the mask is y > 0 on the same fp32 y)
    torch.testing.assert_close(layer.bias.grad, ref.bias.grad, rtol=1e-3, atol=1e-2)


@pytest.mark.parametrize("mode", ["squash", "relu"])
def test_misaligned_input_view_matches_aligned(mode):
    """An input view one element past an aligned base (HW = 784 would take 16-byte accesses) runs
    the element-wise access path: outputs equal the aligned run's bit for bit, forward and
    backward."""
    shape, BLOCK, bits = (8, 16, 28, 28), 256, 2
    N, C = shape[0], shape[1]
    HW = shape[2] * shape[3]
    x, w, b = make(shape, torch.bfloat16, 21)
    g = dict(M=N * HW, HW=HW, stride_n=C * HW, stride_c=HW)
    base = torch.zeros(x.numel() + 1, dtype=torch.bfloat16, device=DEV)
    base[1:].copy_(x.reshape(-1).to(DEV))
    outs = []
    for xd in (x.to(DEV).view(N, C, HW), base[1:].view(N, C, HW)):
        assert xd.data_ptr() % 16 == (2 if xd.storage_offset() else 0)
        s, q = ops.bn_fwd_reduce(xd, **g, BLOCK_M=BLOCK, num_warps=8, num_stages=5)
        if mode == "squash":
            y, packed, scale, mn, mean, var = ops.bn_fwd_norm_quant_pack_fused(
                xd, s, q, w.to(DEV), b.to(DEV), None, None, **g, BLOCK_M=BLOCK, bits=bits, sync=False, avg_alam=False,
                alam_bits=0, num_warps=8, num_stages=5)
            rp = None
        else:
            y, packed, rp, scale, mn, mean, var = ops.bn_relu_fwd_norm_fused_quant_pack(
                xd, s, q, w.to(DEV), b.to(DEV), None, None, **g, relu=True, relu6=False, BLOCK_SIZE=BLOCK, BITS=bits,
                sync=False)
        dyf = torch.zeros(x.numel() + 1, dtype=torch.bfloat16, device=DEV)
        dyf[1:].copy_(torch.randn(x.numel(), generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV))
        dy = dyf[1:].view(N, C, HW) if xd.storage_offset() else dyf[1:].clone().view(N, C, HW)
        if mode == "squash":
            dw, db = ops.bn_bwd_reduce_dequant_unpack_fused(packed, dy, scale, mn, **g, BLOCK_M=BLOCK, bits=bits,
                                                            avg_alam=False, alam_bits=0)
            dx = ops.bn_bwd_dx_dequant_unpack_fused(packed, dy, scale, mn, dw, db, w.to(DEV), var, **g, BLOCK_M=BLOCK,
                                                    bits=bits, sync=False, avg_alam=False, alam_bits=0)
        else:
            dw, db = ops.bn_relu_bwd_reduce_fused_dequant_unpack(packed, rp, dy, scale, mn, **g, BLOCK_SIZE=BLOCK,
                                                                 BITS=bits)
            dx = ops.bn_relu_bwd_dx_fused_dequant_unpack(packed, rp, dy, dw, db, w.to(DEV), var, scale, mn, **g,
                                                         BLOCK_SIZE=BLOCK, BITS=bits)
        outs.append([t for t in (s, q, y, packed, rp, scale, mn, mean, var, dw, db, dx) if t is not None])
    for a, b_ in zip(*outs):
        assert torch.equal(a.cpu(), b_.cpu())


def test_forward_rejects_short_per_channel_vectors():
    """weight / bias / sums with fewer values than channels raise before a kernel reads past them."""
    shape = (4, 16, 16, 16)
    x, w, b = make(shape, torch.bfloat16, 3)
    g = geo(x)
    xd = x.to(DEV).view(shape[0], shape[1], -1)
    s, q = ops.bn_fwd_reduce(xd, **g, BLOCK_M=256, num_warps=8, num_stages=5)
    with pytest.raises(RuntimeError, match="one per channel"):
        ops.bn_fwd_norm_quant_pack_fused(xd, s, q, w[:8].to(DEV), b.to(DEV), None, None, **g, BLOCK_M=256, bits=2,
                                         sync=False, avg_alam=False, alam_bits=0, num_warps=8, num_stages=5)
    with pytest.raises(RuntimeError, match="one per channel"):
        ops.bn_fwd_norm(xd, s[:8], q, w.to(DEV), b.to(DEV), None, None, **g, BLOCK_M=256, sync=False, num_warps=8,
                        num_stages=5)


@pytest.mark.parametrize("mode", ["squash", "relu", "relu6"])
@pytest.mark.parametrize("shape,BLOCK", [((8, 16, 28, 28), 256), ((16, 32, 14, 14), 64)],
                         ids=["8x16x28x28", "16x32x14x14"])
def test_layer_operators_equal_the_reference_operator_pairs(mode, shape, BLOCK):
    """act_lib::bn_train_fwd / bn_train_bwd (one call per pass, running statistics updated in the
    normalize kernel) give bit for bit what the reference's operator pairs give, and the running
    statistics of the torch update (mul_(1 - m).add_(stat, alpha=m)) within one fp32 rounding."""
    from deep_optimization_amd import _lib
    bits, mom = 2, 0.1
    N, C = shape[0], shape[1]
    x, w, b = make(shape, torch.bfloat16, 31)
    g = geo(x)
    xd = x.to(DEV).view(N, C, -1)
    wd, bd = w.to(DEV), b.to(DEV)
    dy = torch.randn(xd.shape, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(DEV)
    rm0 = torch.randn(C, device=DEV)
    rv0 = torch.rand(C, device=DEV) + 0.5
    # the reference operator pairs
    s, q = ops.bn_fwd_reduce(xd, **g, BLOCK_M=BLOCK, num_warps=8, num_stages=5)
    if mode == "squash":
        y, packed, scale, mn, mean, var = ops.bn_fwd_norm_quant_pack_fused(
            xd, s, q, wd, bd, None, None, **g, BLOCK_M=BLOCK, bits=bits, sync=False, avg_alam=False, alam_bits=0,
            num_warps=8, num_stages=5)
        rp = None
        dw, db = ops.bn_bwd_reduce_dequant_unpack_fused(packed, dy, scale, mn, **g, BLOCK_M=BLOCK, bits=bits,
                                                        avg_alam=False, alam_bits=0)
        dx = ops.bn_bwd_dx_dequant_unpack_fused(packed, dy, scale, mn, dw, db, wd, var, **g, BLOCK_M=BLOCK, bits=bits,
                                                sync=False, avg_alam=False, alam_bits=0)
        lmode = _lib.BN_QUANT
    else:
        relu6 = mode == "relu6"
        y, packed, rp, scale, mn, mean, var = ops.bn_relu_fwd_norm_fused_quant_pack(
            xd, s, q, wd, bd, None, None, **g, relu=not relu6, relu6=relu6, BLOCK_SIZE=BLOCK, BITS=bits, sync=False)
        dw, db = ops.bn_relu_bwd_reduce_fused_dequant_unpack(packed, rp, dy, scale, mn, **g, BLOCK_SIZE=BLOCK, BITS=bits)
        dx = ops.bn_relu_bwd_dx_fused_dequant_unpack(packed, rp, dy, dw, db, wd, var, scale, mn, **g, BLOCK_SIZE=BLOCK,
                                                     BITS=bits)
        lmode = _lib.BN_RELU6_QUANT if relu6 else _lib.BN_RELU_QUANT
    # the layer operators
    rm, rv = rm0.clone(), rv0.clone()
    y2, packed2, rp2, scale2, mn2, mean2, var2 = ops.bn_train_fwd(xd, wd, bd, rm, rv, mom, BLOCK, bits, lmode)
    dx2, dw2, db2 = ops.bn_train_bwd(packed2, rp2, dy, scale2, mn2, wd, var2, BLOCK, bits, lmode)
    assert (rp is None) == (rp2.numel() == 0)
    for a, b_ in ((y, y2), (packed, packed2), (rp, rp2), (scale, scale2), (mn, mn2), (mean, mean2), (var, var2),
                  (dw, dw2), (db, db2), (dx, dx2)):
        if a is not None:
            assert torch.equal(a, b_)
    ref_m = rm0.clone().mul_(1.0 - mom).add_(mean, alpha=mom)
    ref_v = rv0.clone().mul_(1.0 - mom).add_(var, alpha=mom)
    torch.testing.assert_close(rm, ref_m, rtol=2 ** -23, atol=1e-7)
    torch.testing.assert_close(rv, ref_v, rtol=2 ** -23, atol=1e-7)


def test_layer_operator_opcheck():
    from deep_optimization_amd import _lib
    shape, BLOCK = (4, 16, 16, 16), 256
    x, w, b = make(shape, torch.bfloat16, 2)
    xd = x.to(DEV).view(4, 16, -1)
    rm, rv = torch.zeros(16, device=DEV), torch.ones(16, device=DEV)
    tests = ("test_schema", "test_faketensor", "test_aot_dispatch_static", "test_aot_dispatch_dynamic")
    torch.library.opcheck(ops.bn_train_fwd.default, (xd, w.to(DEV), b.to(DEV), rm, rv, 0.1, BLOCK, 2, _lib.BN_QUANT),
                          test_utils=tests)
    y, packed, rp, scale, mn, mean, var = ops.bn_train_fwd(xd, w.to(DEV), b.to(DEV), rm, rv, 0.1, BLOCK, 2,
                                                           _lib.BN_RELU_QUANT)
    dy = torch.randn(xd.shape, device=DEV).to(torch.bfloat16)
    torch.library.opcheck(ops.bn_train_bwd.default, (packed, rp, dy, scale, mn, w.to(DEV), var, BLOCK, 2,
                                                     _lib.BN_RELU_QUANT), test_utils=tests)


def test_alam_operator_opcheck():
    """The squashed operators with avg_alam: fake kernels give the [C, M*bits/32/alam_bits] codes."""
    shape, BLOCK = (4, 16, 16, 16), 256
    x, w, b = make(shape, torch.bfloat16, 3)
    xd = x.to(DEV).view(4, 16, -1)
    g = geo(x)
    tests = ("test_schema", "test_faketensor", "test_aot_dispatch_static", "test_aot_dispatch_dynamic")
    s, q = ops.bn_fwd_reduce(xd, **g, BLOCK_M=BLOCK, num_warps=8, num_stages=5)
    kw = dict(**g, BLOCK_M=BLOCK, bits=2, sync=False, avg_alam=True, alam_bits=4, num_warps=8, num_stages=5)
    torch.library.opcheck(ops.bn_fwd_norm_quant_pack_fused.default, (xd, s, q, w.to(DEV), b.to(DEV), None, None),
                          kw, test_utils=tests)
    y, packed, scale, mn, mean, var = ops.bn_fwd_norm_quant_pack_fused(xd, s, q, w.to(DEV), b.to(DEV), None, None,
                                                                       **kw)
    dy = torch.randn(xd.shape, device=DEV).to(torch.bfloat16)
    bk = dict(**g, BLOCK_M=BLOCK, bits=2, avg_alam=True, alam_bits=4)
    torch.library.opcheck(ops.bn_bwd_reduce_dequant_unpack_fused.default, (packed, dy, scale, mn), bk,
                          test_utils=tests)
    dw, db = ops.bn_bwd_reduce_dequant_unpack_fused(packed, dy, scale, mn, **bk)
    torch.library.opcheck(ops.bn_bwd_dx_dequant_unpack_fused.default, (packed, dy, scale, mn, dw, db, w.to(DEV), var),
                          dict(bk, sync=False), test_utils=tests)
