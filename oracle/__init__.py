"""CPU oracle for the activation-compression hot path (TEST INFRASTRUCTURE ONLY).

This package is the checker, never the product: only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import it. The product path (``deep_optimization_amd``)
never imports, links or calls anything under ``oracle/``.

``liboracle.so`` is built from ``dopt_oracle.c`` (a C restatement of the reference quantizer,
Activation_Compression/act_triton_kernel.py:23-433, with the stochastic form of
Activation_Compression/cpp_extension/include/quant_common.h:148-156) by ``oracle/Makefile``.
The wrappers here take and return numpy arrays and mirror the C ABI of ``include/dopt.h``.

Parity status per function is listed in the header of ``dopt_oracle.c``; the squash pre-transform
(tanh) is "parity unpinned" at bit level.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F32, F16, BF16 = 0, 1, 2
NEAREST, STOCH_NOISE, STOCH_PHILOX = 0, 1, 2
FLAG_CLAMP, FLAG_SQUASH = 1, 2
ACT_RELU, ACT_RELU6, ACT_GELU, ACT_SILU = 0, 1, 2, 3

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc + OpenMP)."""
    if force and os.path.exists(_LIB_PATH):
        os.remove(_LIB_PATH)
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i64, i32, u64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint64
        L.oracle_quant_pack.argtypes = [vp, i32, i64, i32, i32, vp, i32, vp, u64, u64, i32,
                                        ctypes.c_float, vp, vp, vp, i32]
        L.oracle_quant_pack.restype = i32
        L.oracle_dequant_unpack.argtypes = [vp, vp, vp, i32, i64, i32, i32, vp, vp, i32]
        L.oracle_dequant_unpack.restype = i32
        L.oracle_pack_codes.argtypes = [vp, i64, i32, i32, vp]
        L.oracle_pack_codes.restype = i32
        L.oracle_unpack_codes.argtypes = [vp, i64, i32, i32, vp]
        L.oracle_unpack_codes.restype = i32
        L.oracle_philox4x32_10.argtypes = [vp, vp, vp]
        L.oracle_philox4x32_10.restype = None
        L.oracle_philox_noise.argtypes = [i64, i64, u64, u64, vp]
        L.oracle_philox_noise.restype = None
        L.oracle_num_threads.restype = i32
        L.oracle_set_num_threads.argtypes = [i32]
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_relu_pack.argtypes = [vp, i32, i64, i32, i32, vp, vp]
        L.oracle_relu_pack.restype = i32
        L.oracle_relu_unpack.argtypes = [vp, vp, i32, i64, i32, vp]
        L.oracle_relu_unpack.restype = i32
        L.oracle_act_forward.argtypes = [vp, i32, i64, i32, vp, vp]
        L.oracle_act_forward.restype = i32
        L.oracle_pact_clamp_fwd.argtypes = [vp, i32, i64, ctypes.c_float, vp, vp]
        L.oracle_pact_clamp_fwd.restype = i32
        L.oracle_pact_clamp_bwd.argtypes = [vp, vp, i32, i64, vp]
        L.oracle_pact_clamp_bwd.restype = i32
        L.oracle_act_quant_pack.argtypes = [vp, i32, i32, i64, i32, i32, vp, vp, vp, vp, vp, i32]
        L.oracle_act_quant_pack.restype = i32
        L.oracle_act_dequant_mul.argtypes = [vp, vp, vp, i32, i64, i32, i32, vp, vp, i32, vp]
        L.oracle_act_dequant_mul.restype = i32
        L.oracle_act_dequant_mul_alam.argtypes = [vp, vp, vp, i32, i64, i32, i32, vp, vp, i32, u64, vp]
        L.oracle_act_dequant_mul_alam.restype = i32
        f32 = ctypes.c_float
        L.oracle_bn_reduce.argtypes = [vp, i32, i64, i64, i64, i64, i64, vp, vp]
        L.oracle_bn_reduce.restype = i32
        L.oracle_bn_norm_quant.argtypes = [vp, i32, i64, i64, i64, i64, i64, vp, vp, vp, vp, i32, vp, vp, f32, i32,
                                           i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, i32]
        L.oracle_bn_norm_quant.restype = i32
        L.oracle_bn_bwd_reduce.argtypes = [i32, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, i32, vp, vp,
                                           i32]
        L.oracle_bn_bwd_reduce.restype = i32
        L.oracle_bn_bwd_dx.argtypes = [i32, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, i32, vp, vp,
                                       vp, vp, f32, i32, vp, i32]
        L.oracle_bn_bwd_dx.restype = i32
        L.oracle_alam_quant_pack.argtypes = [vp, i32, i64, i32, i32, i32, i32, f32, vp, vp, vp]
        L.oracle_alam_quant_pack.restype = i32
        L.oracle_alam_dequant_unpack.argtypes = [vp, vp, vp, i64, i32, i32, i32, u64, vp]
        L.oracle_alam_dequant_unpack.restype = i32
        L.oracle_triton_randn.argtypes = [u64, ctypes.c_uint32]
        L.oracle_triton_randn.restype = f32
        L.oracle_triton_rand.argtypes = [u64, ctypes.c_uint32]
        L.oracle_triton_rand.restype = f32
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def _dtype_code(a: np.ndarray) -> int:
    """numpy storage -> ABI dtype code. bf16 travels as uint16 bit patterns; fp16 as float16."""
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    if a.dtype == np.uint16:
        return BF16
    raise TypeError(f"unsupported oracle input dtype {a.dtype}")


class OracleError(RuntimeError):
    pass


def _check(rc: int):
    if rc == -1:
        raise ValueError("bits must be one of (1,2,4,8)")
    if rc != 0:
        raise OracleError(f"oracle returned {rc}")


def quant_pack(x: np.ndarray, group_size: int, bits: int, *, tile_nchw=None, rounding=NEAREST,
               noise=None, seed=0, offset=0, flags=0, clamp_alpha=0.0, meta_dtype=F32):
    """Returns (packed uint32 [NG, W], scale [NG], min [NG]); meta as float32 or uint16 (bf16)."""
    x = np.ascontiguousarray(x)
    if tile_nchw is not None:
        n, c, h, w = (int(v) for v in tile_nchw)
        s = int(round(group_size ** 0.5))
        ng = n * c * (h // s) * (w // s)
        tile = np.array([n, c, h, w], dtype=np.int64)
    else:
        ng = x.size // group_size
        tile = None
    nw = group_size * bits // 32
    packed = np.zeros((ng, nw), dtype=np.uint32)
    mdt = np.float32 if meta_dtype == F32 else np.uint16
    scale = np.zeros(ng, dtype=mdt)
    mn = np.zeros(ng, dtype=mdt)
    if noise is not None:
        noise = np.ascontiguousarray(noise, dtype=np.float32)
    rc = lib().oracle_quant_pack(_ptr(x), _dtype_code(x), ng, group_size, bits, _ptr(tile),
                                 rounding, _ptr(noise), seed, offset, flags, clamp_alpha,
                                 _ptr(packed), _ptr(scale), _ptr(mn), meta_dtype)
    _check(rc)
    return packed, scale, mn


def dequant_unpack(packed, scale, mn, group_size: int, bits: int, *, tile_nchw=None, y_dtype=F32):
    """Returns y float32 (or uint16 bf16 bits): [NG, g] flat, or the [N, C, H, W] tensor."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    ng = packed.size * 32 // bits // group_size
    meta_dtype = F32 if scale.dtype == np.float32 else BF16
    if tile_nchw is not None:
        shape = tuple(int(v) for v in tile_nchw)
        tile = np.array(shape, dtype=np.int64)
    else:
        shape = (ng, group_size)
        tile = None
    y = np.zeros(shape, dtype=np.float32 if y_dtype == F32 else np.uint16)
    rc = lib().oracle_dequant_unpack(_ptr(packed), _ptr(np.ascontiguousarray(scale)),
                                     _ptr(np.ascontiguousarray(mn)), meta_dtype, ng, group_size,
                                     bits, _ptr(tile), _ptr(y), y_dtype)
    _check(rc)
    return y


ALAM_SEED = 42  # the reference operators' fixed seed (act_triton_kernel.py:339, :374)


def alam_quant_pack(x: np.ndarray, group_size: int, bits: int, alam_bits: int, *, flags=0, clamp_alpha=0.0):
    """The reference quantizer's avg_alam mode -> (packed uint32 [NG, NW / alam_bits], scale and
    min as uint16 bf16 bits [NG])."""
    x = np.ascontiguousarray(x)
    ng = x.size // group_size
    nw = group_size * bits // 32
    packed = np.zeros((ng, max(nw // max(alam_bits, 1), 1)), dtype=np.uint32)
    scale = np.zeros(ng, dtype=np.uint16)
    mn = np.zeros(ng, dtype=np.uint16)
    _check(lib().oracle_alam_quant_pack(_ptr(x), _dtype_code(x), ng, group_size, bits, alam_bits, flags,
                                        clamp_alpha, _ptr(packed), _ptr(scale), _ptr(mn)))
    return packed, scale, mn


def alam_dequant_unpack(packed, scale, mn, group_size: int, bits: int, alam_bits: int, seed: int = ALAM_SEED):
    """avg_alam dequantize: each code repeated alam_bits times plus Triton-randn noise - 0.5 ->
    bf16 bits (uint16) [NG, g]."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    scale = np.ascontiguousarray(scale, dtype=np.uint16)
    mn = np.ascontiguousarray(mn, dtype=np.uint16)
    ng = scale.size
    y = np.zeros((ng, group_size), dtype=np.uint16)
    _check(lib().oracle_alam_dequant_unpack(_ptr(packed), _ptr(scale), _ptr(mn), ng, group_size, bits, alam_bits,
                                            seed, _ptr(y)))
    return y


def triton_randn(seed: int, offset: int) -> float:
    """One value of Triton's tl.randn(seed, offset) as this oracle restates it."""
    return float(lib().oracle_triton_randn(seed, offset))


def triton_rand(seed: int, offset: int) -> float:
    """One value of Triton's tl.rand(seed, offset) as this oracle restates it."""
    return float(lib().oracle_triton_rand(seed, offset))


def pack_codes(codes: np.ndarray, group_size: int, bits: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    ng = codes.size // group_size
    out = np.zeros((ng, group_size * bits // 32), dtype=np.uint32)
    _check(lib().oracle_pack_codes(_ptr(codes), ng, group_size, bits, _ptr(out)))
    return out


def unpack_codes(packed: np.ndarray, group_size: int, bits: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    ng = packed.size * 32 // bits // group_size
    out = np.zeros((ng, group_size), dtype=np.int8)
    _check(lib().oracle_unpack_codes(_ptr(packed), ng, group_size, bits, _ptr(out)))
    return out


def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.array(ctr, dtype=np.uint32)
    k = np.array(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().oracle_philox4x32_10(_ptr(c), _ptr(k), _ptr(out))
    return out


def philox_noise(idx0: int, n: int, seed: int, offset: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().oracle_philox_noise(idx0, n, seed, offset, _ptr(out))
    return out


def relu_pack(x: np.ndarray, bits: int, relu6: bool = False):
    """-> (y in x's storage type, packed uint32 mask codes); x float32 or uint16 (bf16 bits)."""
    x = np.ascontiguousarray(x)
    y = np.zeros_like(x)
    packed = np.zeros(x.size * bits // 32, dtype=np.uint32)
    _check(lib().oracle_relu_pack(_ptr(x), _dtype_code(x), x.size, int(relu6), bits, _ptr(y), _ptr(packed)))
    return y, packed


def relu_unpack(packed: np.ndarray, dy: np.ndarray, bits: int) -> np.ndarray:
    """-> dx as bf16 bit patterns (uint16), same shape as dy."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    dy = np.ascontiguousarray(dy)
    dx = np.zeros(dy.shape, dtype=np.uint16)
    _check(lib().oracle_relu_unpack(_ptr(packed), _ptr(dy), _dtype_code(dy), dy.size, bits, _ptr(dx)))
    return dx


def act_forward(x: np.ndarray, act: int):
    """Unfused helpers: relu/relu6 -> (y in x's type, int8 mask); gelu/silu -> (bf16 y, bf16 dy/dx)."""
    x = np.ascontiguousarray(x)
    if act in (ACT_RELU, ACT_RELU6):
        y, aux = np.zeros_like(x), np.zeros(x.shape, dtype=np.int8)
    else:
        y, aux = np.zeros(x.shape, dtype=np.uint16), np.zeros(x.shape, dtype=np.uint16)
    _check(lib().oracle_act_forward(_ptr(x), _dtype_code(x), x.size, act, _ptr(y), _ptr(aux)))
    return y, aux


def pact_clamp_fwd(x: np.ndarray, alpha: float):
    """PACT clamp -> (bf16 clamp(x, -alpha, alpha) as uint16 bits, int8 mask |x| <= alpha), x's shape."""
    x = np.ascontiguousarray(x)
    y = np.zeros(x.shape, dtype=np.uint16)
    mask = np.zeros(x.shape, dtype=np.int8)
    _check(lib().oracle_pact_clamp_fwd(_ptr(x), _dtype_code(x), x.size, float(alpha), _ptr(y), _ptr(mask)))
    return y, mask


def pact_clamp_bwd(mask: np.ndarray, dy: np.ndarray) -> np.ndarray:
    """Its gradient -> bf16 (uint16 bits) dy where mask != 0, else +0, dy's shape."""
    mask = np.ascontiguousarray(mask, dtype=np.int8)
    dy = np.ascontiguousarray(dy)
    dx = np.zeros(dy.shape, dtype=np.uint16)
    _check(lib().oracle_pact_clamp_bwd(_ptr(mask), _ptr(dy), _dtype_code(dy), dy.size, _ptr(dx)))
    return dx


def act_quant_pack(x: np.ndarray, act: int, group_size: int, bits: int, *, tile_nchw=None, meta_dtype=BF16):
    """Fused GELU/SiLU forward -> (bf16 y shaped like x, packed [NG, W], scale [NG], min [NG])."""
    x = np.ascontiguousarray(x)
    ng = x.size // group_size
    tile = None if tile_nchw is None else np.array([int(v) for v in tile_nchw], dtype=np.int64)
    y = np.zeros(x.shape, dtype=np.uint16)
    packed = np.zeros((ng, group_size * bits // 32), dtype=np.uint32)
    mdt = np.float32 if meta_dtype == F32 else np.uint16
    scale, mn = np.zeros(ng, dtype=mdt), np.zeros(ng, dtype=mdt)
    _check(lib().oracle_act_quant_pack(_ptr(x), _dtype_code(x), act, ng, group_size, bits, _ptr(tile), _ptr(y),
                                       _ptr(packed), _ptr(scale), _ptr(mn), meta_dtype))
    return y, packed, scale, mn


def act_dequant_mul(packed, scale, mn, group_size: int, bits: int, dy: np.ndarray, *, tile_nchw=None,
                    alam_seed=None):
    """Fused GELU/SiLU backward -> dx = bf16(dy * dequant) as uint16, shaped like dy; with
    alam_seed (the SiLU backward's avg_alam at alam_bits = 1) each code carries
    tl.rand(alam_seed + group, element) - 0.5."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    dy = np.ascontiguousarray(dy)
    ng = packed.size * 32 // bits // group_size
    meta_dtype = F32 if scale.dtype == np.float32 else BF16
    tile = None if tile_nchw is None else np.array([int(v) for v in tile_nchw], dtype=np.int64)
    dx = np.zeros(dy.shape, dtype=np.uint16)
    sc, m = np.ascontiguousarray(scale), np.ascontiguousarray(mn)
    if alam_seed is None:
        _check(lib().oracle_act_dequant_mul(_ptr(packed), _ptr(sc), _ptr(m), meta_dtype, ng, group_size, bits,
                                            _ptr(tile), _ptr(dy), _dtype_code(dy), _ptr(dx)))
    else:
        _check(lib().oracle_act_dequant_mul_alam(_ptr(packed), _ptr(sc), _ptr(m), meta_dtype, ng, group_size, bits,
                                                 _ptr(tile), _ptr(dy), _dtype_code(dy), int(alam_seed), _ptr(dx)))
    return dx


BN_NORM, BN_QUANT, BN_RELU_QUANT, BN_RELU6_QUANT = 0, 1, 2, 3


def _bn_geom(x: np.ndarray):
    """[N, C, *spatial] contiguous -> (N, C, HW, stride_n, stride_c)."""
    N, C = int(x.shape[0]), int(x.shape[1])
    HW = int(np.prod(x.shape[2:], dtype=np.int64)) if x.ndim > 2 else 1
    return N, C, HW, C * HW, HW


def bn_reduce(x: np.ndarray):
    """-> (sum, sumsq) float64 [C] over each channel of a contiguous [N, C, ...] array."""
    x = np.ascontiguousarray(x)
    N, C, HW, sn, sc = _bn_geom(x)
    s, q = np.zeros(C), np.zeros(C)
    _check(lib().oracle_bn_reduce(_ptr(x), _dtype_code(x), N, C, HW, sn, sc, _ptr(s), _ptr(q)))
    return s, q


def bn_norm_quant(x: np.ndarray, weight, bias, *, mode, group_size=0, bits=2, eps=1e-5, sum=None, sumsq=None,
                  mean=None, invstd=None, alam_bits=0):
    """Normalize (+ ReLU) (+ quant-pack) of a contiguous [N, C, ...] array. Statistics: fp32 sum /
    sumsq (non-sync) or fp32 mean / invstd (sync). Returns a dict with y (bf16 bits, x's shape),
    x_hat (BN_NORM), packed [C, M*bits/32] ([C, M*bits/32/alam_bits] with avg_alam, alam_bits > 0),
    relu_packed [C, M/32], scale / min (bf16 bits [C, M/g]), mean / var (non-sync) and t (fp32
    [C, M], the quantized values)."""
    x = np.ascontiguousarray(x)
    N, C, HW, sn, sc = _bn_geom(x)
    M = N * HW
    sync = mean is not None
    f = lambda a: None if a is None else np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
    w, b = f(weight), f(bias)
    sum, sumsq, mean, invstd = f(sum), f(sumsq), f(mean), f(invstd)
    out = {"y": np.zeros(x.shape, dtype=np.uint16)}
    quant = mode != BN_NORM
    out["x_hat"] = np.zeros(x.shape, dtype=np.uint16) if not quant else None
    out["packed"] = np.zeros((C, M * bits // 32 // max(alam_bits, 1)), dtype=np.uint32) if quant else None
    out["relu_packed"] = np.zeros((C, M // 32), dtype=np.uint32) if mode in (BN_RELU_QUANT, BN_RELU6_QUANT) else None
    ng = M // group_size if quant else 0
    out["scale"] = np.zeros((C, ng), dtype=np.uint16) if quant else None
    out["min"] = np.zeros((C, ng), dtype=np.uint16) if quant else None
    out["mean"] = np.zeros(C, dtype=np.float32)
    out["var"] = np.zeros(C, dtype=np.float32)
    out["t"] = np.zeros((C, M), dtype=np.float32) if quant else None
    _check(lib().oracle_bn_norm_quant(_ptr(x), _dtype_code(x), N, C, HW, sn, sc, _ptr(sum), _ptr(sumsq), _ptr(mean),
                                      _ptr(invstd), int(sync), _ptr(w), _ptr(b), float(eps), mode, group_size, bits,
                                      _ptr(out["y"]), _ptr(out["x_hat"]), _ptr(out["packed"]),
                                      _ptr(out["relu_packed"]), _ptr(out["scale"]), _ptr(out["min"]),
                                      _ptr(out["mean"]), _ptr(out["var"]), _ptr(out["t"]), int(alam_bits)))
    return out


def _bn_bwd_args(mode, x_hat, packed, relu_packed, scale, mn, dy):
    c = lambda a, dt: None if a is None else np.ascontiguousarray(a, dtype=dt)  # noqa: E731
    return (c(x_hat, np.uint16), c(packed, np.uint32), c(relu_packed, np.uint32), c(scale, np.uint16),
            c(mn, np.uint16), np.ascontiguousarray(dy))


def bn_bwd_reduce(dy: np.ndarray, *, mode, x_hat=None, packed=None, relu_packed=None, scale=None, min=None,
                  group_size=0, bits=2, alam_bits=0):
    """-> (dweight, dbias) float64 [C]: sum(dy*m * x_hat'), sum(dy*m); with avg_alam (alam_bits > 0)
    x_hat' carries the reference's tl.rand noise."""
    xh, p, rp, s, mn, dy = _bn_bwd_args(mode, x_hat, packed, relu_packed, scale, min, dy)
    N, C, HW, sn, sc = _bn_geom(dy)
    dw, db = np.zeros(C), np.zeros(C)
    _check(lib().oracle_bn_bwd_reduce(mode, _ptr(xh), _ptr(p), _ptr(rp), _ptr(s), _ptr(mn), _ptr(dy), _dtype_code(dy),
                                      N, C, HW, sn, sc, group_size, bits, _ptr(dw), _ptr(db), int(alam_bits)))
    return dw, db


def bn_bwd_dx(dy: np.ndarray, dweight, dbias, weight, var, *, mode, eps=1e-7, var_is_invstd=False, x_hat=None,
              packed=None, relu_packed=None, scale=None, min=None, group_size=0, bits=2, alam_bits=0):
    """-> dx as bf16 bits (uint16), dy's shape; dweight / dbias / weight / var fp32 [C]."""
    xh, p, rp, s, mn, dy = _bn_bwd_args(mode, x_hat, packed, relu_packed, scale, min, dy)
    N, C, HW, sn, sc = _bn_geom(dy)
    f = lambda a: np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
    dw, db, w, v = f(dweight), f(dbias), f(weight), f(var)
    dx = np.zeros(dy.shape, dtype=np.uint16)
    _check(lib().oracle_bn_bwd_dx(mode, _ptr(xh), _ptr(p), _ptr(rp), _ptr(s), _ptr(mn), _ptr(dy), _dtype_code(dy), N,
                                  C, HW, sn, sc, group_size, bits, _ptr(dw), _ptr(db), _ptr(w), _ptr(v), float(eps),
                                  int(var_is_invstd), _ptr(dx), int(alam_bits)))
    return dx


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16), vectorised in numpy."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(int(n))
