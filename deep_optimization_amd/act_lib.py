"""``torch.ops.act_lib`` operators backed by the gfx950 HIP kernels of libdopt.so.

Drop-in for Activation_Compression/act_triton_kernel.py:336-473: the four reference operators
keep their names and schemas,

    act_lib::quant_pack_triton(x, bits, group_size, avg_alam, alam_bits, clamp, clamp_alpha)
        -> (packed int32 [N*G, W], scale [N, G], min [N, G])          (reference :336-368)
    act_lib::dequant_unpack_triton(packed, scale, xmin, bits, group_size, avg_alam, alam_bits)
        -> bf16 [N, G, g]                                              (reference :372-395)
    act_lib::pack_triton(x, bits, group_size) -> int32 [N*G, W]        (reference :398-417)
    act_lib::unpack_triton(packed, bits, N, G, group_size) -> int8 [N, G, g]   (reference :419-433)

with the reference's semantics (tanh squash always on, nearest rounding, bf16 scale/min).
The general operators below expose what the reference leaves fixed: rounding mode (nearest,
stochastic from a noise tensor, stochastic from Philox(seed, offset)), the squash pre-transform,
the scale/min dtype (fp32 or bf16), the output dtype, and the fused s x s spatial-tile layout
(act_lib::quant_pack_tiles / act_lib::dequant_unpack_tiles), which removes the permute copy of
tensor_act_reshape_utils.py:128 and :152.

Every operator is registered straight with the dispatcher (``torch.library.Library``: one Python
call per op, no wrapper layers) for CUDA (HIP) tensors only, and has a fake (meta)
implementation with the correct output shapes; there is no CPU implementation. The operators the
compressed layers call most often take their CUDA kernel from the native library instead
(``_native``, csrc/torch_ops.cpp), with the same checks and outputs as the Python implementations
here, which stay callable as functions.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _lib, _native

_DTYPE_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}
_META_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
_OUT_CODE = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}

ROUND_NEAREST = _lib.ROUND_NEAREST
ROUND_STOCH_NOISE = _lib.ROUND_STOCH_NOISE
ROUND_STOCH_PHILOX = _lib.ROUND_STOCH_PHILOX
_ROUNDING_NAMES = {"nearest": ROUND_NEAREST, "stochastic": ROUND_STOCH_PHILOX,
                   "stochastic_philox": ROUND_STOCH_PHILOX, "stochastic_noise": ROUND_STOCH_NOISE}

_U64 = (1 << 64) - 1


def _bits_consts(bits: int, group_size: int):
    """(values per int32 word, words per group, max code); same contract as
    act_triton_kernel.py:328-334 (ValueError for bits outside {1, 2, 4, 8})."""
    if bits not in (1, 2, 4, 8):
        raise ValueError(f"bits must be one of (1,2,4,8). got {bits}")
    vpw = 32 // bits
    nwords = group_size // vpw
    qmax = (1 << bits) - 1
    return vpw, nwords, qmax


def rounding_code(rounding) -> int:
    if isinstance(rounding, int):
        return rounding
    try:
        return _ROUNDING_NAMES[rounding]
    except KeyError:
        raise ValueError(f"unknown rounding mode {rounding!r}") from None


def _stream(t: Tensor) -> int:
    """Raw hipStream_t of torch's current stream on t's device (what the C ABI enqueues on). The
    C ABI launches on the calling thread's current device, so t must live there."""
    dev = t.get_device()
    if dev != torch.cuda.current_device():
        raise RuntimeError(f"act_lib operators launch on the current device ({torch.cuda.current_device()}); "
                           f"the tensors are on cuda:{dev}: call under torch.cuda.device({dev})")
    return torch._C._cuda_getCurrentRawStream(dev)


def _require_cuda(*ts: Tensor) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("act_lib operators run on HIP (cuda) tensors only")


def _aligned(t: Tensor) -> Tensor:
    """Contiguous view with a 16-byte aligned base (the kernels use 128-bit accesses)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def _flags(clamp: bool, squash: bool) -> int:
    return (_lib.FLAG_CLAMP if clamp else 0) | (_lib.FLAG_SQUASH if squash else 0)


def _quant_pack_launch(x: Tensor, n_groups: int, bits: int, group_size: int, tile, clamp: bool,
                       clamp_alpha: float, squash: bool, rounding: int, noise: Optional[Tensor],
                       seed: int, offset: int, scale_dtype: torch.dtype):
    _, nwords, _ = _bits_consts(bits, group_size)
    if x.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"quant_pack: unsupported input dtype {x.dtype}")
    if scale_dtype not in _META_CODE:
        raise RuntimeError(f"quant_pack: scale dtype must be float32 or bfloat16, got {scale_dtype}")
    _require_cuda(x, noise)
    x = _aligned(x)
    packed = torch.empty((n_groups, nwords), dtype=torch.int32, device=x.device)
    scale = torch.empty((n_groups,), dtype=scale_dtype, device=x.device)
    xmin = torch.empty((n_groups,), dtype=scale_dtype, device=x.device)
    nz_ptr = None
    if rounding == ROUND_STOCH_NOISE:
        if noise is None:
            raise RuntimeError("quant_pack: rounding=stochastic_noise needs a noise tensor")
        if noise.numel() != n_groups * group_size:
            raise RuntimeError(f"quant_pack: noise has {noise.numel()} values, expected {n_groups * group_size}")
        noise = _aligned(noise.to(torch.float32))
        nz_ptr = noise.data_ptr()
    tile_arr = None
    if tile is not None:
        import ctypes
        tile_arr = (ctypes.c_int64 * 4)(*tile)
    rc = _lib.lib().dopt_quant_pack(
        x.data_ptr(), _DTYPE_CODE[x.dtype], n_groups, group_size, bits, tile_arr, rounding, nz_ptr,
        seed & _U64, offset & _U64, _flags(clamp, squash), float(clamp_alpha), packed.data_ptr(),
        scale.data_ptr(), xmin.data_ptr(), _META_CODE[scale_dtype], _stream(x))
    _lib.check(rc, "quant_pack")
    return packed, scale, xmin


def _dequant_launch(packed: Tensor, scale: Tensor, xmin: Tensor, n_groups: int, bits: int,
                    group_size: int, tile, out: Tensor):
    _, nwords, _ = _bits_consts(bits, group_size)
    if scale.dtype not in _META_CODE or xmin.dtype != scale.dtype:
        raise RuntimeError("dequant_unpack: scale and min must both be float32 or both bfloat16")
    # the kernel reads these unchecked: every size must match the group count
    if scale.numel() != n_groups or xmin.numel() != n_groups:
        raise RuntimeError(f"dequant_unpack: scale and min must hold {n_groups} values, got {scale.numel()} "
                           f"and {xmin.numel()}")
    if packed.numel() * packed.element_size() != n_groups * nwords * 4:
        raise RuntimeError(f"dequant_unpack: packed holds {packed.numel() * packed.element_size()} bytes, "
                           f"expected {n_groups * nwords * 4} ({n_groups} groups of {nwords} words)")
    _require_cuda(packed, scale, xmin)
    packed = _aligned(packed)
    scale = scale.contiguous()
    xmin = xmin.contiguous()
    tile_arr = None
    if tile is not None:
        import ctypes
        tile_arr = (ctypes.c_int64 * 4)(*tile)
    rc = _lib.lib().dopt_dequant_unpack(
        packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), _META_CODE[scale.dtype], n_groups,
        group_size, bits, tile_arr, out.data_ptr(), _OUT_CODE[out.dtype], _stream(packed))
    _lib.check(rc, "dequant_unpack")
    return out


# --------------------------------------------------------------------------- registration
_LIB = torch.library.Library("act_lib", "DEF")


def _op(schema: str, impl, fake):
    """Define act_lib::<schema>, bind the HIP implementation and the fake (meta) kernel. The
    operators of the native library (``_native.OPS``) get their CUDA kernel from it instead; their
    Python implementation stays callable as a function."""
    name = schema.split("(", 1)[0]
    _LIB.define(schema)
    if not _native.native(name):
        _LIB.impl(name, impl, "CUDA")
    torch.library.register_fake(f"act_lib::{name}", fake, lib=_LIB)
    return getattr(torch.ops.act_lib, name)


def _meta3(x: Tensor, N: int, G: int, bits: int, group_size: int, scale_dtype: torch.dtype):
    _, nwords, _ = _bits_consts(bits, group_size)
    return (x.new_empty((N * G, nwords), dtype=torch.int32), x.new_empty((N, G), dtype=scale_dtype),
            x.new_empty((N, G), dtype=scale_dtype))


# --------------------------------------------------------------------------- general operators
def _quant_pack(x, bits, group_size, clamp, clamp_alpha, squash, rounding, noise, seed, offset, scale_dtype):
    """x [N, G, group_size] -> (packed int32 [N*G, W], scale [N, G], min [N, G])."""
    if x.dim() != 3 or x.shape[-1] != group_size:
        raise RuntimeError(f"quant_pack expects x of shape [N, G, {group_size}], got {tuple(x.shape)}")
    N, G, _ = x.shape
    packed, scale, xmin = _quant_pack_launch(x, N * G, bits, group_size, None, clamp, clamp_alpha,
                                             squash, rounding, noise, seed, offset, scale_dtype)
    return packed, scale.view(N, G), xmin.view(N, G)


quant_pack = _op(
    "quant_pack(Tensor x, int bits, int group_size, bool clamp, float clamp_alpha, bool squash, int rounding, "
    "Tensor? noise, int seed, int offset, ScalarType scale_dtype) -> (Tensor, Tensor, Tensor)",
    _quant_pack,
    lambda x, bits, group_size, clamp, clamp_alpha, squash, rounding, noise, seed, offset, scale_dtype:
        _meta3(x, x.shape[0], x.shape[1], bits, group_size, scale_dtype))


def _tile_groups(shape, group_size: int):
    if len(shape) != 4:
        raise RuntimeError(f"tile layout expects a 4-D [N, C, H, W] tensor, got {tuple(shape)}")
    s = int(round(group_size ** 0.5))
    N, C, H, W = (int(v) for v in shape)
    if s * s != group_size or H % s or W % s:
        raise RuntimeError(f"tile layout needs s*s == group_size and H, W divisible by s "
                           f"(group_size={group_size}, H={H}, W={W})")
    return N, C * (H // s) * (W // s)


def _quant_pack_tiles(x, bits, group_size, clamp, clamp_alpha, squash, rounding, noise, seed, offset, scale_dtype):
    """x [N, C, H, W] grouped into s x s spatial tiles (s*s = group_size), read in place."""
    N, G = _tile_groups(x.shape, group_size)
    packed, scale, xmin = _quant_pack_launch(x, N * G, bits, group_size, tuple(x.shape), clamp,
                                             clamp_alpha, squash, rounding, noise, seed, offset,
                                             scale_dtype)
    return packed, scale.view(N, G), xmin.view(N, G)


def _quant_pack_tiles_fake(x, bits, group_size, clamp, clamp_alpha, squash, rounding, noise, seed, offset,
                           scale_dtype):
    N, G = _tile_groups(x.shape, group_size)
    return _meta3(x, N, G, bits, group_size, scale_dtype)


quant_pack_tiles = _op(
    "quant_pack_tiles(Tensor x, int bits, int group_size, bool clamp, float clamp_alpha, bool squash, "
    "int rounding, Tensor? noise, int seed, int offset, ScalarType scale_dtype) -> (Tensor, Tensor, Tensor)",
    _quant_pack_tiles, _quant_pack_tiles_fake)


def _dequant_unpack(packed, scale, xmin, bits, group_size, out_dtype):
    """-> [N, G, group_size] of out_dtype (float32 or bfloat16)."""
    N, G = scale.shape
    if out_dtype not in _OUT_CODE:
        raise RuntimeError(f"dequant_unpack: output dtype must be float32 or bfloat16, got {out_dtype}")
    y = torch.empty((N, G, group_size), dtype=out_dtype, device=packed.device)
    return _dequant_launch(packed, scale, xmin, N * G, bits, group_size, None, y)


dequant_unpack = _op(
    "dequant_unpack(Tensor packed, Tensor scale, Tensor xmin, int bits, int group_size, ScalarType out_dtype) "
    "-> Tensor",
    _dequant_unpack,
    lambda packed, scale, xmin, bits, group_size, out_dtype:
        packed.new_empty((scale.shape[0], scale.shape[1], group_size), dtype=out_dtype))


def _dequant_unpack_tiles(packed, scale, xmin, bits, group_size, N, C, H, W, out_dtype):
    """-> [N, C, H, W] of out_dtype: the inverse tile scatter is fused into the stores."""
    n, G = _tile_groups((N, C, H, W), group_size)
    if tuple(scale.shape) != (n, G):
        raise RuntimeError(f"dequant_unpack_tiles: scale shape {tuple(scale.shape)} != {(n, G)}")
    if out_dtype not in _OUT_CODE:
        raise RuntimeError(f"dequant_unpack_tiles: output dtype must be float32 or bfloat16, got {out_dtype}")
    y = torch.empty((N, C, H, W), dtype=out_dtype, device=packed.device)
    return _dequant_launch(packed, scale, xmin, n * G, bits, group_size, (N, C, H, W), y)


dequant_unpack_tiles = _op(
    "dequant_unpack_tiles(Tensor packed, Tensor scale, Tensor xmin, int bits, int group_size, int N, int C, "
    "int H, int W, ScalarType out_dtype) -> Tensor",
    _dequant_unpack_tiles,
    lambda packed, scale, xmin, bits, group_size, N, C, H, W, out_dtype:
        packed.new_empty((N, C, H, W), dtype=out_dtype))


# --------------------------------------------------------------------------- reference schemas
ALAM_SEED = 42  # the reference operators' fixed seed (act_triton_kernel.py:339, :374)


def _silu_alam(avg_alam: bool, alam_bits: int, where: str) -> bool:
    """The SiLU operators' avg_alam mode exists at alam_bits = 1 only: the reference's forward
    kernel reshapes the group's G codes to G / alam_bits before packing
    (activations/kernel_implementation.py:330), which Triton rejects for alam_bits >= 2. At
    alam_bits = 1 the codes are the plain ones and the backward adds tl.rand noise (:382-390).
    Returns whether the backward adds that noise."""
    if avg_alam and alam_bits != 1:
        raise NotImplementedError(
            f"{where}: avg_alam=True with alam_bits={alam_bits}: the reference's SiLU forward kernel cannot "
            "reshape the codes for alam_bits >= 2 (alam_bits = 1 is supported)")
    return bool(avg_alam)


def _alam_words(bits: int, group_size: int, alam_bits: int) -> int:
    """Packed words per group with avg_alam: the reference's cdiv(NWORDS, alam_bits), where its
    reshape of the codes into runs of alam_bits requires alam_bits to divide NWORDS."""
    _, nwords, _ = _bits_consts(bits, group_size)
    if alam_bits < 1 or alam_bits & (alam_bits - 1) or nwords % alam_bits:
        raise RuntimeError(f"avg_alam: alam_bits must be a power of two dividing group_size*bits/32 = {nwords}, "
                           f"got {alam_bits}")
    return nwords // alam_bits


def _quant_pack_triton(x, bits, group_size, avg_alam, alam_bits, clamp, clamp_alpha):
    """Reference semantics (act_triton_kernel.py:336-368): [clamp], tanh squash, nearest
    rounding, bf16 scale and min; with avg_alam the mean of every run of alam_bits code
    arguments is truncated into one code (:116-118)."""
    if x.dim() != 3 or x.shape[-1] != group_size:  # the reference's x.view(N * G, group_size)
        raise RuntimeError(f"quant_pack_triton expects x of shape [N, G, {group_size}], got {tuple(x.shape)}")
    N, G, _ = x.shape
    if not avg_alam:
        packed, scale, xmin = _quant_pack_launch(x, N * G, bits, group_size, None, clamp, clamp_alpha,
                                                 True, ROUND_NEAREST, None, 0, 0, torch.bfloat16)
        return packed, scale.view(N, G), xmin.view(N, G)
    anw = _alam_words(bits, group_size, alam_bits)
    if x.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"quant_pack_triton: unsupported input dtype {x.dtype}")
    _require_cuda(x)
    x = x.contiguous()
    packed = torch.empty((N * G, anw), dtype=torch.int32, device=x.device)
    scale = torch.empty((N * G,), dtype=torch.bfloat16, device=x.device)
    xmin = torch.empty((N * G,), dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().dopt_alam_quant_pack(x.data_ptr(), _DTYPE_CODE[x.dtype], N * G, group_size, bits, alam_bits,
                                         _flags(clamp, True), float(clamp_alpha), packed.data_ptr(), scale.data_ptr(),
                                         xmin.data_ptr(), _stream(x))
    _lib.check(rc, "alam_quant_pack")
    return packed, scale.view(N, G), xmin.view(N, G)


def _quant_pack_triton_fake(x, bits, group_size, avg_alam, alam_bits, clamp, clamp_alpha):
    N, G = x.shape[0], x.shape[1]
    if not avg_alam:
        return _meta3(x, N, G, bits, group_size, torch.bfloat16)
    anw = _alam_words(bits, group_size, alam_bits)
    return (x.new_empty((N * G, anw), dtype=torch.int32), x.new_empty((N, G), dtype=torch.bfloat16),
            x.new_empty((N, G), dtype=torch.bfloat16))


quant_pack_triton = _op(
    "quant_pack_triton(Tensor x, int bits, int group_size, bool avg_alam, int alam_bits, bool clamp, "
    "float clamp_alpha) -> (Tensor, Tensor, Tensor)",
    _quant_pack_triton, _quant_pack_triton_fake)


def _dequant_unpack_triton(packed, scale, xmin, bits, group_size, avg_alam, alam_bits):
    """Reference semantics (act_triton_kernel.py:372-395): bf16 output [N, G, g] whatever the
    scale dtype (the reference allocates y as bf16, :382), one rounding from fp32. With avg_alam
    each code covers alam_bits elements and carries Triton-randn noise (seed 42 + group,
    element offset) minus 0.5 (:212-219)."""
    N, G = scale.shape
    y = torch.empty((N, G, group_size), dtype=torch.bfloat16, device=packed.device)
    if not avg_alam:
        return _dequant_launch(packed, scale, xmin, N * G, bits, group_size, None, y)
    anw = _alam_words(bits, group_size, alam_bits)
    if scale.dtype != torch.bfloat16 or xmin.dtype != torch.bfloat16:
        raise RuntimeError("dequant_unpack_triton: avg_alam takes the bf16 scale and min its quantizer writes")
    if packed.numel() != N * G * anw:
        raise RuntimeError(f"dequant_unpack_triton: packed holds {packed.numel()} words, expected {N * G * anw} "
                           f"({N * G} groups of {anw})")
    _require_cuda(packed, scale, xmin)
    packed, scale, xmin = packed.contiguous(), scale.contiguous(), xmin.contiguous()
    rc = _lib.lib().dopt_alam_dequant_unpack(packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), N * G, group_size,
                                             bits, alam_bits, ALAM_SEED, y.data_ptr(), _stream(packed))
    _lib.check(rc, "alam_dequant_unpack")
    return y


dequant_unpack_triton = _op(
    "dequant_unpack_triton(Tensor packed, Tensor scale, Tensor xmin, int bits, int group_size, bool avg_alam, "
    "int alam_bits) -> Tensor",
    _dequant_unpack_triton,
    lambda packed, scale, xmin, bits, group_size, avg_alam, alam_bits:
        packed.new_empty((scale.shape[0], scale.shape[1], group_size), dtype=torch.bfloat16))


def _pack_triton(x, bits, group_size):
    """int8 codes [N, G, g] -> int32 words [N*G, W] (act_triton_kernel.py:398-417)."""
    if x.dim() != 3 or x.shape[-1] != group_size:
        raise RuntimeError(f"pack_triton expects x of shape [N, G, {group_size}], got {tuple(x.shape)}")
    _, nwords, _ = _bits_consts(bits, group_size)
    _require_cuda(x)
    N, G, _ = x.shape
    codes = _aligned(x.to(torch.int8) if x.dtype != torch.int8 else x)
    packed = torch.empty((N * G, nwords), dtype=torch.int32, device=x.device)
    rc = _lib.lib().dopt_pack_codes(codes.data_ptr(), N * G, group_size, bits, packed.data_ptr(), _stream(x))
    _lib.check(rc, "pack_codes")
    return packed


pack_triton = _op(
    "pack_triton(Tensor x, int bits, int group_size) -> Tensor",
    _pack_triton,
    lambda x, bits, group_size:
        x.new_empty((x.shape[0] * x.shape[1], _bits_consts(bits, group_size)[1]), dtype=torch.int32))


def _unpack_triton(packed, bits, N, G, group_size):
    """int32 words [N*G, W] -> int8 codes [N, G, g] (act_triton_kernel.py:419-433)."""
    _, nwords, _ = _bits_consts(bits, group_size)
    _require_cuda(packed)
    NG = packed.shape[0]
    if NG != N * G:
        raise RuntimeError(f"unpack_triton: packed has {NG} groups, expected N*G = {N * G}")
    if packed.numel() * packed.element_size() != NG * nwords * 4:
        raise RuntimeError(f"unpack_triton: packed holds {packed.numel() * packed.element_size()} bytes, expected "
                           f"{NG * nwords * 4} ({NG} groups of {nwords} words)")
    packed = _aligned(packed)
    out = torch.empty((NG, group_size), dtype=torch.int8, device=packed.device)
    rc = _lib.lib().dopt_unpack_codes(packed.data_ptr(), NG, group_size, bits, out.data_ptr(), _stream(packed))
    _lib.check(rc, "unpack_codes")
    return out.view(N, G, group_size)


unpack_triton = _op(
    "unpack_triton(Tensor packed, int bits, int N, int G, int group_size) -> Tensor",
    _unpack_triton,
    lambda packed, bits, N, G, group_size: packed.new_empty((N, G, group_size), dtype=torch.int8))


# --------------------------------------------------------------------------- FP8 GEMM
def _fp8_gemm_nt(a, b, out_scale):
    """a [M, K] e4m3, b [N, K] e4m3 -> bf16 [M, N] = out_scale * a @ b.T (fp32 accumulate)."""
    if a.dtype != torch.float8_e4m3fn or b.dtype != torch.float8_e4m3fn:
        raise RuntimeError("fp8_gemm_nt expects torch.float8_e4m3fn operands")
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[1]:
        raise RuntimeError(f"fp8_gemm_nt: shapes {tuple(a.shape)} x {tuple(b.shape)}^T do not contract")
    _require_cuda(a, b)
    a = _aligned(a)
    b = _aligned(b)
    M, K = a.shape
    N = b.shape[0]
    c = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    rc = _lib.lib().dopt_fp8_gemm_nt(a.data_ptr(), b.data_ptr(), M, N, K, K, K, float(out_scale),
                                     c.data_ptr(), N, _stream(a))
    _lib.check(rc, "fp8_gemm_nt")
    return c


fp8_gemm_nt = _op(
    "fp8_gemm_nt(Tensor a, Tensor b, float out_scale) -> Tensor",
    _fp8_gemm_nt,
    lambda a, b, out_scale: a.new_empty((a.shape[0], b.shape[0]), dtype=torch.bfloat16))


def _kmajor(t: Tensor, rows: int, k: int, stride_r: int, stride_k: int, k_pad: int):
    """(tensor, row stride) of an e4m3 operand as the GEMM reads it: rows K-contiguous, row stride a
    multiple of 16, 16-byte aligned. Used in place when it already is; otherwise packed by
    dopt_fp8_pack_kmajor into a fresh [rows, k_pad] buffer whose padding columns are zero."""
    if stride_k == 1 and k == k_pad and stride_r % 16 == 0 and k <= stride_r < (1 << 23) and t.data_ptr() % 16 == 0:
        return t, stride_r
    out = (torch.zeros if k_pad != k else torch.empty)((rows, k_pad), dtype=torch.uint8, device=t.device)
    rc = _lib.lib().dopt_fp8_pack_kmajor(t.data_ptr(), rows, k, stride_r, stride_k, out.data_ptr(), k_pad, _stream(t))
    _lib.check(rc, "fp8_pack_kmajor")
    return out, k_pad


def _fp8_linear(a, b, out_scale):
    """Triton_Linear's contraction (Activation_Compression/triton_kernel/linear.py:43-95) in e4m3:
    a [M, K] @ b [K, N] with any strides -> bf16 [M, N] = out_scale * a @ b, fp32 accumulate. The
    GEMM reads both operands K-contiguous: an operand in another layout (b in its row-major [K, N]
    layout, a transposed view, unaligned rows, K not a multiple of 16) is first packed by
    dopt_fp8_pack_kmajor (zero-padding K to a multiple of 16), the rest is read in place."""
    if a.dtype != torch.float8_e4m3fn or b.dtype != torch.float8_e4m3fn:
        raise RuntimeError("fp8_linear expects torch.float8_e4m3fn operands")
    if a.dim() != 2 or b.dim() != 2 or a.shape[1] != b.shape[0]:
        raise RuntimeError(f"fp8_linear: shapes {tuple(a.shape)} x {tuple(b.shape)} do not contract")
    _require_cuda(a, b)
    M, K = a.shape
    N = b.shape[1]
    c = torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    if M == 0 or N == 0:
        return c
    if K == 0:
        return c.zero_()
    k_pad = (K + 15) // 16 * 16
    ta, lda = _kmajor(a.view(torch.uint8), M, K, a.stride(0), a.stride(1), k_pad)
    tb, ldb = _kmajor(b.view(torch.uint8), N, K, b.stride(1), b.stride(0), k_pad)
    rc = _lib.lib().dopt_fp8_gemm_nt(ta.data_ptr(), tb.data_ptr(), M, N, k_pad, lda, ldb, float(out_scale),
                                     c.data_ptr(), N, _stream(a))
    _lib.check(rc, "fp8_linear")
    return c


fp8_linear = _op(
    "fp8_linear(Tensor a, Tensor b, float out_scale) -> Tensor",
    _fp8_linear,
    lambda a, b, out_scale: a.new_empty((a.shape[0], b.shape[1]), dtype=torch.bfloat16))


# --------------------------------------------------------------------------- fused activation layers
# Reference: Activation_Compression/modules/activations/kernel_registration.py (op names and
# schemas kept), kernels in kernel_implementation.py. Scale and min are bf16 [N*G] as there.
ACT_RELU, ACT_RELU6, ACT_GELU, ACT_SILU = _lib.ACT_RELU, _lib.ACT_RELU6, _lib.ACT_GELU, _lib.ACT_SILU


def _relu_act(relu: bool, relu6: bool) -> int:
    if relu:
        return ACT_RELU
    if relu6:
        return ACT_RELU6
    raise RuntimeError("relu ops need relu=True or relu6=True (the reference kernel has no other branch)")


def _relu_triton(x, relu, relu6):
    """-> (y, int8 mask), both shaped like x (kernel_registration.py:22-39)."""
    if x.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"relu_triton: unsupported dtype {x.dtype}")
    _require_cuda(x)
    x = _aligned(x)
    y = torch.empty_like(x)
    mask = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    rc = _lib.lib().dopt_act_forward(x.data_ptr(), _DTYPE_CODE[x.dtype], x.numel(), _relu_act(relu, relu6),
                                     y.data_ptr(), mask.data_ptr(), _stream(x))
    _lib.check(rc, "relu_triton")
    return y, mask


relu_triton = _op("relu_triton(Tensor x, bool relu, bool relu6) -> (Tensor, Tensor)", _relu_triton,
                  lambda x, relu, relu6: (torch.empty_like(x), torch.empty_like(x, dtype=torch.int8)))


def _flat_groups(x: Tensor, group_size: int):
    N = x.shape[0]
    if x.numel() % (N * group_size):
        raise RuntimeError(f"x of shape {tuple(x.shape)} does not split into [N, G, {group_size}] groups")
    return N, x.numel() // N // group_size


def _relu_fwd_fused_pack(x, relu, relu6, bits, group_size):
    """-> (y shaped like x, packed mask codes [N*G, W], N, G) (kernel_registration.py:42-72)."""
    _, nwords, _ = _bits_consts(bits, group_size)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"relu_fwd_fused_pack: input must be bfloat16 or float32, got {x.dtype}")
    _require_cuda(x)
    N, G = _flat_groups(x, group_size)
    x = _aligned(x)
    y = torch.empty_like(x)
    packed = torch.empty((N * G, nwords), dtype=torch.int32, device=x.device)
    rc = _lib.lib().dopt_relu_pack(x.data_ptr(), _DTYPE_CODE[x.dtype], x.numel(),
                                   int(_relu_act(relu, relu6) == ACT_RELU6), bits, y.data_ptr(), packed.data_ptr(),
                                   _stream(x))
    _lib.check(rc, "relu_fwd_fused_pack")
    return y, packed, N, G


def _relu_fwd_fused_pack_fake(x, relu, relu6, bits, group_size):
    N, G = _flat_groups(x, group_size)
    return torch.empty_like(x), x.new_empty((N * G, _bits_consts(bits, group_size)[1]), dtype=torch.int32), N, G


relu_fwd_fused_pack = _op(
    "relu_fwd_fused_pack(Tensor x, bool relu, bool relu6, int bits, int group_size) -> (Tensor, Tensor, int, int)",
    _relu_fwd_fused_pack, _relu_fwd_fused_pack_fake)


def _relu_bwd_fused_unpack(packed, dy, bits, N, G, group_size):
    """-> bf16 dx = dy * mask, shaped like dy (kernel_registration.py:74-94)."""
    _bits_consts(bits, group_size)
    if dy.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"relu_bwd_fused_unpack: unsupported dy dtype {dy.dtype}")
    if dy.numel() != N * G * group_size:
        raise RuntimeError(f"relu_bwd_fused_unpack: dy has {dy.numel()} elements, expected {N * G * group_size}")
    if packed.numel() * packed.element_size() * 8 < dy.numel() * bits:
        raise RuntimeError(f"relu_bwd_fused_unpack: packed holds {packed.numel() * packed.element_size()} bytes, "
                           f"too few for {dy.numel()} {bits}-bit masks")
    _require_cuda(packed, dy)
    packed = _aligned(packed)
    dy = _aligned(dy)
    dx = torch.empty(dy.shape, dtype=torch.bfloat16, device=dy.device)
    rc = _lib.lib().dopt_relu_unpack(packed.data_ptr(), dy.data_ptr(), _DTYPE_CODE[dy.dtype], dy.numel(), bits,
                                     dx.data_ptr(), _stream(dy))
    _lib.check(rc, "relu_bwd_fused_unpack")
    return dx


relu_bwd_fused_unpack = _op(
    "relu_bwd_fused_unpack(Tensor packed, Tensor dy, int bits, int N, int G, int group_size) -> Tensor",
    _relu_bwd_fused_unpack,
    lambda packed, dy, bits, N, G, group_size: torch.empty_like(dy, dtype=torch.bfloat16))


def _act_forward(x, act):
    if x.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"unsupported input dtype {x.dtype}")
    _require_cuda(x)
    x = _aligned(x)
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    d = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().dopt_act_forward(x.data_ptr(), _DTYPE_CODE[x.dtype], x.numel(), act, y.data_ptr(), d.data_ptr(),
                                     _stream(x))
    _lib.check(rc, "act_forward")
    return y, d


def _bf16_pair(x):
    return torch.empty_like(x, dtype=torch.bfloat16), torch.empty_like(x, dtype=torch.bfloat16)


silu_triton = _op("silu_triton(Tensor x) -> (Tensor, Tensor)", lambda x: _act_forward(x, ACT_SILU), _bf16_pair)
gelu_triton = _op("gelu_triton(Tensor x) -> (Tensor, Tensor)", lambda x: _act_forward(x, ACT_GELU), _bf16_pair)


def _group_pact_clamp_fwd(x, alpha):
    """-> (bf16 clamp(x, -alpha, alpha), int8 mask |x| <= alpha), both shaped like x
    (AC/modules/ops.py:587-603)."""
    if x.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"group_pact_clamp_fwd: unsupported dtype {x.dtype}")
    _require_cuda(x)
    x = _aligned(x)
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    mask = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    rc = _lib.lib().dopt_pact_clamp_forward(x.data_ptr(), _DTYPE_CODE[x.dtype], x.numel(), float(alpha), y.data_ptr(),
                                            mask.data_ptr(), _stream(x))
    _lib.check(rc, "group_pact_clamp_fwd")
    return y, mask


def _group_pact_clamp_bwd(mask, alpha, dy):
    """-> bf16 dx = dy where mask != 0, else 0, shaped like dy; alpha is not used (as in the
    reference, AC/modules/ops.py:606-622)."""
    if dy.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"group_pact_clamp_bwd: unsupported dy dtype {dy.dtype}")
    if mask.dtype != torch.int8 or mask.numel() != dy.numel():
        raise RuntimeError(f"group_pact_clamp_bwd: mask must be int8 with dy's {dy.numel()} elements, "
                           f"got {mask.dtype} with {mask.numel()}")
    _require_cuda(mask, dy)
    mask = _aligned(mask).view(dy.shape)
    dy = _aligned(dy)
    dx = torch.empty(dy.shape, dtype=torch.bfloat16, device=dy.device)
    rc = _lib.lib().dopt_pact_clamp_backward(mask.data_ptr(), dy.data_ptr(), _DTYPE_CODE[dy.dtype], dy.numel(),
                                             dx.data_ptr(), _stream(dy))
    _lib.check(rc, "group_pact_clamp_bwd")
    return dx


group_pact_clamp_fwd = _op(
    "group_pact_clamp_fwd(Tensor x, float alpha) -> (Tensor, Tensor)", _group_pact_clamp_fwd,
    lambda x, alpha: (torch.empty_like(x, dtype=torch.bfloat16), torch.empty_like(x, dtype=torch.int8)))
group_pact_clamp_bwd = _op(
    "group_pact_clamp_bwd(Tensor mask, float alpha, Tensor dy) -> Tensor", _group_pact_clamp_bwd,
    lambda mask, alpha, dy: torch.empty_like(dy, dtype=torch.bfloat16))


def _act_quant_pack_launch(x, act, n_groups, bits, group_size, tile):
    _, nwords, _ = _bits_consts(bits, group_size)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"fused activation quant-pack: input must be bfloat16 or float32, got {x.dtype}")
    _require_cuda(x)
    x = _aligned(x)
    y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
    packed = torch.empty((n_groups, nwords), dtype=torch.int32, device=x.device)
    scale = torch.empty((n_groups,), dtype=torch.bfloat16, device=x.device)  # every group's written
    xmin = torch.empty((n_groups,), dtype=torch.bfloat16, device=x.device)
    tile_arr = None
    if tile is not None:
        import ctypes
        tile_arr = (ctypes.c_int64 * 4)(*tile)
    rc = _lib.lib().dopt_act_quant_pack(x.data_ptr(), _DTYPE_CODE[x.dtype], act, n_groups, group_size, bits, tile_arr,
                                        y.data_ptr(), packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), _lib.BF16,
                                        _stream(x))
    _lib.check(rc, "act_quant_pack")
    return y, packed, scale, xmin


def _act_dequant_mul_launch(packed, dy, scale, xmin, n_groups, bits, group_size, tile, alam_seed=None):
    _bits_consts(bits, group_size)
    if dy.dtype not in (torch.bfloat16, torch.float32):
        raise RuntimeError(f"fused activation backward: dy must be bfloat16 or float32, got {dy.dtype}")
    if scale.dtype not in _META_CODE or xmin.dtype != scale.dtype:
        raise RuntimeError("fused activation backward: scale and min must both be float32 or both bfloat16")
    if dy.numel() != n_groups * group_size:
        raise RuntimeError(f"fused activation backward: dy has {dy.numel()} elements, expected {n_groups * group_size}")
    _, nwords, _ = _bits_consts(bits, group_size)
    if scale.numel() != n_groups or xmin.numel() != n_groups or \
            packed.numel() * packed.element_size() != n_groups * nwords * 4:
        raise RuntimeError(f"fused activation backward: packed / scale / min do not hold {n_groups} groups")
    _require_cuda(packed, dy, scale, xmin)
    packed = _aligned(packed)
    dy = _aligned(dy)
    dx = torch.empty(dy.shape, dtype=torch.bfloat16, device=dy.device)
    tile_arr = None
    if tile is not None:
        import ctypes
        tile_arr = (ctypes.c_int64 * 4)(*tile)
    if alam_seed is None:
        rc = _lib.lib().dopt_act_dequant_mul(packed.data_ptr(), scale.contiguous().data_ptr(),
                                             xmin.contiguous().data_ptr(), _META_CODE[scale.dtype], n_groups,
                                             group_size, bits, tile_arr, dy.data_ptr(), _DTYPE_CODE[dy.dtype],
                                             dx.data_ptr(), _stream(dy))
    else:
        rc = _lib.lib().dopt_act_dequant_mul_alam(packed.data_ptr(), scale.contiguous().data_ptr(),
                                                  xmin.contiguous().data_ptr(), _META_CODE[scale.dtype], n_groups,
                                                  group_size, bits, tile_arr, dy.data_ptr(), _DTYPE_CODE[dy.dtype],
                                                  alam_seed, dx.data_ptr(), _stream(dy))
    _lib.check(rc, "act_dequant_mul")
    return dx


def _gelu_fwd_fused_quan_pack(x, bits, group_size):
    """-> (bf16 y shaped like x, packed [N*G, W], bf16 scale [N*G], bf16 min [N*G], N, G); flat
    [N, -1, g] grouping (kernel_registration.py:261-292)."""
    N, G = _flat_groups(x, group_size)
    y, packed, scale, xmin = _act_quant_pack_launch(x, ACT_GELU, N * G, bits, group_size, None)
    return y, packed, scale, xmin, N, G


def _gelu_fwd_fused_quan_pack_fake(x, bits, group_size):
    N, G = _flat_groups(x, group_size)
    nw = _bits_consts(bits, group_size)[1]
    return (torch.empty_like(x, dtype=torch.bfloat16), x.new_empty((N * G, nw), dtype=torch.int32),
            x.new_empty((N * G,), dtype=torch.bfloat16), x.new_empty((N * G,), dtype=torch.bfloat16), N, G)


gelu_fwd_fused_quan_pack = _op(
    "gelu_fwd_fused_quan_pack(Tensor x, int bits, int group_size) -> (Tensor, Tensor, Tensor, Tensor, int, int)",
    _gelu_fwd_fused_quan_pack, _gelu_fwd_fused_quan_pack_fake)


def _gelu_bwd_fused_dequan_unpack(packed, dy, scale, min, bits, N, G, group_size):
    """-> bf16 dx = dy * dequant(packed), shaped like dy (kernel_registration.py:295-319)."""
    return _act_dequant_mul_launch(packed, dy, scale, min, N * G, bits, group_size, None)


gelu_bwd_fused_dequan_unpack = _op(
    "gelu_bwd_fused_dequan_unpack(Tensor packed, Tensor dy, Tensor scale, Tensor min, int bits, int N, int G, "
    "int group_size) -> Tensor",
    _gelu_bwd_fused_dequan_unpack,
    lambda packed, dy, scale, min, bits, N, G, group_size: torch.empty_like(dy, dtype=torch.bfloat16))


def _silu_layout(x, group_size):
    """(N, G, new_H, new_W, pad_elig, reshape_elig, tile) of the reference's spatial-aware grouping
    (tensor_act_reshape_utils.py:100-128), without materialising it."""
    from .modules.tensor_act_reshape_utils import tile_layout_applies

    if tile_layout_applies(x, group_size, False):
        n, c, h, w = (int(v) for v in x.shape)
        s = int(round(group_size ** 0.5))
        return n, c * (h // s) * (w // s), h // s, w // s, False, True, (n, c, h, w)
    N, G = _flat_groups(x, group_size)
    return N, G, 0, 0, False, False, None


def _silu_fwd_quan_pack(x, bits, group_size, avg_alam, alam_bits, pack_only):
    """-> (bf16 y shaped like x, packed, bf16 scale [N*G], bf16 min [N*G], N, G, new_H, new_W,
    padding eligibility, reshape eligibility) (kernel_registration.py:148-198); the spatial-tile
    grouping is read and written in place."""
    _silu_alam(avg_alam, alam_bits, "silu_fwd_quan_pack")  # alam_bits = 1: the plain codes
    N, G, nh, nw, pad_e, rs_e, tile = _silu_layout(x, group_size)
    y, packed, scale, xmin = _act_quant_pack_launch(x, ACT_SILU, N * G, bits, group_size, tile)
    return y, packed, scale, xmin, N, G, nh, nw, pad_e, rs_e


def _silu_fwd_quan_pack_fake(x, bits, group_size, avg_alam, alam_bits, pack_only):
    N, G, nh, nw, pad_e, rs_e, _ = _silu_layout(x, group_size)
    nwords = _bits_consts(bits, group_size)[1]
    return (torch.empty_like(x, dtype=torch.bfloat16), x.new_empty((N * G, nwords), dtype=torch.int32),
            x.new_empty((N * G,), dtype=torch.bfloat16), x.new_empty((N * G,), dtype=torch.bfloat16), N, G, nh, nw,
            pad_e, rs_e)


silu_fwd_quan_pack = _op(
    "silu_fwd_quan_pack(Tensor x, int bits, int group_size, bool avg_alam, int alam_bits, bool pack_only) -> "
    "(Tensor, Tensor, Tensor, Tensor, int, int, int, int, bool, bool)",
    _silu_fwd_quan_pack, _silu_fwd_quan_pack_fake)


def _silu_bwd_fused_dequan_unpack(packed, dy, scale, min, bits, N, G, group_size, pack_only, new_H, new_W,
                                  spatical_padding_eligibility, spatical_reshape_eligibility, avg_alam, alam_bits):
    """-> bf16 dx = dy * dequant(packed), shaped like dy (kernel_registration.py:202-237); with
    avg_alam (alam_bits = 1) the codes carry tl.rand(42 + group, element) - 0.5 (seed 42, :208)."""
    noise = _silu_alam(avg_alam, alam_bits, "silu_bwd_fused_dequan_unpack")
    tile = tuple(int(v) for v in dy.shape) if spatical_reshape_eligibility else None
    return _act_dequant_mul_launch(packed, dy, scale, min, N * G, bits, group_size, tile,
                                   ALAM_SEED if noise else None)


silu_bwd_fused_dequan_unpack = _op(
    "silu_bwd_fused_dequan_unpack(Tensor packed, Tensor dy, Tensor scale, Tensor min, int bits, int N, int G, "
    "int group_size, bool pack_only, int new_H, int new_W, bool spatical_padding_eligibility, "
    "bool spatical_reshape_eligibility, bool avg_alam, int alam_bits) -> Tensor",
    _silu_bwd_fused_dequan_unpack,
    lambda packed, dy, scale, min, bits, N, G, group_size, pack_only, new_H, new_W, pe, re, aa, ab:
        torch.empty_like(dy, dtype=torch.bfloat16))
