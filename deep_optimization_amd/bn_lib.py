"""BatchNorm operators of ``torch.ops.act_lib``: statistics, normalize + quant-pack, and the
backward reduce / input gradient, on the gfx950 kernels behind the C ABI (dopt_bn_*).

Same names, schemas and outputs as the reference's Triton operators:
  Activation_Compression/modules/normalization/kernel_registration.py:13-276
    bn_fwd_reduce, bn_fwd_norm, bn_fwd_norm_quant_pack_fused, bn_bwd_reduce, bn_bwd_dx,
    bn_bwd_reduce_dequant_unpack_fused, bn_bwd_dx_dequant_unpack_fused
  Activation_Compression/triton_kernel/norm_act_fusion/kernel_registration.py:19-166
    bn_relu_fwd_norm_fused_quant_pack, bn_relu_bwd_reduce_fused_dequant_unpack,
    bn_relu_bwd_dx_fused_dequant_unpack
Launch-tuning arguments (num_warps, num_stages) are accepted and ignored. As in the reference,
the fused quant-pack groups are BLOCK_M // 2 elements of a channel, the constants eps are the
kernels' own (1e-5 in the fused forwards and the BatchNorm+ReLU backward, 1e-7 in the plain
normalize and the DOBatchNorm backward), and with ``sync`` the ``var`` argument carries the
inverse standard deviation. Every element tensor is made contiguous [N, C, HW] first (the
reference's callers pass ``input.view(N, C, HW)``, which already is).

Differences from the reference: sums are deterministic (ordered two-stage reduction, where the
reference accumulates fp32 atomics); relu6 clamps y to [0, 6] (the reference's fused kernel
writes 0 for y >= 6, bn_act_fusion.py:73-75).

avg_alam (the squashed operators): one code per run of alam_bits elements, the truncated mean of
the run's code arguments; packed [C, M * bits / 32 / alam_bits]; the backward reduce adds the
reference's tl.rand noise to the codes, the input gradient does not
(kernel_implementation.py:194-237, :374-391, :455-462).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _lib
from .act_lib import _DTYPE_CODE, _alam_words, _bits_consts, _op, _require_cuda, _stream

EPS_FUSED = 1e-5
EPS_PLAIN = 1e-7


def _geom(X: Tensor, M: int, HW: int):
    """-> (X3 contiguous [N, C, HW], N, C). M = N * HW must match X."""
    if X.dim() < 2:
        raise RuntimeError(f"BatchNorm operators expect an [N, C, ...] tensor, got {tuple(X.shape)}")
    N, C = int(X.shape[0]), int(X.shape[1])
    hw = X.numel() // max(N * C, 1) if N * C else int(HW)
    if hw != HW or N * HW != M:
        raise RuntimeError(f"BatchNorm operator: X of shape {tuple(X.shape)} does not match M={M}, HW={HW}")
    return X.contiguous().view(N, C, HW), N, C


def _f32(t: Optional[Tensor]) -> Optional[Tensor]:
    if t is None or (t.dtype == torch.float32 and t.is_contiguous()):
        return t
    return t.detach().contiguous().to(torch.float32)


def _ptr(t: Optional[Tensor]):
    return None if t is None else t.data_ptr()


def _workspace(X: Tensor, N: int, C: int, HW: int) -> Tensor:
    n = int(_lib.lib().dopt_bn_workspace_floats(N, C, HW))
    return torch.empty(max(n, 1), dtype=torch.float32, device=X.device)


def _alam_run(avg_alam: bool, alam_bits: int, group: int, bits: int) -> int:
    """avg_alam's elements per code, alam_bits (checked as the reference's reshape needs it), or 0
    without avg_alam. alam_bits = 1 keeps the plain codes, but the backward reduce still adds the
    reference's noise."""
    if not avg_alam:
        return 0
    _alam_words(bits, group, alam_bits)
    return int(alam_bits)


def _group(BLOCK: int) -> int:
    g = BLOCK // 2
    if g < 32 or g > 512 or g & (g - 1):
        raise RuntimeError(f"BLOCK_M // 2 must be a power of two in [32, 512], got BLOCK_M={BLOCK}")
    return g


# ------------------------------------------------------------------ forward
def _bn_fwd_reduce(X, *, M, HW, stride_n, stride_c, BLOCK_M, num_warps, num_stages):
    """-> (sum, sum of squares) fp32 [C] (kernel_registration.py:13-39)."""
    _require_cuda(X)
    X3, N, C = _geom(X, M, HW)
    s = torch.empty(C, dtype=torch.float32, device=X.device)
    q = torch.empty_like(s)
    ws = _workspace(X, N, C, HW)
    rc = _lib.lib().dopt_bn_reduce(X3.data_ptr(), _DTYPE_CODE[X3.dtype], N, C, HW, C * HW, HW, ws.data_ptr(),
                                   s.data_ptr(), q.data_ptr(), _stream(X))
    _lib.check(rc, "bn_fwd_reduce")
    return s, q


def _bn_fwd_reduce_fake(X, *, M, HW, stride_n, stride_c, BLOCK_M, num_warps, num_stages):
    C = X.shape[1]
    return X.new_empty((C,), dtype=torch.float32), X.new_empty((C,), dtype=torch.float32)


bn_fwd_reduce = _op(
    "bn_fwd_reduce(Tensor X, *, int M, int HW, int stride_n, int stride_c, int BLOCK_M, int num_warps, "
    "int num_stages) -> (Tensor, Tensor)", _bn_fwd_reduce, _bn_fwd_reduce_fake)


def _norm_launch(X, SUM, SUM_SQUARE, GAMMA, BETA, mean, var, M, HW, sync, mode, group, bits, eps, alam=0):
    _require_cuda(X, GAMMA, BETA)
    X3, N, C = _geom(X, M, HW)
    dev = X.device
    y = torch.empty(X3.shape, dtype=torch.bfloat16, device=dev)
    quant = mode != _lib.BN_NORM
    x_hat = None if quant else torch.empty(X3.shape, dtype=torch.bfloat16, device=dev)
    packed = relu_packed = scale = xmin = None
    if quant:
        packed = torch.empty((C, M * bits // 32 // max(alam, 1)), dtype=torch.int32, device=dev)
        scale = torch.empty((C, M // group), dtype=torch.bfloat16, device=dev)
        xmin = torch.empty_like(scale)
        if mode in (_lib.BN_RELU_QUANT, _lib.BN_RELU6_QUANT):
            relu_packed = torch.empty((C, M // 32), dtype=torch.int32, device=dev)
    used = (("weight", GAMMA), ("bias", BETA)) + ((("mean", mean), ("var", var)) if sync else
                                                   (("sum", SUM), ("sum of squares", SUM_SQUARE)))
    for name, t in used:
        if t is not None and t.numel() != C:  # the kernels read one value per channel
            raise RuntimeError(f"BatchNorm forward: {name} must hold {C} values (one per channel), got {t.numel()}")
    w, b = _f32(GAMMA), _f32(BETA)
    if sync:
        if mean is None or var is None:
            raise RuntimeError("sync=True needs mean and var (the inverse std)")
        mean_in, inv_in = _f32(mean), _f32(var)
        s = q = mean_out = var_out = None
    else:
        s, q = _f32(SUM), _f32(SUM_SQUARE)
        mean_in = inv_in = None
        mean_out = torch.empty(C, dtype=torch.float32, device=dev)
        var_out = torch.empty_like(mean_out)
    if alam:
        rc = _lib.lib().dopt_bn_norm_quant_alam(
            X3.data_ptr(), _DTYPE_CODE[X3.dtype], N, C, HW, C * HW, HW, _ptr(s), _ptr(q), _ptr(mean_in),
            _ptr(inv_in), int(bool(sync)), w.data_ptr(), b.data_ptr(), float(eps), group, bits, alam, y.data_ptr(),
            _ptr(packed), _ptr(scale), _ptr(xmin), _ptr(mean_out), _ptr(var_out), _stream(X))
    else:
        rc = _lib.lib().dopt_bn_norm_quant(
            X3.data_ptr(), _DTYPE_CODE[X3.dtype], N, C, HW, C * HW, HW, _ptr(s), _ptr(q), _ptr(mean_in),
            _ptr(inv_in), int(bool(sync)), w.data_ptr(), b.data_ptr(), float(eps), mode, group, bits, y.data_ptr(),
            _ptr(x_hat), _ptr(packed), _ptr(relu_packed), _ptr(scale), _ptr(xmin), _ptr(mean_out), _ptr(var_out),
            _stream(X))
    _lib.check(rc, "bn normalize")
    return y, x_hat, packed, relu_packed, scale, xmin, mean_out, var_out


def _bn_fwd_norm(X, SUM, SUM_SQUARE, GAMMA, BETA, mean=None, var=None, *, M, HW, stride_n, stride_c, BLOCK_M, sync,
                 num_warps, num_stages):
    """-> (y bf16, x_hat bf16, mean, var) (kernel_registration.py:42-80); eps 1e-7."""
    y, x_hat, _, _, _, _, mo, vo = _norm_launch(X, SUM, SUM_SQUARE, GAMMA, BETA, mean, var, M, HW, sync,
                                                _lib.BN_NORM, 0, 1, EPS_PLAIN)
    return y, x_hat, mo, vo


def _bn_fwd_norm_fake(X, SUM, SUM_SQUARE, GAMMA, BETA, mean=None, var=None, *, M, HW, stride_n, stride_c, BLOCK_M,
                      sync, num_warps, num_stages):
    N, C = X.shape[0], X.shape[1]
    y = X.new_empty((N, C, HW), dtype=torch.bfloat16)
    st = None if sync else X.new_empty((C,), dtype=torch.float32)
    return y, torch.empty_like(y), st, None if sync else torch.empty_like(st)


bn_fwd_norm = _op(
    "bn_fwd_norm(Tensor X, Tensor? SUM, Tensor? SUM_SQUARE, Tensor GAMMA, Tensor BETA, Tensor? mean=None, "
    "Tensor? var=None, *, int M, int HW, int stride_n, int stride_c, int BLOCK_M, bool sync, int num_warps, "
    "int num_stages) -> (Tensor, Tensor, Tensor?, Tensor?)", _bn_fwd_norm, _bn_fwd_norm_fake)


def _bn_fwd_norm_quant_pack_fused(X, SUM, SUM_SQUARE, GAMMA, BETA, mean=None, var=None, *, M, HW, stride_n, stride_c,
                                  BLOCK_M, bits, sync, avg_alam, alam_bits, num_warps, num_stages):
    """-> (y bf16, packed [C, M*bits/32] (/ alam_bits with avg_alam), scale, min bf16
    [C, M/(BLOCK_M/2)], mean, var) (kernel_registration.py:83-150); eps 1e-5, codes of
    2 tanh(clamp(x_hat, -3, 3)/2)."""
    g = _group(BLOCK_M)
    _bits_consts(bits, g)
    alam = _alam_run(avg_alam, alam_bits, g, bits)
    y, _, packed, _, scale, xmin, mo, vo = _norm_launch(X, SUM, SUM_SQUARE, GAMMA, BETA, mean, var, M, HW, sync,
                                                        _lib.BN_QUANT, g, bits, EPS_FUSED, alam)
    return y, packed, scale, xmin, mo, vo


def _quant_fakes(X, M, HW, g, bits, sync, alam=0):
    N, C = X.shape[0], X.shape[1]
    y = X.new_empty((N, C, HW), dtype=torch.bfloat16)
    packed = X.new_empty((C, M * bits // 32 // max(alam, 1)), dtype=torch.int32)
    scale = X.new_empty((C, M // g), dtype=torch.bfloat16)
    st = None if sync else X.new_empty((C,), dtype=torch.float32)
    return y, packed, scale, st


def _bn_fwd_norm_quant_pack_fused_fake(X, SUM, SUM_SQUARE, GAMMA, BETA, mean=None, var=None, *, M, HW, stride_n,
                                       stride_c, BLOCK_M, bits, sync, avg_alam, alam_bits, num_warps, num_stages):
    y, packed, scale, st = _quant_fakes(X, M, HW, BLOCK_M // 2, bits, sync,
                                        _alam_run(avg_alam, alam_bits, BLOCK_M // 2, bits))
    return y, packed, scale, torch.empty_like(scale), st, None if sync else torch.empty_like(st)


bn_fwd_norm_quant_pack_fused = _op(
    "bn_fwd_norm_quant_pack_fused(Tensor X, Tensor? SUM, Tensor? SUM_SQUARE, Tensor GAMMA, Tensor BETA, "
    "Tensor? mean=None, Tensor? var=None, *, int M, int HW, int stride_n, int stride_c, int BLOCK_M, int bits, "
    "bool sync, bool avg_alam, int alam_bits, int num_warps, int num_stages) -> "
    "(Tensor, Tensor, Tensor, Tensor, Tensor?, Tensor?)",
    _bn_fwd_norm_quant_pack_fused, _bn_fwd_norm_quant_pack_fused_fake)


def _bn_relu_fwd_norm_fused_quant_pack(X, Sum, Sum_Square, Weight, Bias, mean=None, var=None, *, M, HW, stride_n,
                                       stride_c, relu, relu6, BLOCK_SIZE, BITS, sync):
    """-> (y bf16, x_hat packed, relu mask packed [C, M/32], scale, min, mean, var)
    (norm_act_fusion/kernel_registration.py:19-74); eps 1e-5, codes of x_hat itself."""
    if not (relu or relu6):
        raise RuntimeError("bn_relu_fwd_norm_fused_quant_pack needs relu or relu6")
    g = _group(BLOCK_SIZE)
    _bits_consts(BITS, g)
    mode = _lib.BN_RELU_QUANT if relu else _lib.BN_RELU6_QUANT
    y, _, packed, rp, scale, xmin, mo, vo = _norm_launch(X, Sum, Sum_Square, Weight, Bias, mean, var, M, HW, sync,
                                                         mode, g, BITS, EPS_FUSED)
    return y, packed, rp, scale, xmin, mo, vo


def _bn_relu_fwd_fake(X, Sum, Sum_Square, Weight, Bias, mean=None, var=None, *, M, HW, stride_n, stride_c, relu,
                      relu6, BLOCK_SIZE, BITS, sync):
    y, packed, scale, st = _quant_fakes(X, M, HW, BLOCK_SIZE // 2, BITS, sync)
    rp = X.new_empty((X.shape[1], M // 32), dtype=torch.int32)
    return y, packed, rp, scale, torch.empty_like(scale), st, None if sync else torch.empty_like(st)


bn_relu_fwd_norm_fused_quant_pack = _op(
    "bn_relu_fwd_norm_fused_quant_pack(Tensor X, Tensor? Sum, Tensor? Sum_Square, Tensor Weight, Tensor Bias, "
    "Tensor? mean=None, Tensor? var=None, *, int M, int HW, int stride_n, int stride_c, bool relu, bool relu6, "
    "int BLOCK_SIZE, int BITS, bool sync) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor?, Tensor?)",
    _bn_relu_fwd_norm_fused_quant_pack, _bn_relu_fwd_fake)


# ------------------------------------------------------------------ backward
def _bwd_common(mode, DY, M, HW, x_hat=None, packed=None, relu_packed=None, scale=None, xmin=None):
    _require_cuda(DY)
    DY3, N, C = _geom(DY, M, HW)
    xh = None if x_hat is None else _geom(x_hat, M, HW)[0].to(torch.bfloat16).contiguous()
    c = lambda t: None if t is None else t.contiguous()  # noqa: E731
    return DY3, N, C, xh, c(packed), c(relu_packed), c(scale), c(xmin)


def _check_saved(C, M, group, bits, p, rp, sc, mn, *vecs, alam=0):
    """The kernels read the saved tensors unchecked: their sizes must match the channel layout."""
    a = max(alam, 1)
    if p is not None and p.numel() * p.element_size() * 8 * a != C * M * bits:
        raise RuntimeError(f"BatchNorm backward: packed codes hold {p.numel() * p.element_size()} bytes, "
                           f"expected {C * M * bits // 8 // a}")
    if rp is not None and rp.numel() * rp.element_size() * 8 < C * M:
        raise RuntimeError("BatchNorm backward: the ReLU mask is too small for the tensor")
    for t in (sc, mn):
        if t is not None and t.numel() != C * (M // group):
            raise RuntimeError(f"BatchNorm backward: scale/min hold {t.numel()} values, expected {C * (M // group)}")
    for t in vecs:
        if t is not None and t.numel() != C:
            raise RuntimeError(f"BatchNorm backward: per-channel vectors must hold {C} values, got {t.numel()}")


def _bwd_reduce(mode, DY, M, HW, group, bits, alam=0, **kw):
    DY3, N, C, xh, p, rp, sc, mn = _bwd_common(mode, DY, M, HW, **kw)
    _check_saved(C, M, group, bits, p, rp, sc, mn, alam=alam)
    dw = torch.empty(C, dtype=torch.float32, device=DY.device)
    db = torch.empty_like(dw)
    ws = _workspace(DY, N, C, HW)
    if alam:
        rc = _lib.lib().dopt_bn_bwd_reduce_alam(_ptr(p), _ptr(sc), _ptr(mn), DY3.data_ptr(), _DTYPE_CODE[DY3.dtype], N,
                                                C, HW, C * HW, HW, group, bits, alam, ws.data_ptr(), dw.data_ptr(),
                                                db.data_ptr(), _stream(DY))
    else:
        rc = _lib.lib().dopt_bn_bwd_reduce(mode, _ptr(xh), _ptr(p), _ptr(rp), _ptr(sc), _ptr(mn), DY3.data_ptr(),
                                           _DTYPE_CODE[DY3.dtype], N, C, HW, C * HW, HW, group, bits, ws.data_ptr(),
                                           dw.data_ptr(), db.data_ptr(), _stream(DY))
    _lib.check(rc, "bn backward reduce")
    return dw, db


def _bwd_dx(mode, DY, M, HW, group, bits, DW, DB, W, VAR, eps, var_is_invstd, alam=0, **kw):
    DY3, N, C, xh, p, rp, sc, mn = _bwd_common(mode, DY, M, HW, **kw)
    dx = torch.empty(DY3.shape, dtype=torch.bfloat16, device=DY.device)
    dw, db, w, v = _f32(DW), _f32(DB), _f32(W), _f32(VAR)
    _check_saved(C, M, group, bits, p, rp, sc, mn, dw, db, w, v, alam=alam)
    if alam:
        rc = _lib.lib().dopt_bn_bwd_dx_alam(_ptr(p), _ptr(sc), _ptr(mn), DY3.data_ptr(), _DTYPE_CODE[DY3.dtype], N, C,
                                            HW, C * HW, HW, group, bits, alam, dw.data_ptr(), db.data_ptr(),
                                            w.data_ptr(), v.data_ptr(), float(eps), int(bool(var_is_invstd)),
                                            dx.data_ptr(), _stream(DY))
    else:
        rc = _lib.lib().dopt_bn_bwd_dx(mode, _ptr(xh), _ptr(p), _ptr(rp), _ptr(sc), _ptr(mn), DY3.data_ptr(),
                                       _DTYPE_CODE[DY3.dtype], N, C, HW, C * HW, HW, group, bits, dw.data_ptr(),
                                       db.data_ptr(), w.data_ptr(), v.data_ptr(), float(eps),
                                       int(bool(var_is_invstd)), dx.data_ptr(), _stream(DY))
    _lib.check(rc, "bn backward dx")
    return dx


def _reduce_fake(DY):
    C = DY.shape[1]
    return DY.new_empty((C,), dtype=torch.float32), DY.new_empty((C,), dtype=torch.float32)


def _bn_bwd_reduce(X, DY, *, M, HW, stride_n, stride_c, BLOCK_M, num_warps, num_stages):
    """X = bf16 x_hat -> (dgamma, dbeta) (kernel_registration.py:153-178)."""
    return _bwd_reduce(_lib.BN_NORM, DY, M, HW, 0, 1, x_hat=X)


bn_bwd_reduce = _op(
    "bn_bwd_reduce(Tensor X, Tensor DY, *, int M, int HW, int stride_n, int stride_c, int BLOCK_M, int num_warps, "
    "int num_stages) -> (Tensor, Tensor)", _bn_bwd_reduce,
    lambda X, DY, *, M, HW, stride_n, stride_c, BLOCK_M, num_warps, num_stages: _reduce_fake(DY))


def _bn_bwd_dx(X, DY, VAR, GAMMA, DBETA, DGAMMA, *, M, HW, stride_n, stride_c, BLOCK_M, sync, num_warps, num_stages):
    """-> bf16 dx [N, C, HW] (kernel_registration.py:181-208); eps 1e-7, VAR = invstd with sync."""
    return _bwd_dx(_lib.BN_NORM, DY, M, HW, 0, 1, DGAMMA, DBETA, GAMMA, VAR, EPS_PLAIN, sync, x_hat=X)


bn_bwd_dx = _op(
    "bn_bwd_dx(Tensor X, Tensor DY, Tensor VAR, Tensor GAMMA, Tensor DBETA, Tensor DGAMMA, *, int M, int HW, "
    "int stride_n, int stride_c, int BLOCK_M, bool sync, int num_warps, int num_stages) -> Tensor", _bn_bwd_dx,
    lambda X, DY, VAR, GAMMA, DBETA, DGAMMA, *, M, HW, stride_n, stride_c, BLOCK_M, sync, num_warps, num_stages:
        DY.new_empty((DY.shape[0], DY.shape[1], HW), dtype=torch.bfloat16))


def _bn_bwd_reduce_dequant_unpack_fused(x_hat_packed, dy, scale, min, *, M, HW, stride_n, stride_c, BLOCK_M, bits,
                                        avg_alam, alam_bits):
    """-> (DW, DB) (kernel_registration.py:211-240)."""
    g = _group(BLOCK_M)
    _bits_consts(bits, g)
    return _bwd_reduce(_lib.BN_QUANT, dy, M, HW, g, bits, _alam_run(avg_alam, alam_bits, g, bits),
                       packed=x_hat_packed, scale=scale, xmin=min)


bn_bwd_reduce_dequant_unpack_fused = _op(
    "bn_bwd_reduce_dequant_unpack_fused(Tensor x_hat_packed, Tensor dy, Tensor scale, Tensor min, *, int M, int HW, "
    "int stride_n, int stride_c, int BLOCK_M, int bits, bool avg_alam, int alam_bits) -> (Tensor, Tensor)",
    _bn_bwd_reduce_dequant_unpack_fused,
    lambda x_hat_packed, dy, scale, min, *, M, HW, stride_n, stride_c, BLOCK_M, bits, avg_alam, alam_bits:
        _reduce_fake(dy))


def _bn_bwd_dx_dequant_unpack_fused(x_hat_packed, dy, scale, min, DW, DB, W, VAR, *, M, HW, stride_n, stride_c,
                                    BLOCK_M, bits, sync, avg_alam, alam_bits):
    """-> bf16 dx [N, C, HW] (kernel_registration.py:243-276); eps 1e-7, VAR = invstd with sync."""
    g = _group(BLOCK_M)
    _bits_consts(bits, g)
    return _bwd_dx(_lib.BN_QUANT, dy, M, HW, g, bits, DW, DB, W, VAR, EPS_PLAIN, sync,
                   _alam_run(avg_alam, alam_bits, g, bits), packed=x_hat_packed, scale=scale, xmin=min)


bn_bwd_dx_dequant_unpack_fused = _op(
    "bn_bwd_dx_dequant_unpack_fused(Tensor x_hat_packed, Tensor dy, Tensor scale, Tensor min, Tensor DW, Tensor DB, "
    "Tensor W, Tensor VAR, *, int M, int HW, int stride_n, int stride_c, int BLOCK_M, int bits, bool sync, "
    "bool avg_alam, int alam_bits) -> Tensor", _bn_bwd_dx_dequant_unpack_fused,
    lambda x_hat_packed, dy, scale, min, DW, DB, W, VAR, *, M, HW, stride_n, stride_c, BLOCK_M, bits, sync, avg_alam,
    alam_bits: dy.new_empty((dy.shape[0], dy.shape[1], HW), dtype=torch.bfloat16))


def _bn_relu_bwd_reduce(X_hat_packed, ReLU_mask_packed, DY, Scale, Min, *, M, HW, stride_n, stride_c, BLOCK_SIZE,
                        BITS):
    """-> (DW, DB) over dy * mask (norm_act_fusion/kernel_registration.py:77-119)."""
    g = _group(BLOCK_SIZE)
    _bits_consts(BITS, g)
    return _bwd_reduce(_lib.BN_RELU_QUANT, DY, M, HW, g, BITS, packed=X_hat_packed, relu_packed=ReLU_mask_packed,
                       scale=Scale, xmin=Min)


bn_relu_bwd_reduce_fused_dequant_unpack = _op(
    "bn_relu_bwd_reduce_fused_dequant_unpack(Tensor X_hat_packed, Tensor ReLU_mask_packed, Tensor DY, Tensor Scale, "
    "Tensor Min, *, int M, int HW, int stride_n, int stride_c, int BLOCK_SIZE, int BITS) -> (Tensor, Tensor)",
    _bn_relu_bwd_reduce,
    lambda X_hat_packed, ReLU_mask_packed, DY, Scale, Min, *, M, HW, stride_n, stride_c, BLOCK_SIZE, BITS:
        _reduce_fake(DY))


def _bn_relu_bwd_dx(X_hat_packed, ReLU_mask_packed, DY, DW, DB, Weight, Var, Scale, Min, *, M, HW, stride_n,
                    stride_c, BLOCK_SIZE, BITS):
    """-> bf16 dx [N, C, HW] (norm_act_fusion/kernel_registration.py:122-166); eps 1e-5."""
    g = _group(BLOCK_SIZE)
    _bits_consts(BITS, g)
    return _bwd_dx(_lib.BN_RELU_QUANT, DY, M, HW, g, BITS, DW, DB, Weight, Var, EPS_FUSED, False,
                   packed=X_hat_packed, relu_packed=ReLU_mask_packed, scale=Scale, xmin=Min)


bn_relu_bwd_dx_fused_dequant_unpack = _op(
    "bn_relu_bwd_dx_fused_dequant_unpack(Tensor X_hat_packed, Tensor ReLU_mask_packed, Tensor DY, Tensor DW, "
    "Tensor DB, Tensor Weight, Tensor Var, Tensor Scale, Tensor Min, *, int M, int HW, int stride_n, int stride_c, "
    "int BLOCK_SIZE, int BITS) -> Tensor", _bn_relu_bwd_dx,
    lambda X_hat_packed, ReLU_mask_packed, DY, DW, DB, Weight, Var, Scale, Min, *, M, HW, stride_n, stride_c,
    BLOCK_SIZE, BITS: DY.new_empty((DY.shape[0], DY.shape[1], HW), dtype=torch.bfloat16))


# ------------------------------------------------------------------ layer operators
# Not in the reference: the compressed BatchNorm layers' training forward and backward, each one
# operator call. The reference's layers issue two operators per pass and update the running
# statistics with four tensor ops (normalization_ops.py:45-57 and :95-157, fused_ops.py:19-86);
# these run the same kernels, the running statistics updated inside the normalize kernel.
_LAYER_EPS = {_lib.BN_QUANT: (EPS_FUSED, EPS_PLAIN), _lib.BN_RELU_QUANT: (EPS_FUSED, EPS_FUSED),
              _lib.BN_RELU6_QUANT: (EPS_FUSED, EPS_FUSED)}  # (forward, backward) as the operators above


def _layer_mode(kind: int) -> int:
    """The kernels' mode for a layer kind (BN_QUANT, BN_RELU_QUANT or BN_RELU6_QUANT; the ReLU6 backward
    is the ReLU one, its mask already marks 0 < y < 6)."""
    if kind not in _LAYER_EPS:
        raise RuntimeError(f"BatchNorm layer operators take kind BN_QUANT, BN_RELU_QUANT or BN_RELU6_QUANT, got {kind}")
    return _lib.BN_RELU_QUANT if kind == _lib.BN_RELU6_QUANT else kind


def _bn_train_fwd(X, weight, bias, running_mean, running_var, momentum, BLOCK_M, bits, kind):
    """X [N, C, ...] -> (y bf16 [N, C, HW], packed [C, M*bits/32], ReLU mask [C, M/32] ([C, 0] without ReLU), scale, min
    bf16 [C, M/g], batch mean, biased batch variance); the running statistics are updated in place:
    run = run * (1 - momentum) + momentum * statistic (an empty tensor stands for no statistic)."""
    _layer_mode(kind)
    running_mean = running_mean if running_mean is not None and running_mean.numel() else None
    running_var = running_var if running_var is not None and running_var.numel() else None
    g = _group(BLOCK_M)
    _bits_consts(bits, g)
    _require_cuda(X, weight, bias, running_mean, running_var)
    if X.dim() < 2 or X.dtype not in _DTYPE_CODE:
        raise RuntimeError(f"bn_train_fwd: X must be an [N, C, ...] float tensor, got {tuple(X.shape)} {X.dtype}")
    N, C = int(X.shape[0]), int(X.shape[1])
    HW = X.numel() // (N * C) if N * C else 0
    X3 = X.contiguous().view(N, C, HW)
    M, dev = N * HW, X.device
    for name, t in (("weight", weight), ("bias", bias), ("running_mean", running_mean), ("running_var", running_var)):
        if t is not None and t.numel() != C:
            raise RuntimeError(f"bn_train_fwd: {name} must hold {C} values (one per channel), got {t.numel()}")
    in_kernel = all(t is None or (t.dtype == torch.float32 and t.is_contiguous()) for t in (running_mean, running_var))
    y = torch.empty((N, C, HW), dtype=torch.bfloat16, device=dev)
    packed = torch.empty((C, M * bits // 32), dtype=torch.int32, device=dev)
    scale = torch.empty((C, M // g), dtype=torch.bfloat16, device=dev)
    xmin = torch.empty_like(scale)
    rp = torch.empty((C, M // 32 if kind != _lib.BN_QUANT else 0), dtype=torch.int32, device=dev)
    mean = torch.empty(C, dtype=torch.float32, device=dev)
    var = torch.empty_like(mean)
    ws = _workspace(X3, N, C, HW)
    w, b = _f32(weight), _f32(bias)
    rm, rv = (running_mean, running_var) if in_kernel else (None, None)
    rc = _lib.lib().dopt_bn_train_forward(
        X3.data_ptr(), _DTYPE_CODE[X3.dtype], N, C, HW, C * HW, HW, ws.data_ptr(), w.data_ptr(), b.data_ptr(),
        _LAYER_EPS[kind][0], kind, g, bits, y.data_ptr(), None,
        packed.data_ptr(), rp.data_ptr() if rp.numel() else None, scale.data_ptr(), xmin.data_ptr(), mean.data_ptr(),
        var.data_ptr(),
        _ptr(rm), _ptr(rv), float(momentum), _stream(X))
    _lib.check(rc, "bn_train_fwd")
    if not in_kernel:
        for run, stat in ((running_mean, mean), (running_var, var)):
            if run is not None:
                run.mul_(1.0 - momentum).add_(stat, alpha=momentum)
    return y, packed, rp, scale, xmin, mean, var


def _bn_train_fwd_fake(X, weight, bias, running_mean, running_var, momentum, BLOCK_M, bits, kind):
    N, C = X.shape[0], X.shape[1]
    HW = X.numel() // (N * C) if N * C else 0
    M, g = N * HW, BLOCK_M // 2
    rp = X.new_empty((C, M // 32 if kind != _lib.BN_QUANT else 0), dtype=torch.int32)
    scale = X.new_empty((C, M // g), dtype=torch.bfloat16)
    return (X.new_empty((N, C, HW), dtype=torch.bfloat16), X.new_empty((C, M * bits // 32), dtype=torch.int32), rp,
            scale, torch.empty_like(scale), X.new_empty((C,), dtype=torch.float32),
            X.new_empty((C,), dtype=torch.float32))


bn_train_fwd = _op(
    "bn_train_fwd(Tensor X, Tensor weight, Tensor bias, Tensor(a!) running_mean, Tensor(b!) running_var, "
    "float momentum, int BLOCK_M, int bits, int kind) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)",
    _bn_train_fwd, _bn_train_fwd_fake)


def _bn_train_bwd(packed, relu_packed, dy, scale, min, weight, var, BLOCK_M, bits, kind):
    """dy [N, C, ...] -> (bf16 dx [N, C, HW], dweight, dbias) of the layer whose forward was bn_train_fwd."""
    m = _layer_mode(kind)
    g = _group(BLOCK_M)
    _bits_consts(bits, g)
    if dy.dim() < 2:
        raise RuntimeError(f"bn_train_bwd: dy must be [N, C, ...], got {tuple(dy.shape)}")
    N, C = int(dy.shape[0]), int(dy.shape[1])
    HW = dy.numel() // (N * C) if N * C else 0
    M = N * HW
    DY3, _, _, _, p, rp, sc, mn = _bwd_common(m, dy, M, HW, packed=packed,
                                              relu_packed=relu_packed if m == _lib.BN_RELU_QUANT else None,
                                              scale=scale, xmin=min)
    if p is None or sc is None or mn is None:
        raise RuntimeError("bn_train_bwd: packed codes, scale and min are required")
    w, v = _f32(weight), _f32(var)
    _check_saved(C, M, g, bits, p, rp, sc, mn, w, v)
    if m == _lib.BN_RELU_QUANT and rp is None:
        raise RuntimeError("bn_train_bwd: the ReLU kinds need the saved ReLU mask")
    dx = torch.empty(DY3.shape, dtype=torch.bfloat16, device=dy.device)
    dw = torch.empty(C, dtype=torch.float32, device=dy.device)
    db = torch.empty_like(dw)
    ws = _workspace(DY3, N, C, HW)
    rc = _lib.lib().dopt_bn_train_backward(m, p.data_ptr(), _ptr(rp), sc.data_ptr(), mn.data_ptr(), DY3.data_ptr(),
                                           _DTYPE_CODE[DY3.dtype], N, C, HW, C * HW, HW, g, bits, ws.data_ptr(),
                                           w.data_ptr(), v.data_ptr(), _LAYER_EPS[kind][1], dw.data_ptr(),
                                           db.data_ptr(), dx.data_ptr(), _stream(dy))
    _lib.check(rc, "bn_train_bwd")
    return dx, dw, db


def _bn_train_bwd_fake(packed, relu_packed, dy, scale, min, weight, var, BLOCK_M, bits, kind):
    N, C = dy.shape[0], dy.shape[1]
    HW = dy.numel() // (N * C) if N * C else 0
    return (dy.new_empty((N, C, HW), dtype=torch.bfloat16), dy.new_empty((C,), dtype=torch.float32),
            dy.new_empty((C,), dtype=torch.float32))


bn_train_bwd = _op(
    "bn_train_bwd(Tensor packed, Tensor? relu_packed, Tensor dy, Tensor scale, Tensor min, Tensor weight, Tensor var, "
    "int BLOCK_M, int bits, int kind) -> (Tensor, Tensor, Tensor)", _bn_train_bwd, _bn_train_bwd_fake)


__all__ = [
    "bn_train_fwd", "bn_train_bwd", "bn_fwd_reduce", "bn_fwd_norm", "bn_fwd_norm_quant_pack_fused", "bn_relu_fwd_norm_fused_quant_pack",
    "bn_bwd_reduce", "bn_bwd_dx", "bn_bwd_reduce_dequant_unpack_fused", "bn_bwd_dx_dequant_unpack_fused",
    "bn_relu_bwd_reduce_fused_dequant_unpack", "bn_relu_bwd_dx_fused_dequant_unpack",
]
