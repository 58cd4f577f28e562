"""Weight-gradient operator of the compressed Linear layer: dW = dy^T . x_hat (+ db = sum of dy
over tokens) on the gfx950 kernel behind dopt_dw_gemm, with x_hat decoded inside the GEMM from
the quantizer's packed codes (or read as a bf16 tensor).

Registered as ``torch.ops.act_lib.dw_gemm`` (no counterpart operator in the reference: it
replaces the dequantize + ``dy_flatten.T.mm(input_flatten)`` pair of
Activation_Compression/modules/ops.py:508-512, whose Triton fusion the reference tried only in
test2.ipynb).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _lib
from .act_lib import _bits_consts, _op, _require_cuda, _stream


def _aligned16(t: Tensor) -> Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def dw_gemm_supported(M: int, N: int) -> bool:
    """Shapes the kernel takes: out and in features multiples of 256."""
    return M > 0 and N > 0 and M % 256 == 0 and N % 256 == 0


def _dw_gemm(dy: Tensor, x_hat: Optional[Tensor], packed: Optional[Tensor], scale: Optional[Tensor],
             min: Optional[Tensor], N: int, bits: int, group_size: int, bias_grad: bool, out_dtype: torch.dtype):
    """dy bf16 [K, M]; x_hat bf16 [K, N] or (packed, scale, min) codes of the flat [K*N] activation
    -> (dW [M, N] in out_dtype (float32 or bfloat16), db fp32 [M] or None)."""
    _require_cuda(dy)
    if dy.dim() != 2 or dy.dtype != torch.bfloat16:
        raise RuntimeError(f"dw_gemm: dy must be a bf16 [K, M] matrix, got {tuple(dy.shape)} {dy.dtype}")
    if out_dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"dw_gemm: out_dtype must be float32 or bfloat16, got {out_dtype}")
    K, M = int(dy.shape[0]), int(dy.shape[1])
    dy = _aligned16(dy)
    L = _lib.lib()
    ws = torch.empty(max(int(L.dopt_dw_gemm_workspace_floats(M, N, K)), 4), dtype=torch.float32, device=dy.device)
    dw = torch.empty((M, N), dtype=out_dtype, device=dy.device)
    db = torch.empty(M, dtype=torch.float32, device=dy.device) if bias_grad else None
    d32 = dw.data_ptr() if out_dtype == torch.float32 else None
    d16 = dw.data_ptr() if out_dtype == torch.bfloat16 else None
    if x_hat is not None:
        if x_hat.dtype != torch.bfloat16 or x_hat.numel() != K * N:
            raise RuntimeError(f"dw_gemm: x_hat must be bf16 with K*N = {K * N} elements")
        xh = _aligned16(x_hat.reshape(K, N))
        rc = L.dopt_dw_gemm(dy.data_ptr(), M, xh.data_ptr(), N, None, None, None, 0, 0, M, N, K, ws.data_ptr(), d32,
                            d16, None if db is None else db.data_ptr(), _stream(dy))
    else:
        _bits_consts(bits, group_size)
        if packed is None or scale is None or min is None:
            raise RuntimeError("dw_gemm: give x_hat or packed, scale and min")
        if packed.numel() * 32 != K * N * bits:
            raise RuntimeError(f"dw_gemm: packed holds {packed.numel()} words, expected {K * N * bits // 32}")
        if (K * N) % group_size:
            raise RuntimeError(f"dw_gemm: K*N = {K * N} is not a whole number of groups of {group_size}")
        p = _aligned16(packed)
        sc, mn = scale.contiguous(), min.contiguous()
        if sc.dtype != torch.bfloat16 or mn.dtype != torch.bfloat16:
            raise RuntimeError("dw_gemm: scale and min must be bf16 (the reference quantizer's)")
        n_groups = K * N // group_size
        if sc.numel() != n_groups or mn.numel() != n_groups:
            raise RuntimeError(f"dw_gemm: scale and min must hold one value per group ({n_groups}), got "
                               f"{sc.numel()} and {mn.numel()}")
        rc = L.dopt_dw_gemm(dy.data_ptr(), M, None, 0, p.data_ptr(), sc.data_ptr(), mn.data_ptr(), group_size, bits,
                            M, N, K, ws.data_ptr(), d32, d16, None if db is None else db.data_ptr(), _stream(dy))
    _lib.check(rc, "dw_gemm")
    return dw, db


def _dw_gemm_fake(dy, x_hat, packed, scale, min, N, bits, group_size, bias_grad, out_dtype):
    M = dy.shape[1]
    return dy.new_empty((M, N), dtype=out_dtype), (dy.new_empty((M,), dtype=torch.float32) if bias_grad else None)


dw_gemm = _op(
    "dw_gemm(Tensor dy, Tensor? x_hat, Tensor? packed, Tensor? scale, Tensor? min, int N, int bits, int group_size, "
    "bool bias_grad, ScalarType out_dtype) -> (Tensor, Tensor?)", _dw_gemm, _dw_gemm_fake)

__all__ = ["dw_gemm", "dw_gemm_supported"]
