"""Compressed Linear / Conv autograd Functions: the forward saves the layer input quantized
(per-group min/max, b bits, packed) instead of the input itself; the backward dequantizes it and
computes the weight and input gradients.

Mirrors Activation_Compression/modules/ops.py: ``_DOConvnd.run_forward`` / ``run_backward``
(:200-387), ``_DOConv1d/2d/3d`` (:390-435) and ``_DOLinear`` (:438-540), with the same ``apply``
arguments and ``meta`` keys (bits, group_size, act_padding, pack_only, AVG_ALAM, ALAM_BITS,
DIVISION and the optional rounding keys of module_utils). As in the reference, the saved input is
quantized with ``clamp=True`` and the layer's ``clamp_alpha`` (the tanh squash of the quantizer
applies), an optional DIVISION low-pass (average pool) is stored beside it and added back when
the input is restored, and under autocast the computation runs in the autocast dtype. The input
is quantized whole, not minus its low-pass, so a DIVISION layer's restored input is
x_hat + upsample(avgpool(x)), about x plus its low-pass (ops.py:245-264, :457-474 with
module_utils.py:86-102); this is kept as the reference computes it, for parity.

The Linear weight gradient ``dy^T . x_hat`` (and the bias gradient) runs on the gfx950 kernel
behind ``act_lib::dw_gemm`` when dy is bf16 and both feature counts are multiples of 256; the
per-layer meta key ``dw_fused_unpack`` (default False) makes that kernel decode the packed codes
itself instead of reading the dequantized x_hat.

Differences from the reference:
  * ``_DOLinear`` takes the bias and applies it (the reference calls ``F.linear(input, W, None)``
    and never trains the bias, ops.py:481); its gradient is ``dy`` summed over the rows;
  * on the dw_gemm path the weight gradient comes back in the weight's dtype (fp32 master
    weights get an fp32 gradient; the reference's is bf16 under autocast);
  * the Conv Functions take an optional bias the same way (the reference's DOConv layers are
    built with ``bias=False``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch.amp import custom_bwd, custom_fwd
from torch.autograd import Function
from torch.nn.modules.utils import _pair, _single, _triple

from ..dw_lib import dw_gemm_supported
from .module_utils import unified_dequantize, unified_quantize


def _compute_dtype():
    return torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None


class _DOConvnd(Function):
    @staticmethod
    def run_forward(ctx, forward_op, input, weight, learnable_scale, stride=1, padding=0, dilation=1, groups=1,
                    clamp_alpha=3.0, target_name=None, meta=None, ema_grad_meta=None, bias=None):
        """ops.py:200-270."""
        dt = _compute_dtype()
        if dt is not None:
            input = input.to(dt)
            weight_compute = weight.to(dt)
            bias_compute = None if bias is None else bias.to(dt)
        else:
            weight_compute, bias_compute = weight, bias
        m = meta[f"{target_name}"]
        input_l = None
        if m.get("DIVISION") is not None and not m["pack_only"]:
            k = min(input.shape[-2], input.shape[-1], m["DIVISION"]["pool_kernel_size"])
            input_l = F.avg_pool2d(input.to(torch.bfloat16), k, stride=k, padding=0)
        q_tensor, q_meta, input_l = unified_quantize(input.to(torch.bfloat16), input_l, target_name, meta, clamp=True,
                                                     clamp_alpha=clamp_alpha)
        ctx.meta = stride, padding, dilation, groups, ema_grad_meta, clamp_alpha, bias is not None
        # the backward computes with the weight in bf16 under autocast: keep the forward's cast
        # (as autograd does for a plain convolution) instead of casting again
        w_saved = weight if dt is None else (weight_compute if dt == torch.bfloat16 else weight.to(torch.bfloat16))
        ctx.save_for_backward(w_saved, q_tensor[0], q_tensor[1], q_tensor[2], input_l, learnable_scale)
        ctx.q_inputs_meta = q_meta
        return forward_op(input, weight_compute, bias=bias_compute, stride=stride, padding=padding, dilation=dilation,
                          groups=groups)

    @staticmethod
    def run_backward(ctx, dy, dim, pad_fn):
        """ops.py:273-387: restores the input, then the input and weight gradients (the
        conv*_input / conv*_weight pair of the reference, computed by one convolution_backward
        call: the same two products, one dispatch)."""
        stride, padding, dilation, groups, _, _, has_bias = ctx.meta
        weight_compute, q0, q1, q2, input_l, _ = ctx.saved_tensors  # bf16 under autocast (see run_forward)
        dt = _compute_dtype()
        if dt is not None:
            dy = dy.to(dt)
        stride, padding, dilation = pad_fn(stride), pad_fn(padding), pad_fn(dilation)
        input = unified_dequantize((q0, q1, q2), ctx.q_inputs_meta, input_l)
        dx = dw = db = None
        need_dx, need_dw = bool(ctx.needs_input_grad[0]), bool(ctx.needs_input_grad[1])
        if need_dx or need_dw:
            dx, dw, _ = torch.ops.aten.convolution_backward(
                dy, input.to(dy.dtype), weight_compute.to(dy.dtype), None, list(stride), list(padding),
                list(dilation), False, [0] * dim, groups, [need_dx, need_dw, False])
        if has_bias:
            db = dy.sum(dim=[0] + list(range(2, dy.dim())))
        if dx is not None and dt is not None:
            dx = dx.to(torch.bfloat16)
        if dw is not None and dt is not None:
            dw = dw.to(torch.bfloat16)
        return dx, dw, None, None, None, None, None, None, None, None, None, db


def _conv_function(dim, op, pad_fn, name):
    class _Fn(Function):
        @staticmethod
        @custom_fwd(device_type="cuda")
        def forward(ctx, input, weight, learnable_scale, stride=1, padding=0, dilation=1, groups=1, clamp_alpha=3.0,
                    target_name=None, meta=None, ema_grad_meta=None, bias=None):
            return _DOConvnd.run_forward(ctx, op, input, weight, learnable_scale, stride=stride, padding=padding,
                                         dilation=dilation, groups=groups, clamp_alpha=clamp_alpha,
                                         target_name=target_name, meta=meta, ema_grad_meta=ema_grad_meta, bias=bias)

        @staticmethod
        @custom_bwd(device_type="cuda")
        def backward(ctx, dy):
            return _DOConvnd.run_backward(ctx, dy, dim, pad_fn)

    _Fn.__name__ = _Fn.__qualname__ = name
    return _Fn


_DOConv1d = _conv_function(1, F.conv1d, _single, "_DOConv1d")  # ops.py:390-403
_DOConv2d = _conv_function(2, F.conv2d, _pair, "_DOConv2d")  # ops.py:406-419
_DOConv3d = _conv_function(3, F.conv3d, _triple, "_DOConv3d")  # ops.py:422-435


class _DOLinear(Function):
    """ops.py:438-540 (plus the bias, see the module docstring)."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, input, weight, clamp_alpha, target_name, meta, ema_grad_meta, bias=None):
        dt = _compute_dtype()
        if dt is not None:
            input = input.to(dt)
            weight_compute = weight.to(dt)
            bias_compute = None if bias is None else bias.to(dt)
        else:
            weight_compute, bias_compute = weight, bias
        m = meta[f"{target_name}"]
        input_l = None
        if m.get("DIVISION") is not None and input.ndim not in (1, 2) and not m["pack_only"]:
            k = min(input.shape[2], m["DIVISION"]["pool_kernel_size"])
            input_l = F.avg_pool1d(input.to(torch.bfloat16), k, stride=k, padding=0)
        q_tensor, q_meta, input_l = unified_quantize(input, input_l, target_name, meta, clamp=True,
                                                     clamp_alpha=clamp_alpha)
        ctx.q_inputs_meta = q_meta
        ctx.meta = input.shape, ema_grad_meta, clamp_alpha, bias is not None
        # the packed codes can feed the weight-gradient GEMM directly when they are the flat
        # [tokens * in_features] bitstream (no padding, no low-pass, no ALAM)
        (bits, pack_only, group_size, act_padding, _, _, _, _, _, reshape_elig, _, avg_alam, _, _) = q_meta
        ctx.fused_unpack = (bool(m.get("dw_fused_unpack", False)) and not (pack_only or act_padding or reshape_elig
                                                                             or avg_alam) and input_l is None)
        # the backward's input gradient uses the weight in the autocast dtype: keep the forward's cast
        ctx.w_dtype = weight.dtype
        ctx.save_for_backward(weight_compute, q_tensor[0], q_tensor[1], q_tensor[2], input_l)
        return F.linear(input, weight_compute, bias_compute)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        input_shape, _, _, has_bias = ctx.meta
        weight_compute, q0, q1, q2, input_l = ctx.saved_tensors  # the forward's (autocast-dtype) weight
        dt = _compute_dtype()
        if dt is not None:
            weight_compute = weight_compute.to(dt)
            dy = dy.to(dt)
        C_in, C_out = input_shape[-1], dy.shape[-1]
        dy_flat = dy.reshape(-1, C_out)
        if dy.dtype == torch.bfloat16 and dw_gemm_supported(C_out, C_in):
            # weight (and bias) gradient on the gfx950 split-K GEMM for K-outer operands, in the
            # weight's precision; x_hat is either dequantized first or decoded inside the GEMM
            out_dtype = ctx.w_dtype if ctx.w_dtype in (torch.float32, torch.bfloat16) else torch.float32
            if ctx.fused_unpack and q1.dtype == torch.bfloat16:
                bits, group_size = ctx.q_inputs_meta[0], ctx.q_inputs_meta[2]
                dw, db = torch.ops.act_lib.dw_gemm(dy_flat, None, q0, q1, q2, C_in, bits, group_size, has_bias,
                                                   out_dtype)
                input = None
            else:
                input = unified_dequantize((q0, q1, q2), ctx.q_inputs_meta, input_l)
                dw, db = torch.ops.act_lib.dw_gemm(dy_flat, input.reshape(-1, C_in), None, None, None, C_in, 0, 0,
                                                   has_bias, out_dtype)
        else:
            input = unified_dequantize((q0, q1, q2), ctx.q_inputs_meta, input_l).to(dy.dtype)
            dw = dy_flat.t().mm(input.reshape(-1, C_in))
            db = dy_flat.sum(0) if has_bias else None
        dx = dy_flat.mm(weight_compute.to(dy.dtype))
        return dx.view(*input_shape), dw, None, None, None, None, db


class GroupPACTClampFn(Function):
    """The reference's PACT clamp Function (AC/modules/ops.py:625-668): forward returns
    bf16 clamp(x, -alpha, alpha) (act_lib::group_pact_clamp_fwd, in the autocast dtype under
    autocast) and saves the mask |x| <= alpha bit-packed (1-bit pack-only quantize under
    meta["<target_name>_clamp"], with the target's act_padding and N); the backward restores the
    mask and returns dy * mask. ``alpha`` may be a float or a one-element tensor."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x, alpha, group_size, meta, target_name):
        if torch.is_autocast_enabled("cuda"):
            x = x.to(torch.get_autocast_dtype("cuda"))
        a = float(alpha.item() if isinstance(alpha, torch.Tensor) else alpha)
        y, mask = torch.ops.act_lib.group_pact_clamp_fwd(x, a)
        clamp_name = f"{target_name}_clamp"
        clamp_meta = {clamp_name: {"bits": 1, "pack_only": True, "group_size": group_size,
                                   "act_padding": meta[f"{target_name}"]["act_padding"],
                                   "N": meta[f"{target_name}"]["N"], "AVG_ALAM": False, "ALAM_BITS": 0}}
        q_tensor, q_meta, _ = unified_quantize(mask, None, clamp_name, clamp_meta, clamp=False, clamp_alpha=a)
        ctx.save_for_backward(q_tensor[0])
        ctx.q_meta = q_meta
        return y

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        (packed,) = ctx.saved_tensors
        mask = unified_dequantize((packed, None, None), ctx.q_meta, None)
        return dy * mask, None, None, None, None


__all__ = ["_DOConvnd", "_DOConv1d", "_DOConv2d", "_DOConv3d", "_DOLinear", "GroupPACTClampFn"]
