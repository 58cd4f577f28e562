"""Compressed activation layers: ReLU / ReLU6, SiLU and GELU that save a packed mask or a quantized
derivative for the backward pass instead of their input.

Mirrors Activation_Compression/modules/activations/act_ops.py (autograd Functions ``_DOReLU``,
``_DOSiLU``, ``_DOGELU``, :16-164) and act_layers.py (modules ``DOReLU_Variance``, ``DOSiLU``,
``DOGELU``) with the same constructor and ``apply`` arguments and the same per-layer ``meta`` keys
(bits, group_size, act_padding, pack_only, AVG_ALAM, ALAM_BITS). In training the forward runs the
fused gfx950 kernels behind ``torch.ops.act_lib`` (relu_fwd_fused_pack, silu_fwd_quan_pack,
gelu_fwd_fused_quan_pack) and the backward their fused counterparts; layers whose activation
needs padding to a whole number of groups take the unfused operator + generic quantizer path, as
the reference does. In eval mode the modules are the plain torch activations.

Difference from the reference: its ``DOGELU`` subclasses ``nn.SiLU`` (act_layers.py), so in eval
mode it computes SiLU; here it subclasses ``nn.GELU(approximate='tanh')``, the function its
training path implements.
"""
from __future__ import annotations

import torch
from torch import nn
from torch.amp import custom_bwd, custom_fwd
from torch.autograd import Function

from .. import act_lib  # noqa: F401  (registers torch.ops.act_lib.*)
from .module_utils import unified_dequantize, unified_quantize


class _DOReLU(Function):
    """act_ops.py:16-58."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, input, relu, relu6, target_name, meta):
        m = meta[f"{target_name}"]
        ctx.act_padding = m["act_padding"]
        if ctx.act_padding:
            y, relu_mask = torch.ops.act_lib.relu_triton(input, relu, relu6)
            q_tensor, q_meta, _ = unified_quantize(relu_mask, None, target_name, meta, clamp=False, clamp_alpha=0.0)
            ctx.q_meta = q_meta
            ctx.save_for_backward(q_tensor[0])
            return y
        bits, group_size = m["bits"], m["group_size"]
        y, relu_mask, N, G = torch.ops.act_lib.relu_fwd_fused_pack(input, relu, relu6, bits, group_size)
        ctx.meta = N, G, bits, group_size
        ctx.save_for_backward(relu_mask)
        return y

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        if ctx.act_padding:
            (q,) = ctx.saved_tensors
            relu_mask = unified_dequantize((q, None, None), ctx.q_meta, None)
            return dy * relu_mask, None, None, None, None
        N, G, bits, group_size = ctx.meta
        (relu_mask,) = ctx.saved_tensors
        return torch.ops.act_lib.relu_bwd_fused_unpack(relu_mask, dy, bits, N, G, group_size), None, None, None, None


class _DOSiLU(Function):
    """act_ops.py:61-113."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, input, target_name, meta):
        m = meta[f"{target_name}"]
        ctx.act_padding = m["act_padding"]
        ctx.pack_only = m["pack_only"]
        if ctx.act_padding:
            y, act = torch.ops.act_lib.silu_triton(input)
            q_tensor, q_meta, _ = unified_quantize(act, None, target_name, meta, clamp=False, clamp_alpha=0.0)
            ctx.q_meta = q_meta
            ctx.save_for_backward(*q_tensor)
            return y
        bits, group_size = m["bits"], m["group_size"]
        avg_alam, alam_bits = m["AVG_ALAM"], m["ALAM_BITS"]
        (y, packed, scale, xmin, N, G, new_H, new_W, pad_elig,
         reshape_elig) = torch.ops.act_lib.silu_fwd_quan_pack(input, bits, group_size, avg_alam, alam_bits,
                                                             ctx.pack_only)
        ctx.meta = N, G, bits, group_size, avg_alam, alam_bits, new_H, new_W, pad_elig, reshape_elig
        ctx.save_for_backward(packed, scale, xmin)
        return y

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        if ctx.act_padding:
            act = unified_dequantize(tuple(ctx.saved_tensors), ctx.q_meta, None)
            return dy * act, None, None
        N, G, bits, group_size, avg_alam, alam_bits, new_H, new_W, pad_elig, reshape_elig = ctx.meta
        packed, scale, xmin = ctx.saved_tensors
        dx = torch.ops.act_lib.silu_bwd_fused_dequan_unpack(packed, dy, scale, xmin, bits, N, G, group_size,
                                                            ctx.pack_only, new_H, new_W, pad_elig, reshape_elig,
                                                            avg_alam, alam_bits)
        return dx, None, None


class _DOGELU(Function):
    """act_ops.py:116-164."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, input, target_name, meta):
        m = meta[f"{target_name}"]
        ctx.act_padding = m["act_padding"]
        if ctx.act_padding:
            y, act = torch.ops.act_lib.gelu_triton(input)
            q_tensor, q_meta, _ = unified_quantize(act, None, target_name, meta, clamp=False, clamp_alpha=0.0)
            ctx.q_meta = q_meta
            ctx.save_for_backward(*q_tensor)
            return y
        bits, group_size = m["bits"], m["group_size"]
        y, packed, scale, xmin, N, G = torch.ops.act_lib.gelu_fwd_fused_quan_pack(input, bits, group_size)
        ctx.meta = N, G, bits, group_size
        ctx.save_for_backward(packed, scale, xmin)
        return y

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        if ctx.act_padding:
            act = unified_dequantize(tuple(ctx.saved_tensors), ctx.q_meta, None)
            return dy * act, None, None
        N, G, bits, group_size = ctx.meta
        packed, scale, xmin = ctx.saved_tensors
        return torch.ops.act_lib.gelu_bwd_fused_dequan_unpack(packed, dy, scale, xmin, bits, N, G, group_size), None, None


class DOReLU_Variance(nn.ReLU):
    """act_layers.py: ReLU (relu=True) or ReLU6's band mask (relu6=True) with a packed-mask backward."""

    def __init__(self, inplace=False, relu=True, relu6=False, target_name=None, meta={}):
        super().__init__(inplace=inplace)
        self.target_name = target_name
        self.meta = meta
        self.relu = relu
        self.relu6 = relu6

    def forward(self, x):
        if self.training:
            return _DOReLU.apply(x, self.relu, self.relu6, self.target_name, self.meta)
        return super().forward(x)


class DOSiLU(nn.SiLU):
    def __init__(self, inplace=False, target_name=None, meta={}):
        super().__init__(inplace=inplace)
        self.target_name = target_name
        self.meta = meta

    def forward(self, x):
        if self.training:
            return _DOSiLU.apply(x, self.target_name, self.meta)
        return super().forward(x)


class DOGELU(nn.GELU):
    def __init__(self, inplace=False, target_name=None, meta={}):
        super().__init__(approximate="tanh")
        self.target_name = target_name
        self.meta = meta

    def forward(self, x):
        if self.training:
            return _DOGELU.apply(x, self.target_name, self.meta)
        return super().forward(x)


__all__ = ["_DOReLU", "_DOSiLU", "_DOGELU", "DOReLU_Variance", "DOSiLU", "DOGELU"]
