"""Drop-in compressed Linear / Conv modules: in training they save their input quantized through
the act_lib operators (modules/ops.py); in eval they are the plain torch layers.

Mirrors Activation_Compression/layers.py: ``DOLinear`` (:8-24), ``DOConv1d`` (:27-64),
``DOConv2d`` (:67-100) and ``DOConv3d`` (:103-140), with the reference's constructor arguments
(``clamp_alpha``, ``target_name``, ``meta``) and attributes (``ema_grad_meta``,
``learnable_scale``).

Differences from the reference:
  * the bias is applied and trained (``bias=`` argument; DOLinear defaults to True as nn.Linear
    does, the Conv layers to False as the reference builds them). The reference's DOLinear owns
    a bias that its training forward never uses (layers.py:21, ops.py:481);
  * DOConv1d / DOConv3d train through the same compressed Function path as DOConv2d. The
    reference's versions call ``GroupPACTClampFn`` with an attribute they never define
    (``self.pact_alpha``, layers.py:44, :49, :120, :125) and DOConv3d calls the Function class
    without ``.apply`` (:126), so their training forward raises in the reference. Their eval
    forward keeps the reference's input clamp to [-clamp_alpha, clamp_alpha] (:62, :138);
  * with a non-zeros ``padding_mode`` the input is padded once, as nn.Conv does; the reference
    pads it with F.pad and then again through the Function's ``padding`` (layers.py:86-90);
  * the PACT clamp the reference's DOConv1d / DOConv3d put in front of the Function (layers.py:69,
    :74, :152, :157, with the never-defined ``self.pact_alpha``) is opt-in on every Conv layer: a
    ``pact_alpha`` (float or one-element tensor) runs ``GroupPACTClampFn`` on the training input
    first (read as a float at construction); without autocast its bf16 output is cast back to the
    input's dtype (exactly: the values are bf16) so that the convolution's operands agree. The default, None, is the reference's
    behaviour on every path that runs there.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .modules.ops import GroupPACTClampFn, _DOConv1d, _DOConv2d, _DOConv3d, _DOLinear


class DOLinear(nn.Linear):
    def __init__(self, in_features, out_features, clamp_alpha=3.0, target_name=None, meta=None, bias=True,
                 device=None, dtype=None):
        super().__init__(in_features, out_features, bias=bias, device=device, dtype=dtype)
        self.clamp_alpha = clamp_alpha
        self.target_name = target_name
        self.meta = {} if meta is None else meta
        self.ema_grad_meta = None

    def forward(self, x):
        if self.training:
            return _DOLinear.apply(x, self.weight, self.clamp_alpha, self.target_name, self.meta, self.ema_grad_meta,
                                   self.bias)
        return super().forward(x)


class _DOConvMixin:
    _fn = None
    _eval_clamp = False

    def _init_do(self, clamp_alpha, target_name, meta, pact_alpha):
        self.clamp_alpha = clamp_alpha
        # a constant (GroupPACTClampFn gives alpha no gradient, as the reference's does): read once
        # here, so the training forward makes no host synchronisation and stays graph-capturable
        self.pact_alpha = None if pact_alpha is None else float(pact_alpha)
        self.target_name = target_name
        self.meta = {} if meta is None else meta
        self.ema_grad_meta = None
        self.learnable_scale = None

    def forward(self, x):
        if self.training:
            if self.pact_alpha is not None:
                y = GroupPACTClampFn.apply(x, self.pact_alpha, self.meta[f"{self.target_name}"]["group_size"],
                                           self.meta, self.target_name)
                x = y if torch.is_autocast_enabled("cuda") else y.to(x.dtype)
            if self.padding_mode != "zeros":
                x = F.pad(x, self._reversed_padding_repeated_twice, mode=self.padding_mode)
                padding = 0
            elif self.padding == "valid":
                padding = 0
            elif self.padding == "same":
                # the gradient helpers take integer padding only: pad explicitly, as nn.Conv does for 'same'
                x = F.pad(x, self._reversed_padding_repeated_twice)
                padding = 0
            else:
                padding = self.padding
            return self._fn.apply(x, self.weight, self.learnable_scale, self.stride, padding, self.dilation,
                                  self.groups, self.clamp_alpha, self.target_name, self.meta, self.ema_grad_meta,
                                  self.bias)
        if self._eval_clamp:
            x = torch.clamp(x, -self.clamp_alpha, self.clamp_alpha)
        return super().forward(x)


class DOConv1d(_DOConvMixin, nn.Conv1d):
    _fn = _DOConv1d
    _eval_clamp = True

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1, groups=1,
                 padding_mode="zeros", clamp_alpha=3.0, target_name=None, meta=None, bias=False, device=None,
                 dtype=None, pact_alpha=None):
        nn.Conv1d.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias=bias,
                           padding_mode=padding_mode, device=device, dtype=dtype)
        self._init_do(clamp_alpha, target_name, meta, pact_alpha)


class DOConv2d(_DOConvMixin, nn.Conv2d):
    _fn = _DOConv2d

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1, groups=1,
                 padding_mode="zeros", clamp_alpha=3.0, target_name=None, meta=None, bias=False, device=None,
                 dtype=None, pact_alpha=None):
        nn.Conv2d.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias=bias,
                           padding_mode=padding_mode, device=device, dtype=dtype)
        self._init_do(clamp_alpha, target_name, meta, pact_alpha)


class DOConv3d(_DOConvMixin, nn.Conv3d):
    _fn = _DOConv3d
    _eval_clamp = True

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, dilation=1, groups=1,
                 padding_mode="zeros", clamp_alpha=3.0, target_name=None, meta=None, bias=False, device=None,
                 dtype=None, pact_alpha=None):
        nn.Conv3d.__init__(self, in_channels, out_channels, kernel_size, stride, padding, dilation, groups, bias=bias,
                           padding_mode=padding_mode, device=device, dtype=dtype)
        self._init_do(clamp_alpha, target_name, meta, pact_alpha)


class RMSNorm(nn.Module):
    """RMS normalisation over the last axis with a learned gain (Activation_Compression/layers.py:
    206-216): ``x / sqrt(mean(x^2) + eps) * weight``. Not compressed; the reference's notebooks
    swap it in for LayerNorm before handing the model to the Controller."""

    def __init__(self, dims, eps=1e-8):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dims))

    def forward(self, x):
        rms = x.pow(2).mean(dim=-1, keepdim=True).add(self.eps).sqrt()
        return x / rms * self.weight


__all__ = ["DOLinear", "DOConv1d", "DOConv2d", "DOConv3d", "RMSNorm"]
