"""Compressed BatchNorm: the forward saves x_hat quantized per channel group (fused with the
normalization on the GPU) instead of the input; the backward restores it inside the reduction
and input-gradient kernels.

Mirrors Activation_Compression/modules/normalization/normalization_ops.py (``_DOBatchNorm``,
:8-157; ``_DOSyncBatchNorm``, :160-340) and normalization_layers.py (``DOBatchNorm2d``,
``DOSyncBatchNorm2d``): same ``apply`` arguments, the same per-layer ``meta`` keys (group_size =
BLOCK_M, bits, act_padding, AVG_ALAM, ALAM_BITS) and the same two paths:
  * act_padding False: the forward saves 2 tanh(clamp(x_hat)/2) codes (groups of group_size // 2
    per channel) and the backward restores them inside its reduction and input-gradient kernels;
    each pass is one operator call (act_lib::bn_train_fwd / bn_train_bwd: the kernels of the
    reference's bn_fwd_reduce + bn_fwd_norm_quant_pack_fused and bn_bwd_reduce_dequant_unpack_fused
    + bn_bwd_dx_dequant_unpack_fused, with the running statistics updated in the normalize kernel);
  * act_padding True: act_lib::bn_fwd_norm, then the generic quantizer on x_hat; the backward
    dequantizes and runs bn_bwd_reduce + bn_bwd_dx.
As in the reference, the running variance is updated with the biased batch variance, the
module's eps is not used by the kernels (they use 1e-5 / 1e-7), and the gradients of weight and
bias come back in fp32.

Differences from the reference: a module without running statistics (track_running_stats=False)
skips their update instead of failing; DOSyncBatchNorm2d runs the single-process path (one GPU)
and raises NotImplementedError when its process group spans several ranks (the reference's
single-rank fallback passes arguments _DOBatchNorm does not take, normalization_layers.py:84-88).
"""
from __future__ import annotations

import torch
from torch import nn
from torch.amp import custom_bwd, custom_fwd
from torch.autograd import Function

from .. import _lib, bn_lib  # noqa: F401  (bn_lib registers the BatchNorm act_lib operators)
from .module_utils import unified_dequantize, unified_quantize

_NW, _NS = 8, 5  # launch-tuning arguments of the reference's operators (ignored by the kernels)


def _stat(t, like):
    """A running-statistics buffer for act_lib::bn_train_fwd (an empty tensor when the module keeps none)."""
    return t if t is not None else like.new_empty((0,), dtype=torch.float32)


def _update_running(running_mean, running_var, mean, var, momentum):
    """running = running * (1 - momentum) + momentum * batch statistic (normalization_ops.py:56-57),
    both buffers in one multi-tensor kernel per step."""
    run = [t for t, b in ((running_mean, mean), (running_var, var)) if t is not None and b is not None]
    new = [b for t, b in ((running_mean, mean), (running_var, var)) if t is not None and b is not None]
    if run:
        torch._foreach_mul_(run, 1.0 - momentum)
        torch._foreach_add_(run, new, alpha=momentum)


class _DOBatchNorm(Function):
    """normalization_ops.py:8-157."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, input, weight, bias, running_mean, running_var, exponential_average_factor, eps, target_name,
                meta, ema_grad_meta):
        ctx.set_materialize_grads(False)
        m = meta[f"{target_name}"]
        BLOCK_M = m["group_size"]
        momentum = exponential_average_factor
        N, C, H, W = input.shape
        HW = H * W
        x3 = input.contiguous().view(N, C, HW)
        M = N * HW
        geo = dict(M=M, HW=HW, stride_n=C * HW, stride_c=HW)
        if m["act_padding"]:
            sum_, sumsq_ = torch.ops.act_lib.bn_fwd_reduce(x3, **geo, BLOCK_M=BLOCK_M, num_warps=_NW, num_stages=_NS)
            y3, x_hat, mean, var = torch.ops.act_lib.bn_fwd_norm(x3, sum_, sumsq_, weight, bias, None, None, **geo,
                                                                 BLOCK_M=BLOCK_M, sync=False, num_warps=_NW,
                                                                 num_stages=_NS)
            _update_running(running_mean, running_var, mean, var, momentum)
            q, q_meta, _ = unified_quantize(x_hat, None, target_name, meta, clamp=False, clamp_alpha=0.0)
            ctx.q_meta = q_meta
            ctx.save_for_backward(weight, q[0], q[1], q[2], var)
            ctx.meta = (BLOCK_M, meta, target_name, None, None, True)
            return y3.view(N, C, H, W)
        avg_alam, alam_bits = m["AVG_ALAM"], m["ALAM_BITS"]
        if avg_alam:
            # the reference's path (normalization_ops.py:72-98): statistics, then normalize +
            # quant-pack with one code per run of alam_bits elements, then the running statistics
            sum_, sumsq_ = torch.ops.act_lib.bn_fwd_reduce(x3, **geo, BLOCK_M=BLOCK_M, num_warps=_NW, num_stages=_NS)
            y, packed, scale, xmin, mean, var = torch.ops.act_lib.bn_fwd_norm_quant_pack_fused(
                x3, sum_, sumsq_, weight, bias, None, None, **geo, BLOCK_M=BLOCK_M, bits=m["bits"], sync=False,
                avg_alam=True, alam_bits=alam_bits, num_warps=_NW, num_stages=_NS)
            _update_running(running_mean, running_var, mean, var, momentum)
            ctx.save_for_backward(weight, packed, scale, xmin, var)
            ctx.meta = (BLOCK_M, meta, target_name, True, alam_bits, False)
            return y.view(N, C, H, W)
        # statistics, normalize + quant-pack and the running-statistics update in one operator
        # call (the reference's bn_fwd_reduce + bn_fwd_norm_quant_pack_fused + update)
        y, packed, _, scale, xmin, mean, var = torch.ops.act_lib.bn_train_fwd(
            x3, weight, bias, _stat(running_mean, x3), _stat(running_var, x3), momentum, BLOCK_M, m["bits"],
            _lib.BN_QUANT)
        ctx.save_for_backward(weight, packed, scale, xmin, var)
        ctx.meta = (BLOCK_M, meta, target_name, False, 0, False)
        return y.view(N, C, H, W)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        BLOCK_M, meta, target_name, avg_alam, alam_bits, padded = ctx.meta
        N, C, H, W = dy.shape
        HW = H * W
        M = N * HW
        dy3 = dy.contiguous().view(N, C, HW)
        geo = dict(M=M, HW=HW, stride_n=C * HW, stride_c=HW)
        if padded:
            weight, q0, q1, q2, var = ctx.saved_tensors
            x_hat = unified_dequantize((q0, q1, q2), ctx.q_meta, None).view(N, C, HW)
            dgamma, dbeta = torch.ops.act_lib.bn_bwd_reduce(x_hat, dy3, **geo, BLOCK_M=BLOCK_M, num_warps=_NW,
                                                            num_stages=_NS)
            dx = torch.ops.act_lib.bn_bwd_dx(x_hat, dy3, var, weight, dbeta, dgamma, **geo, BLOCK_M=BLOCK_M,
                                             sync=False, num_warps=_NW, num_stages=_NS)
        elif avg_alam:
            # normalization_ops.py:141-157: the reduce restores the codes with the reference's noise,
            # the input gradient without
            weight, packed, scale, xmin, var = ctx.saved_tensors
            bits = meta[f"{target_name}"]["bits"]
            dgamma, dbeta = torch.ops.act_lib.bn_bwd_reduce_dequant_unpack_fused(
                packed, dy3, scale, xmin, **geo, BLOCK_M=BLOCK_M, bits=bits, avg_alam=True, alam_bits=alam_bits)
            dx = torch.ops.act_lib.bn_bwd_dx_dequant_unpack_fused(
                packed, dy3, scale, xmin, dgamma, dbeta, weight, var, **geo, BLOCK_M=BLOCK_M, bits=bits, sync=False,
                avg_alam=True, alam_bits=alam_bits)
        else:
            weight, packed, scale, xmin, var = ctx.saved_tensors
            bits = meta[f"{target_name}"]["bits"]
            dx, dgamma, dbeta = torch.ops.act_lib.bn_train_bwd(packed, None, dy3, scale, xmin, weight, var, BLOCK_M,
                                                              bits, _lib.BN_QUANT)
        return dx.view(N, C, H, W), dgamma, dbeta, None, None, None, None, None, None, None


def _ema_factor(bn: nn.modules.batchnorm._BatchNorm) -> float:
    """exponential_average_factor as nn.BatchNorm computes it (normalization_layers.py:26-38)."""
    factor = 0.0 if bn.momentum is None else bn.momentum
    if bn.training and bn.track_running_stats and bn.num_batches_tracked is not None:
        bn.num_batches_tracked.add_(1)
        factor = 1.0 / float(bn.num_batches_tracked) if bn.momentum is None else bn.momentum
    return factor


class DOBatchNorm2d(nn.BatchNorm2d):
    """normalization_layers.py:8-42."""

    def __init__(self, num_features, eps=1e-05, momentum=0.1, affine=True, track_running_stats=True, group=0,
                 target_name=None, meta=None, device=None, dtype=None):
        super().__init__(num_features, eps, momentum, affine, track_running_stats, device=device, dtype=dtype)
        self.target_name = target_name
        self.meta = {} if meta is None else meta
        self.ema_grad_meta = None

    def _affine(self, x):
        if self.affine:
            return self.weight, self.bias
        ones = torch.ones(self.num_features, device=x.device, dtype=torch.float32)
        return ones, torch.zeros_like(ones)

    def forward(self, x):
        if not self.training:
            return super().forward(x)
        self._check_input_dim(x)
        factor = _ema_factor(self)
        w, b = self._affine(x)
        return _DOBatchNorm.apply(x, w, b, self.running_mean, self.running_var, factor, self.eps, self.target_name,
                                  self.meta, self.ema_grad_meta)


class DOSyncBatchNorm2d(nn.SyncBatchNorm):
    """normalization_layers.py:45-109, single process (see the module docstring)."""

    def __init__(self, num_features, eps=1e-5, momentum=0.1, affine=True, track_running_stats=True,
                 process_group=None, group=0, target_name=None, meta=None, device=None, dtype=None):
        super().__init__(num_features, eps, momentum, affine, track_running_stats, process_group, device=device,
                         dtype=dtype)
        self.target_name = target_name
        self.meta = {} if meta is None else meta
        self.ema_grad_meta = None

    def forward(self, x):
        if not self.training:
            return super().forward(x)
        if not x.is_cuda:
            raise ValueError("SyncBatchNorm expected input tensor to be on GPU")
        self._check_input_dim(x)
        if torch.distributed.is_available() and torch.distributed.is_initialized():
            pg = self.process_group or torch.distributed.group.WORLD
            if torch.distributed.get_world_size(pg) > 1:
                raise NotImplementedError(
                    "DOSyncBatchNorm2d across several ranks is not part of this single-GPU build: the statistics "
                    "exchange (all_gather of mean / invstd) would feed the sync=True path of the BatchNorm operators")
        factor = _ema_factor(self)
        return _DOBatchNorm.apply(x, self.weight, self.bias, self.running_mean, self.running_var, factor, self.eps,
                                  self.target_name, self.meta, self.ema_grad_meta)


__all__ = ["_DOBatchNorm", "DOBatchNorm2d", "DOSyncBatchNorm2d"]
