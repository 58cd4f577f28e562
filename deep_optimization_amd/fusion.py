"""BatchNorm + ReLU fusion: one kernel normalizes, applies the ReLU, stores a 1-bit mask and the
quantized x_hat; the backward reduces and forms dx from them.

Mirrors Activation_Compression/fusion/fused_ops.py (``_DOBatchNormReLU2d``, :9-86),
fused_layers.py (``DOBatchNormReLU2d``, :8-42) and fusion_utils.py (``fuse_bn_act``, :57-110,
which rewrites DOBatchNorm2d -> DOReLU_Variance pairs of an fx GraphModule into one
DOBatchNormReLU2d named ``rename_fmt.format(bn_name)``, moving the BatchNorm's meta entry to the
new name).

Differences from the reference: the fused-away ReLU modules are deleted from the GraphModule; the
module counts ``num_batches_tracked`` as nn.BatchNorm does
(the reference's test is inverted, fused_layers.py:27-30, so it never counts); a module without
affine parameters uses weight 1 and bias 0; relu6 clamps to [0, 6] (bn_lib).
"""
from __future__ import annotations

from typing import Any, Dict, Iterable, Tuple, Type

import torch
import torch.fx as fx
import torch.nn.functional as F
from torch import nn
from torch.amp import custom_bwd, custom_fwd
from torch.autograd import Function

from . import _lib, bn_lib  # noqa: F401  (bn_lib registers the BatchNorm act_lib operators)
from .modules.activations import DOReLU_Variance
from .modules.normalization import DOBatchNorm2d, _ema_factor, _stat


class _DOBatchNormReLU2d(Function):
    """fused_ops.py:9-86."""

    @staticmethod
    @custom_fwd(device_type="cuda")
    def forward(ctx, x, weight, bias, relu, relu6, running_mean, running_var, exponential_average_factor,
                target_name, meta, ema_grad_meta):
        ctx.set_materialize_grads(False)
        m = meta[f"{target_name}"]
        BLOCK, BITS = m["group_size"], m["bits"]
        N, C, H, W = x.shape
        HW = H * W
        x3 = x.contiguous().view(N, C, HW)
        if not (relu or relu6):
            raise RuntimeError("DOBatchNormReLU2d needs relu or relu6")
        mode = _lib.BN_RELU_QUANT if relu else _lib.BN_RELU6_QUANT
        # statistics, normalize + ReLU + quant-pack and the running-statistics update in one
        # operator call (the reference's bn_fwd_reduce + bn_relu_fwd_norm_fused_quant_pack + update)
        y, packed, relu_packed, scale, xmin, mean, var = torch.ops.act_lib.bn_train_fwd(
            x3, weight, bias, _stat(running_mean, x3), _stat(running_var, x3), exponential_average_factor, BLOCK,
            BITS, mode)
        ctx.other_meta = BLOCK, BITS, mode
        ctx.save_for_backward(weight, packed, relu_packed, var, scale, xmin)
        return y.view(N, C, H, W)

    @staticmethod
    @custom_bwd(device_type="cuda")
    def backward(ctx, dy):
        BLOCK, BITS, mode = ctx.other_meta
        weight, packed, relu_packed, var, scale, xmin = ctx.saved_tensors
        N, C, H, W = dy.shape
        dy3 = dy.contiguous().view(N, C, H * W)
        DX, DW, DB = torch.ops.act_lib.bn_train_bwd(packed, relu_packed, dy3, scale, xmin, weight, var, BLOCK, BITS,
                                                    mode)
        return DX.view(N, C, H, W), DW, DB, None, None, None, None, None, None, None, None


class DOBatchNormReLU2d(nn.BatchNorm2d):
    """fused_layers.py:8-42: BatchNorm followed by ReLU (or ReLU6) in one compressed layer."""

    def __init__(self, num_features, eps=1e-5, momentum=0.1, relu=True, relu6=False, affine=True,
                 track_running_stats=True, group=0, target_name=None, meta=None, device=None, dtype=None):
        super().__init__(num_features, eps, momentum, affine, track_running_stats, device=device, dtype=dtype)
        self.target_name = target_name
        self.meta = {} if meta is None else meta
        self.relu = relu
        self.relu6 = relu6
        self.ema_grad_meta = None

    def forward(self, x):
        if not self.training:
            y = super().forward(x)
            return F.relu6(y) if (self.relu6 and not self.relu) else F.relu(y)
        self._check_input_dim(x)
        factor = _ema_factor(self)
        if self.affine:
            w, b = self.weight, self.bias
        else:
            w = torch.ones(self.num_features, device=x.device)
            b = torch.zeros_like(w)
        return _DOBatchNormReLU2d.apply(x, w, b, self.relu, self.relu6, self.running_mean, self.running_var, factor,
                                        self.target_name, self.meta, self.ema_grad_meta)


def _matches(pattern: Iterable[Type], node: fx.Node, modules: Dict[str, Any]) -> bool:
    """fusion_utils.py:15-35: node is pattern[1] applied to the output of a pattern[0] module."""
    if len(node.args) == 0:
        return False
    for expected, cur in zip(pattern, (node.args[0], node)):
        if not isinstance(cur, fx.Node) or cur.op != "call_module" or not isinstance(cur.target, str):
            return False
        if cur.target not in modules or type(modules[cur.target]) is not expected:
            return False
    return True


def _replace(node: fx.Node, modules: Dict[str, Any], new_module: nn.Module, new_child: str) -> None:
    """fusion_utils.py:38-54."""
    parent_name, _, old_child = node.target.rpartition(".")
    new_qual = f"{parent_name}.{new_child}" if parent_name else new_child
    parent = modules[parent_name]
    setattr(parent, new_child, new_module)
    if hasattr(parent, old_child) and old_child != new_child:
        delattr(parent, old_child)
    modules[new_qual] = new_module
    modules.pop(node.target, None)
    node.target = new_qual


def fuse_bn_act(model: fx.GraphModule, rename_fmt: str = "{}_bnact") -> fx.GraphModule:
    """Fuses every DOBatchNorm2d -> DOReLU_Variance pair whose BatchNorm output has no other user
    (fusion_utils.py:57-110)."""
    patterns: Tuple[Tuple[Type, Type], ...] = ((DOBatchNorm2d, DOReLU_Variance),)
    modules = dict(model.named_modules())
    graph = model.graph
    for pattern in patterns:
        for node in list(graph.nodes):
            if not _matches(pattern, node, modules) or len(node.args[0].users) > 1:
                continue
            bn, act = modules[node.args[0].target], modules[node.target]
            old_qual = node.args[0].target
            new_child = rename_fmt.format(old_qual.rpartition(".")[2])
            target_name = rename_fmt.format(old_qual)
            bn.meta[target_name] = bn.meta[f"{bn.target_name}"]
            bn.meta.pop(old_qual, None)
            fused = DOBatchNormReLU2d(bn.num_features, bn.eps, bn.momentum, relu=act.relu, relu6=act.relu6,
                                      affine=bn.affine, track_running_stats=bn.track_running_stats,
                                      target_name=target_name, meta=bn.meta)
            fused.load_state_dict(bn.state_dict())
            fused.to(next(iter(bn.buffers()), torch.empty(0)).device)
            _replace(node.args[0], modules, fused, new_child)
            node.replace_all_uses_with(node.args[0])
            graph.erase_node(node)
    graph.lint()
    model.recompile()
    model.delete_all_unused_submodules()
    return model


__all__ = ["_DOBatchNormReLU2d", "DOBatchNormReLU2d", "fuse_bn_act"]
