"""Controller: rewrites a model so that its large saved activations are compressed, and the
per-layer compression meta (group size, padding and group counts) that goes with it.

Mirrors Activation_Compression/controller.py. ``Controller.warp_model`` (:63-351) traces the model
with torch.fx, propagates shapes under FakeTensorMode with bf16 autocast, selects every Linear /
Conv1d/2d/3d / ReLU / SiLU / GELU call whose output exceeds 10 MiB, writes the layer's entry of the
shared ``meta`` dict and swaps in the compressed drop-in (DOLinear, DOConv*, DOReLU_Variance,
DOSiLU, DOGELU), copying the weights. The per-layer arithmetic comes out the same as the
reference's (controller.py:127-177 and :364-390):

  * ``find_group_size(S, bits, special)`` takes the first of [512, 256, 128, 64] (BatchNorm:
    [1024, 512, 256, 128, 64]) that divides the per-sample (per-channel for BatchNorm) element
    count S, else (256, act_padding=True) (controller.py:364-378). Bits outside {1, 2, 4, 8} also
    fall through to (256, True), as in the reference.
  * ``layer_group_meta(shape, bits, batchnorm)`` restates controller.py:127-177: the grouped
    extent is C*H*W per sample (C*L for 3-D, features for 2-D), or N*H*W per channel for
    BatchNorm, and G = ceil(S / group_size).
"""
from __future__ import annotations

from typing import Dict, Optional, Sequence, Tuple

import torch
from torch import nn

_GROUPS = (512, 256, 128, 64)
_GROUPS_BN = (1024, 512, 256, 128, 64)


def find_group_size(S: int, bits: int, max_group: int = 512, special: bool = False) -> Tuple[int, bool]:
    """-> (group_size, act_padding); reference controller.py:364-378 (max_group is unused there too)."""
    for gs in (_GROUPS_BN if special else _GROUPS):
        if bits in (1, 2, 4, 8) and S % gs == 0:
            return gs, False
    return 256, True


def layer_group_meta(shape: Sequence[int], bits: int, batchnorm: bool = False) -> Dict[str, object]:
    """Group layout of one layer's saved activation (reference controller.py:127-177).

    Returns {'group_size', 'act_padding', 'N', 'NG'}: N is the batch (the channel count for
    BatchNorm) and NG = N * ceil(S / group_size)."""
    shape = tuple(int(s) for s in shape)
    if len(shape) == 4:
        if batchnorm:
            S, N = shape[0] * shape[2] * shape[3], shape[1]
        else:
            S, N = shape[1] * shape[2] * shape[3], shape[0]
    elif len(shape) == 3:
        if batchnorm:
            S, N = shape[0] * shape[2], shape[1]
        else:
            S, N = shape[1] * shape[2], shape[0]
    elif len(shape) == 2:
        S, N = shape[1], shape[0]
    else:
        raise ValueError(f"layer_group_meta expects a 2-, 3- or 4-D activation shape, got {shape}")
    group_size, act_padding = find_group_size(S, bits, special=batchnorm)
    G = (S + group_size - 1) // group_size
    return {"group_size": group_size, "act_padding": act_padding, "N": N, "NG": N * G}


def compute_activation_size_in_bytes(shape: Sequence[int], dtype: torch.dtype) -> float:
    """Activation size in MiB, the unit of the reference's >10 MB selection rule (controller.py:381-390)."""
    numel = 1
    for s in shape:
        numel *= int(s)
    return numel * torch.tensor([], dtype=dtype).element_size() / (1024 ** 2)


def _node_input_meta(node):
    """tensor_meta of the first tensor argument of an fx node (controller.py:353-361)."""
    for arg in node.args:
        if isinstance(arg, torch.fx.Node) and arg.op != "get_attr":
            return arg.meta.get("tensor_meta")
        return None
    return None


_SELECTED = (nn.Linear, nn.Conv1d, nn.Conv2d, nn.Conv3d, nn.BatchNorm2d, nn.SyncBatchNorm, nn.ReLU, nn.SiLU, nn.GELU)
_BATCHNORM = (nn.BatchNorm2d, nn.SyncBatchNorm)


class Controller:
    """Rewrites ``model`` for compressed activation saving (controller.py:11-351).

    ``config`` keys read (as the reference's): ``batch_size``, ``default_bits``, ``group_size``,
    ``fp8``, ``analyze``, ``AVG_ALAM`` / ``AVG_ALAM_BTS``. The reference's Quantizer (which picks a
    bit width per layer from gradient statistics) and its DIVISION selection are research code
    outside this library: every selected layer gets ``default_bits`` unless ``config['bits']``
    (a {target: bits} dict) names it, and ``DIVISION`` is None (a caller may set a layer's
    ``meta[target]['DIVISION']`` by hand; the layer Functions honour it). ReLU layers are
    mask-only (``pack_only``, 1 bit) as in the reference. BatchNorm and SyncBatchNorm layers get
    the per-channel group layout (the reference applies it to BatchNorm2d only, controller.py:
    131-135, and gives SyncBatchNorm the per-sample one its kernels do not use) and keep their
    bias and running statistics (the reference copies the weight only, controller.py:330-332).

    ``input_shape`` (per sample) replaces the reference's peek at the first batch of
    ``train_loader``; either may be given. ``device`` is where the model runs ('cuda' as in the
    reference; the CPU works for tracing and meta only, the compressed layers need the GPU to
    train).
    """

    def __init__(self, model: nn.Module, config: dict, train_loader=None, criterion=None, test: bool = True,
                 input_shape: Optional[Sequence[int]] = None, device="cuda"):
        self.device = torch.device(device)
        self.model = model.to(self.device)
        self.config = config
        self.train_loader = train_loader
        self.criterion = criterion
        if input_shape is None:
            if train_loader is None:
                raise ValueError("Controller needs input_shape or a train_loader to read it from")
            x, _ = next(iter(train_loader))
            input_shape = x.shape[1:]
        self.input_shape = tuple(int(s) for s in input_shape)
        self.meta = {"group_size": config.get("group_size", 256), "fp8": config.get("fp8", False),
                     "analyze": config.get("analyze", False)}
        self.traced_model = None
        self.target_dict = {}
        if not test:
            self.warp_model()

    def _bits_for(self, target: str) -> int:
        return int(self.config.get("bits", {}).get(target, self.config["default_bits"]))

    def select_layers(self):
        """-> (traced GraphModule, {target: {'mod', 'tensor_meta'}}) of the layers to compress
        (controller.py:71-112): the fx trace, shape propagation under FakeTensorMode with bf16
        autocast, and the > 10 MiB output-size rule."""
        import torch.fx as fx
        from torch._subclasses.fake_tensor import FakeTensorMode
        from torch.fx.passes.shape_prop import ShapeProp

        traced = fx.symbolic_trace(self.model)
        named = dict(traced.named_modules())
        with FakeTensorMode(allow_non_fake_inputs=True):
            with torch.autocast(self.device.type, dtype=torch.bfloat16):
                fake = torch.empty(self.config["batch_size"], *self.input_shape, dtype=torch.bfloat16,
                                   device=self.device)
                ShapeProp(traced).propagate(fake)
        chosen = {}
        for node in traced.graph.nodes:
            if node.op != "call_module":
                continue
            mod = named[node.target]
            if not isinstance(mod, _SELECTED):
                continue
            tm = node.meta.get("tensor_meta")
            if tm is None or compute_activation_size_in_bytes(tm.shape, tm.dtype) <= 10:
                continue
            chosen[node.target] = {"mod": mod, "tensor_meta": _node_input_meta(node)}
        return traced, chosen

    def _new_module(self, target, mod):
        from .layers import DOConv1d, DOConv2d, DOConv3d, DOLinear
        from .modules.activations import DOGELU, DOReLU_Variance, DOSiLU
        from .modules.normalization import DOBatchNorm2d, DOSyncBatchNorm2d

        kw = dict(target_name=target, meta=self.meta)
        clamp = self.layer_clamp
        if isinstance(mod, nn.Linear):
            new = DOLinear(mod.in_features, mod.out_features, clamp_alpha=clamp, bias=mod.bias is not None, **kw)
        elif isinstance(mod, (nn.Conv1d, nn.Conv2d, nn.Conv3d)):
            cls = {nn.Conv1d: DOConv1d, nn.Conv2d: DOConv2d, nn.Conv3d: DOConv3d}[
                next(c for c in (nn.Conv1d, nn.Conv2d, nn.Conv3d) if isinstance(mod, c))]
            new = cls(mod.in_channels, mod.out_channels, mod.kernel_size, mod.stride, mod.padding, mod.dilation,
                      mod.groups, mod.padding_mode, clamp_alpha=clamp, bias=mod.bias is not None, **kw)
        elif isinstance(mod, _BATCHNORM):
            if isinstance(mod, nn.SyncBatchNorm):
                new = DOSyncBatchNorm2d(mod.num_features, mod.eps, mod.momentum, mod.affine, mod.track_running_stats,
                                        mod.process_group, **kw)
            else:
                new = DOBatchNorm2d(mod.num_features, mod.eps, mod.momentum, mod.affine, mod.track_running_stats, **kw)
            new.load_state_dict(mod.state_dict())
            return new.to(self.device)
        elif isinstance(mod, nn.ReLU):
            new = DOReLU_Variance(inplace=False, relu=True, relu6=False, **kw)
        elif isinstance(mod, nn.SiLU):
            new = DOSiLU(inplace=False, **kw)
        else:
            new = DOGELU(inplace=False, **kw)
        with torch.no_grad():
            for name in ("weight", "bias"):
                src = getattr(mod, name, None)
                if isinstance(src, torch.Tensor) and isinstance(getattr(new, name, None), torch.Tensor):
                    getattr(new, name).copy_(src)
        return new.to(self.device)

    def warp_model(self, graph_mode: bool = False, quantizer: bool = True):
        """controller.py:63-351. With ``quantizer=False`` the model is traced and nothing is
        swapped, as in the reference. ``graph_mode`` is accepted for the reference's signature; the
        reference uses it to hand the model to torch.compile, which this library replaces with
        HIP-graph capture of the whole train step (``deep_optimization_amd.graph``)."""
        del graph_mode
        self.layer_clamp = 3.0  # controller.py:61
        traced, chosen = self.select_layers()
        if quantizer:
            self.meta["batch_size"] = self.config["batch_size"]
            for target, d in chosen.items():
                mod, tm = d["mod"], d["tensor_meta"]
                bits = self._bits_for(target)
                relu = isinstance(mod, nn.ReLU)
                entry = {"tensor_meta": tm, "pack_only": relu, "bits": 1 if relu else bits}
                entry.update(layer_group_meta(tm.shape, bits, batchnorm=isinstance(mod, _BATCHNORM)))
                if self.config.get("AVG_ALAM") is not None:
                    entry.update({"AVG_ALAM": self.config["AVG_ALAM"], "ALAM_BITS": self.config["AVG_ALAM_BTS"]})
                else:
                    entry.update({"AVG_ALAM": False, "ALAM_BITS": 0})
                if isinstance(mod, (nn.Linear, nn.Conv1d, nn.Conv2d, nn.Conv3d)):
                    entry["AVG_ALAM"] = False
                entry["DIVISION"] = None
                self.meta[target] = entry
                parent, _, child = target.rpartition(".")
                setattr(traced.get_submodule(parent), child, self._new_module(target, mod))
            traced.graph.eliminate_dead_code()
            traced.graph.lint()
            traced.recompile()
        self.traced_model = traced.to(self.device).train()
        self.target_dict = chosen
        return self.traced_model


__all__ = ["Controller", "find_group_size", "layer_group_meta", "compute_activation_size_in_bytes"]
