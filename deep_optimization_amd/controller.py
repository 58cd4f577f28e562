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


class _Tracer:
    """torch.fx tracer that keeps this library's compressed layers as leaves, so a model that
    already holds them traces (their forward is an autograd Function, not traceable ops)."""

    @staticmethod
    def make():
        import torch.fx as fx
        from .fusion import DOBatchNormReLU2d
        from .layers import DOConv1d, DOConv2d, DOConv3d, DOLinear
        from .modules.activations import DOGELU, DOReLU_Variance, DOSiLU
        from .modules.normalization import DOBatchNorm2d, DOSyncBatchNorm2d

        compressed = (DOLinear, DOConv1d, DOConv2d, DOConv3d, DOGELU, DOReLU_Variance, DOSiLU, DOBatchNorm2d,
                      DOSyncBatchNorm2d, DOBatchNormReLU2d)

        class Tracer(fx.Tracer):
            def is_leaf_module(self, m, qualname):
                return isinstance(m, compressed) or super().is_leaf_module(m, qualname)

        return Tracer(), compressed


class Controller:
    """Rewrites ``model`` for compressed activation saving (controller.py:11-351), with the
    reference's call API:

        c = Controller(model, config, train_loader, criterion, test=False)
        c.iterate(criterion)
        c.warp_model(graph_mode=True, quantizer=True)
        model = c.traced_model

    (Train/Trainer.py:179-183; test8.ipynb cell 2.) With ``test=False`` the constructor runs the
    DIVISION layer analysis (``select_division_layer``: one forward and backward on 64 training
    samples), traces the model without swapping anything, and seeds ``quantizer.bits`` with the
    selected targets (controller.py:31-38). ``iterate`` gives every target its bit width
    (``Quantizer.iterate``: ``default_bits`` when ``auto_precision`` is None).
    ``warp_model(quantizer=True)`` writes each selected layer's ``meta`` entry and swaps in the
    compressed drop-in (DOLinear, DOConv*, DOBatchNorm2d, DOSyncBatchNorm2d, DOReLU_Variance,
    DOSiLU, DOGELU), copying the weights; ``quantizer=False`` (the default, as in the reference)
    traces and selects only. ``enable_graph_mode(stream)`` and ``warmup(loader, criterion,
    stream)`` replace the reference's ``torch.compile(mode='reduce-overhead')`` of the rewritten
    model with HIP-graph replay of its forward and backward (``graph.graph_module_in_place``).

    ``config`` keys read, as the reference's: ``batch_size``, ``default_bits``, ``group_size``,
    ``fp8``, ``analyze``, ``auto_precision``, ``DIVISION``, ``AVG_ALAM`` / ``AVG_ALAM_BTS``,
    ``depth_point_conv``, ``rms_norm``; and ``bits``, a {target: bits} dict of per-layer widths
    that take precedence over the quantizer's (this library's addition).

    Differences from the reference:
      * a layer's ``meta[target]['bits']`` is the width its group size was chosen for (the
        quantizer's); the reference writes ``default_bits`` there and picks the group size from
        the quantizer's width, which agree whenever ``auto_precision`` is None (controller.py:118,
        :127-177);
      * ``config['depth_point_conv']`` true raises ``NotImplementedError``: the reference's
        ``DODepthPointConv2d`` passes an argument its convolutions do not take (layers.py:
        173-188), so that configuration cannot construct there either;
      * ``config['rms_norm']`` true raises ``NotImplementedError``: the reference swaps a
        LayerNorm for RMSNorm only inside the loop over selected layers, which never holds a
        LayerNorm (controller.py:99-100 against :283-288), so the option changes nothing there.
        Replace the LayerNorms in the model before the Controller (``layers.RMSNorm``) instead;
      * BatchNorm and SyncBatchNorm layers get the per-channel group layout (the reference
        applies it to BatchNorm2d only, controller.py:131-135, and gives SyncBatchNorm the
        per-sample one its kernels do not use) and keep their bias and running statistics (the
        reference copies the weight only, controller.py:291);
      * compressed layers already in the model are traced as leaves and left as they are, and the
        swap is made in ``self.model`` as well as in ``traced_model`` (the reference's swap reaches
        ``self.model`` only below its root, through the submodules the trace shares), so
        ``warp_model(quantizer=True)`` twice swaps each layer once;
      * ``input_shape`` (per sample) may replace the reference's peek at the first batch of
        ``train_loader``; ``device`` is where the model runs ('cuda' as in the reference; the
        CPU serves for tracing and meta, the compressed layers need the GPU to train).
    """

    def __init__(self, model: nn.Module, config: dict, train_loader=None, criterion=None, test: bool = True,
                 input_shape: Optional[Sequence[int]] = None, device="cuda"):
        from .quantizer import Quantizer

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
        self.quantizer = Quantizer(config, {})
        self.quantizer.filter_tensors(self.model.named_parameters())
        self.meta = {"group_size": config.get("group_size", 256), "fp8": config.get("fp8", False),
                     "analyze": config.get("analyze", False)}
        self.traced_model = None
        self.target_dict = {}
        self.layer_clamp = 3.0
        self.low_frequency_energy_ratio_grad = None
        if not test:
            self.select_division_layer()
            self.warp_model()
            self.quantizer.bits = self.target_dict.copy()

    def iterate(self, criterion=None, trainloader=None):
        """controller.py:41-45."""
        if trainloader is not None:
            self.quantizer.iterate(self.model, criterion, trainloader)
        else:
            self.quantizer.iterate(self.model, self.criterion, self.train_loader)

    def select_division_layer(self):
        """controller.py:47-61: per-layer statistics from ``Quantizer.select_division_layer_helper``
        and their thresholds, the 75th percentile of the activation and gradient LFERs (gradient
        LFERs of exactly 1 left out) and the medians of the signal-to-noise and LARS ratios. A
        layer is given ``config['DIVISION']`` when its gradient LFER exceeds the gradient
        threshold (``warp_model``)."""
        if self.criterion is None or self.train_loader is None:
            raise ValueError("the DIVISION layer analysis (Controller(test=False)) needs train_loader and criterion")
        (self.low_frequency_energy_ratio_grad, self.low_frequency_energy_ratio_act, self.lars_trust_ratio,
         self.signal_noise_ratio, self.activation_var) = self.quantizer.select_division_layer_helper(
            self.model, self.criterion, self.train_loader, device=self.device)

        def quantile(values, q):
            t = torch.tensor(list(values), dtype=torch.float32)
            return torch.quantile(t, q).item() if t.numel() else float("inf")

        self.base_division_threshold_act = quantile(self.low_frequency_energy_ratio_act.values(), 0.75)
        self.base_division_threshold_grad = quantile(
            (d for d in self.low_frequency_energy_ratio_grad.values() if d != 1), 0.75)
        self.base_threshold_signal_noise_ratio = quantile(self.signal_noise_ratio.values(), 0.50)
        self.base_threshold_lars_trust_ratio = quantile(self.lars_trust_ratio.values(), 0.5)
        self.layer_clamp = 3.0

    def _bits_for(self, target: str) -> int:
        override = self.config.get("bits", {}).get(target)
        if override is not None:
            bits = override
        else:
            bits = self.quantizer.bits.get(target, self.config["default_bits"])
            if not isinstance(bits, int):  # an entry the constructor seeded that iterate() has not set
                bits = self.config["default_bits"]
        self.quantizer.bits[target] = int(bits)
        return int(bits)

    def _division_for(self, target: str):
        division = self.config.get("DIVISION")
        if division is None:
            return None
        if self.low_frequency_energy_ratio_grad is None:
            self.select_division_layer()
        lfer = self.low_frequency_energy_ratio_grad.get(target)
        if lfer is not None and lfer > self.base_division_threshold_grad and lfer != 1:
            return division
        return None

    def select_layers(self):
        """-> (traced GraphModule, {target: {'mod', 'tensor_meta'}}) of the layers to compress
        (controller.py:71-112): the fx trace, shape propagation under FakeTensorMode with bf16
        autocast, and the > 10 MiB output-size rule."""
        import torch.fx as fx
        from torch._subclasses.fake_tensor import FakeTensorMode
        from torch.fx.passes.shape_prop import ShapeProp

        tracer, compressed = _Tracer.make()
        graph = tracer.trace(self.model)
        name = self.model.__class__.__name__
        traced = fx.GraphModule(tracer.root, graph, name)
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
            if not isinstance(mod, _SELECTED) or isinstance(mod, compressed):
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

    def _check_config(self):
        if self.config.get("depth_point_conv"):
            raise NotImplementedError(
                "config['depth_point_conv']: the reference's DODepthPointConv2d passes acc_var= to DOConv2d, which "
                "takes no such argument (Activation_Compression/layers.py:173-188), so no depthwise-pointwise "
                "swap exists to reproduce; set it False")
        if self.config.get("rms_norm"):
            raise NotImplementedError(
                "config['rms_norm']: the reference's LayerNorm -> RMSNorm swap sits inside the loop over selected "
                "layers, which never holds a LayerNorm (Activation_Compression/controller.py:99-100, :283-288), so "
                "the option changes nothing there; replace the model's LayerNorms with "
                "deep_optimization_amd.layers.RMSNorm before the Controller and set it False")

    def warp_model(self, graph_mode: bool = False, quantizer: bool = False):
        """controller.py:63-315. Traces and selects; with ``quantizer=True`` also gives each selected
        layer its bits (``iterate``), its ``meta`` entry (group layout, pack-only for ReLU,
        AVG_ALAM off for Linear/Conv, DIVISION from the layer analysis) and its compressed module.
        ``graph_mode`` sets ``graph_mode`` on the quantizer and every module that has the attribute
        and the reference's TF32 matmul flags (controller.py:301-307); the graph replay itself is
        ``enable_graph_mode``. Sets ``traced_model`` and ``target_dict`` and returns the former."""
        self._check_config()
        self.layer_clamp = 3.0  # controller.py:61
        traced, chosen = self.select_layers()
        if quantizer:
            self.iterate()
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
                entry["DIVISION"] = self._division_for(target)
                self.meta[target] = entry
                parent, _, child = target.rpartition(".")
                new = self._new_module(target, mod)
                setattr(traced.get_submodule(parent), child, new)
                # the traced module shares every submodule but the root with self.model; swap the
                # root's children there too, so the model holds the same layers as traced_model
                setattr(self.model.get_submodule(parent), child, new)
            traced.graph.eliminate_dead_code()
            traced.graph.lint()
            traced.recompile()
        self.traced_model = traced.to(self.device).train()
        self.target_dict = chosen
        if graph_mode:
            self._set_graph_mode()
        return self.traced_model

    def _set_graph_mode(self):
        torch.backends.cuda.matmul.allow_tf32 = True
        torch.backends.cudnn.allow_tf32 = True
        torch.set_float32_matmul_precision("high")
        self.quantizer.graph_mode = True
        for m in self.traced_model.modules():
            if hasattr(m, "graph_mode"):
                m.graph_mode = True

    def enable_graph_mode(self, stream=None):
        """controller.py:318-331. The reference compiles the rewritten model with
        ``torch.compile(fullgraph=True, mode='reduce-overhead')`` on ``stream``; here the
        model's training forward and backward become HIP-graph replays, captured on its first
        training call (``graph.graph_module_in_place``). ``stream`` is accepted for the
        reference's signature: capture runs on a side stream of its own, replays on the caller's
        current stream."""
        from .graph import graph_module_in_place

        if self.traced_model is None:
            raise RuntimeError("enable_graph_mode needs warp_model() first")
        self._set_graph_mode()
        graph_module_in_place(self.traced_model)
        if self.device.type == "cuda":
            torch.cuda.synchronize()

    def warmup(self, data_loader, criterion, stream=None):
        """controller.py:335-351: ``iterate``, ``warp_model(graph_mode=True, quantizer=True)``,
        ``enable_graph_mode`` and one bf16-autocast forward and backward on a batch of
        ``data_loader`` (on ``stream`` when one is given), which captures the graphs. The
        backward's gradients stay in ``.grad`` as in the reference."""
        self.iterate(criterion)
        self.warp_model(graph_mode=True, quantizer=True)
        self.enable_graph_mode(stream)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream() if stream is None else stream
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            with torch.autocast("cuda", dtype=torch.bfloat16):
                x, y = next(iter(data_loader))
                x, y = x.to("cuda", non_blocking=True), y.to("cuda", non_blocking=True)
                loss = criterion(self.traced_model(x), y)
            loss.backward()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()


__all__ = ["Controller", "find_group_size", "layer_group_meta", "compute_activation_size_in_bytes"]
