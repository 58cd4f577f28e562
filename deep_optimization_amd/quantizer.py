"""Quantizer: the per-layer bit-width table the Controller reads, and the DIVISION layer analysis.

Mirrors Activation_Compression/quantizer.py with the reference's names and arguments:

  * ``Quantizer(config, target_dict)`` (:13-23) holds ``bits`` ({target: bits}), ``default_bit``,
    ``config``, ``dims``, ``unrelated_tensors`` and ``graph_mode``;
  * ``filter_tensors(pairs)`` (:25-27) records the storage of every (name, tensor) pair, the
    model's parameters, as never quantized;
  * ``check_quantize(t)`` (:29-45) says whether a tensor is one the quantizer would compress:
    not a recorded parameter, a floating dtype (fp16/bf16/fp32), requiring grad, and 2-, 3- or
    4-D. The reference's version is never called and raises on its rank test (it compares a
    shape with an int before taking ``len``); this one implements the checks it spells out;
  * ``clean_iterate()`` (:47-49) empties ``bits`` and ``dims``;
  * ``iterate(model, criterion, dataloader)`` (:51-80): with ``config['auto_precision']`` None
    every target in ``bits`` gets ``config['default_bits']``. The other branch of the reference
    runs a low-rank eigen-analysis of the activations (:290-356, research code that feeds no
    bit-width back: its result is only stored); here it raises ``NotImplementedError``;
  * ``select_division_layer_helper(model, criterion, dataloader)`` (:170-288): one bf16-autocast
    forward and backward on 64 training samples, then per Conv/Linear layer the low-frequency
    energy ratio (LFER) of its weight gradient and of its input activation, the LARS trust ratio
    |W| / |dW|, the gradient signal-to-noise ratio |mean dW| / std dW and the input variance.
    The Controller's DIVISION selection reads the LFER of the gradient (controller.py:198-204).

Differences from the reference, all in the analysis's side effects, none in its statistics:
  * the forward hooks it registers are removed afterwards (the reference leaves them on the
    modules, where they keep every later forward's input alive);
  * the parameters' ``.grad`` are restored to what they were before its backward;
  * the 64 samples are the first 64 of ``dataloader.dataset`` in order (the reference shuffles
    them; the statistics are sums over the batch, so only BatchNorm's batch statistics see the
    order), or, for a loader without a ``dataset`` (a list of batches), the first 64 of its first
    batch.
"""
from __future__ import annotations

from typing import Dict, Iterable, Tuple

import torch
import torch.nn.functional as F
from torch import nn

_DIVISION_LAYERS = (nn.Conv3d, nn.Conv2d, nn.Conv1d, nn.Linear)
_FLOAT_DTYPES = (torch.float16, torch.float32, torch.bfloat16)


class Quantizer:
    def __init__(self, config: dict, target_dict: dict):
        self.unrelated_tensors = set()
        self.default_bit = config["default_bits"]
        self.config = config
        self.bits = target_dict
        self.dims = {}
        self.graph_mode = False

    def filter_tensors(self, pair: Iterable[Tuple[str, torch.Tensor]]) -> None:
        for _, v in pair:
            self.unrelated_tensors.add(v.data_ptr())

    def check_quantize(self, input_tensor: torch.Tensor) -> bool:
        if input_tensor.data_ptr() in self.unrelated_tensors:
            return False
        if input_tensor.dtype not in _FLOAT_DTYPES:
            return False
        if not input_tensor.requires_grad:
            return False
        return input_tensor.dim() in (2, 3, 4)

    def clean_iterate(self) -> None:
        self.bits.clear()
        self.dims.clear()

    def iterate(self, model=None, criterion=None, dataloader=None) -> None:
        if self.config.get("auto_precision") is None:
            for target in self.bits:
                self.bits[target] = self.config["default_bits"]
            return
        raise NotImplementedError(
            "Quantizer.iterate with config['auto_precision'] set runs the reference's Hessian / low-rank "
            "activation analysis (Activation_Compression/quantizer.py:80, :290-356). That analysis assigns no bit "
            "widths and is outside this library; use auto_precision=None (every layer gets default_bits) or "
            "set per-layer widths in config['bits']")

    # -- DIVISION layer analysis (quantizer.py:170-288) ------------------------------------------

    def select_division_layer_helper(self, model: nn.Module, criterion, dataloader, device=None):
        """-> (lfer_grad, lfer_act, lars_trust_ratio, signal_noise_ratio, activation_var), each a
        {module name: float} over the model's Conv1d/2d/3d and Linear layers that got a gradient."""
        device = torch.device(device) if device is not None else next(model.parameters()).device
        x, y = _first_samples(dataloader, 64)
        x, y = x.to(device), y.to(device)
        model.train()
        cache: Dict[str, torch.Tensor] = {}
        hooks = []
        for name, module in model.named_modules():
            if isinstance(module, _DIVISION_LAYERS):
                hooks.append(module.register_forward_hook(
                    lambda m, inp, out, name=name: cache.__setitem__(name, inp[0])))
        saved_grads = {p: p.grad for p in model.parameters()}
        for p in saved_grads:
            p.grad = None
        try:
            with torch.autocast(device.type, dtype=torch.bfloat16):
                raw = model(x)
                logits = raw[0] if isinstance(raw, tuple) else raw
                loss = criterion(logits, y)
            loss.backward()
            lfer_grad, lfer_act, lars, snr, act_var = {}, {}, {}, {}, {}
            with torch.no_grad():
                for name, module in model.named_modules():
                    if not isinstance(module, _DIVISION_LAYERS) or module.weight.grad is None:
                        continue
                    w, dw = module.weight, module.weight.grad
                    lfer_grad[name] = lfer_of_grad(dw)
                    lfer_act[name] = lfer_of_act(cache[name])
                    lars[name] = torch.norm(w).item() / (torch.norm(dw).item() + 1e-7)
                    snr[name] = torch.abs(dw.mean()).item() / (torch.sqrt(dw.var()) + 1e-7).item()
                    act_var[name] = cache[name].var().item()
        finally:
            for h in hooks:
                h.remove()
            for p, g in saved_grads.items():
                p.grad = g
        return lfer_grad, lfer_act, lars, snr, act_var


def _first_samples(dataloader, n: int):
    dataset = getattr(dataloader, "dataset", None)
    if dataset is not None:
        m = min(n, len(dataset))
        xs, ys = zip(*(dataset[i] for i in range(m)))
        x = torch.stack([torch.as_tensor(v) for v in xs])
        y = torch.stack([torch.as_tensor(v) for v in ys])
        return x, y
    x, y = next(iter(dataloader))
    return x[:n], y[:n]


@torch.no_grad()
def lfer_of_act(x: torch.Tensor, k: int = 4) -> float:
    """Low-frequency energy ratio of a layer input (quantizer.py:190-205): |lowpass(x)|^2 / |x|^2,
    the low pass a k x k (4-D) or length-k (3-D, last axis) average pool expanded back by nearest
    interpolation; for a 2-D input the mean over the feature axis."""
    if x.dim() == 4:
        H, W = x.shape[-2:]
        k = min(k, H, W)
        lp = F.interpolate(F.avg_pool2d(x, kernel_size=k, stride=k, padding=0), size=x.shape[-2:], mode="nearest")
    else:
        feat = x.shape[-1]
        k = min(k, feat)
        if x.dim() != 2:
            lp = F.interpolate(F.avg_pool1d(x, kernel_size=k, stride=k, padding=0), size=feat, mode="nearest")
        else:
            lp = x.mean(dim=-1, keepdim=True).expand_as(x)
    return (lp.square().sum() / (x.square().sum() + 1e-7)).item()


@torch.no_grad()
def lfer_of_grad(dW: torch.Tensor, k: int = 4) -> float:
    """Low-frequency energy ratio of a weight gradient (quantizer.py:207-258). 2-D (Linear): the
    row mean; 3-D (Conv1d): a length-k average pool with stride 3 (as the reference has it)
    expanded back; 4-D (Conv2d): a k x k average pool over the kernel window expanded back; 1 when
    the pooled axis has extent 1 (a 1x1 kernel, a single input feature); otherwise the mean over
    the last axis."""
    if dW.dim() == 2:
        if dW.shape[-1] == 1:
            return 1
        lf = dW.mean(dim=-1, keepdim=True).expand_as(dW)
    elif dW.dim() == 3:
        feat = dW.shape[-1]
        if feat == 1:
            return 1
        k = min(k, feat)
        lf = F.interpolate(F.avg_pool1d(dW, kernel_size=k, stride=3, padding=0), size=feat, mode="nearest")
    elif dW.dim() == 4:
        H, W = dW.shape[-2:]
        if H == 1 and W == 1:
            return 1
        k = min(k, H, W)
        lf = F.interpolate(F.avg_pool2d(dW, kernel_size=k, stride=k, padding=0), size=(H, W), mode="nearest")
    else:
        if dW.shape[0] == 1:
            return 1
        lf = dW.mean(dim=-1, keepdim=True).expand_as(dW)
    return (lf.square().sum() / (dW.square().sum() + 1e-7)).item()


__all__ = ["Quantizer", "lfer_of_act", "lfer_of_grad"]
