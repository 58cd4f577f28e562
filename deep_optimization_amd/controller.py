"""Per-layer compression meta: group size, padding and group counts.

Mirrors the host arithmetic the reference's Controller runs once per layer while it rewrites a
model (Activation_Compression/controller.py:127-177 and :364-390), so a layer's ``meta`` entry
(group_size, act_padding, N, NG) comes out the same:

  * ``find_group_size(S, bits, special)`` takes the first of [512, 256, 128, 64] (BatchNorm:
    [1024, 512, 256, 128, 64]) that divides the per-sample (per-channel for BatchNorm) element
    count S, else (256, act_padding=True) (controller.py:364-378). Bits outside {1, 2, 4, 8} also
    fall through to (256, True), as in the reference.
  * ``layer_group_meta(shape, bits, batchnorm)`` restates controller.py:127-177: the grouped
    extent is C*H*W per sample (C*L for 3-D, features for 2-D), or N*H*W per channel for
    BatchNorm, and G = ceil(S / group_size).
"""
from __future__ import annotations

from typing import Dict, Sequence, Tuple

import torch

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


__all__ = ["find_group_size", "layer_group_meta", "compute_activation_size_in_bytes"]
