"""Group layout of an activation tensor: [N, ...] -> [N, G, g] and back.

Mirrors Activation_Compression/modules/tensor_act_reshape_utils.py (same function names,
arguments and return tuples) so that callers written against the reference keep working:

  * flat: ``x.reshape(N, -1, g)`` (reference :46), optionally zero-padded per sample to a
    multiple of g when ``act_padding`` (reference :36-44; the pad zeros take part in min/max);
  * spatial tiles: a 4-D [N, C, H, W] tensor with s = int(sqrt(g)), s*s == g and H, W divisible
    by s is grouped into s x s tiles, group k of sample n = (c, th, tw) holding
    x[n, c, th*s + i, tw*s + j] at element i*s + j (reference :100-128).

The compressed path in ``module_utils`` does not call the tile functions: the gfx950 kernels
read and write the tile layout in place (act_lib::quant_pack_tiles / dequant_unpack_tiles).
They remain for the pack-only path and for callers that want the materialised layout.

Deliberate differences from the reference (its results for these inputs are errors or wrong):
  * ``spatical_aware_act_tensor_reshape_back`` inverts the tile layout correctly for any H, W;
    the reference views the tile grid as (new_W, new_H) (:138), which scrambles non-square maps;
  * a 4-D tensor whose H and W are divisible by int(sqrt(g)) while g is not a perfect square
    raises a RuntimeError naming the cause (the reference fails inside ``view``).
"""
from __future__ import annotations

import math
from functools import reduce
import operator
from typing import Tuple

import torch.nn.functional as F
from torch import Tensor


def _tile_side(group_size: int) -> int:
    return int(math.isqrt(int(group_size)))


def default_act_tensor_reshape(X: Tensor, Group_Size: int, act_padding: bool, pack_only: bool):
    """-> (x [N, G, g], N, G, original shape, channel_mean=False) (reference :17-49)."""
    N = X.shape[0]
    shape = X.shape
    if act_padding:
        flat = X.reshape(N, -1)
        pad = (-flat.shape[1]) % Group_Size
        if pad:
            flat = F.pad(flat, (0, pad))
        X = flat
    x2 = X.reshape(N, -1, Group_Size)
    return x2, N, x2.shape[1], shape, False


def default_act_tensor_reshape_back(X: Tensor, _shape, act_padding: bool, channel_mean: bool) -> Tensor:
    """Inverse of default_act_tensor_reshape: drops the padding (reference :53-68)."""
    N = _shape[0]
    flat = X.reshape(N, -1)
    if act_padding:
        flat = flat[:, : reduce(operator.mul, _shape[1:], 1)]
    out = flat.reshape(*_shape)
    if channel_mean:
        out = out.repeat(1, 2, 1, 1)
    return out


def act_tensor_reshape_pad_hepler(X: Tensor, H: int, W: int, sgs: int):
    """Zero-pads H and W up to multiples of sgs; returns (X, H/sgs, W/sgs) (reference :72-79)."""
    pad_h = (-H) % sgs
    pad_w = (-W) % sgs
    if pad_h or pad_w:
        X = F.pad(X, (0, pad_w, 0, pad_h))
    return X, X.shape[2] // sgs, X.shape[3] // sgs


def spatical_aware_act_tensor_reshape_eligibility(X: Tensor, Group_Size: int, act_padding: bool) -> Tuple[bool, bool]:
    """-> (g is NOT a perfect square, H and W divisible by int(sqrt(g))) (reference :82-96)."""
    if act_padding or X.dim() != 4:
        return False, False
    s = _tile_side(Group_Size)
    return s * s != Group_Size, (X.shape[2] % s == 0) and (X.shape[3] % s == 0)


def tile_layout_applies(X: Tensor, Group_Size: int, act_padding: bool) -> bool:
    """True when the reference groups X into spatial tiles; raises for the case it cannot do."""
    not_square, divisible = spatical_aware_act_tensor_reshape_eligibility(X, Group_Size, act_padding)
    if divisible and not_square:
        raise RuntimeError(
            f"spatial tile grouping needs a square group size: group_size={Group_Size} is not s*s "
            f"although H={X.shape[2]} and W={X.shape[3]} are divisible by s={_tile_side(Group_Size)}")
    return divisible


def spatical_aware_act_tensor_reshape(X: Tensor, Group_Size: int, act_padding: bool, pack_only: bool):
    """-> (x [N, G, g], N, G, new_H, new_W, shape, padding_elig, reshape_elig, channel_mean)
    (reference :100-128)."""
    if not tile_layout_applies(X, Group_Size, act_padding):
        x2, N, G, shape, channel_mean = default_act_tensor_reshape(X, Group_Size, act_padding, pack_only)
        return x2, N, G, 0, 0, shape, False, False, channel_mean
    N, C, H, W = X.shape
    s = _tile_side(Group_Size)
    nh, nw = H // s, W // s
    tiles = X.reshape(N, C, nh, s, nw, s).permute(0, 1, 2, 4, 3, 5).reshape(N, C * nh * nw, Group_Size)
    return tiles.contiguous(), N, C * nh * nw, nh, nw, X.shape, False, True, False


def spatical_aware_act_tensor_reshape_back(X: Tensor, _shape, Group_Size: int, new_H: int, new_W: int,
                                           act_padding: bool, spatical_padding_eligibility: bool,
                                           spatical_reshape_eligibility: bool, channel_mean: bool) -> Tensor:
    """Inverse of spatical_aware_act_tensor_reshape (reference :131-154, corrected for H != W)."""
    if not spatical_reshape_eligibility:
        return default_act_tensor_reshape_back(X, _shape, act_padding, channel_mean).contiguous()
    N, C = _shape[0], _shape[1]
    s = _tile_side(Group_Size)
    out = X.reshape(N, C, new_H, new_W, s, s).permute(0, 1, 2, 4, 3, 5).reshape(N, C, new_H * s, new_W * s)
    out = out[:, :, : _shape[2], : _shape[3]]
    if channel_mean:
        out = out.reshape(*_shape).repeat(1, 2, 1, 1)
    return out.contiguous()
