"""Quantize / dequantize plumbing between the autograd Functions and the act_lib operators.

Mirrors Activation_Compression/modules/module_utils.py:28-102: ``quantize``, ``unified_quantize``,
``dequantize`` and ``unified_dequantize`` keep their names, positional arguments and the 14-field
meta tuple

    (bits, pack_only, group_size, act_padding, N, G, new_H, new_W, spatical_padding_eligibility,
     spatical_reshape_eligibility, channel_mean, avg_alam, alam_bits, ori_shape)

(reference :37, :51), so layers written against the reference can save and restore activations
through this module unchanged.

What differs is where the work happens:
  * the spatial-tile grouping is read in place by act_lib::quant_pack_tiles and written back by
    act_lib::dequant_unpack_tiles, so neither the permuted copy of the forward pass
    (tensor_act_reshape_utils.py:128) nor the inverse copy of the backward pass (:152) exists;
  * the per-layer ``meta`` dict may carry four optional keys the reference does not have:
      'rounding'    'nearest' (default, the reference), 'stochastic' (Philox noise) or
                    'stochastic_noise' (needs 'noise', a [N, G, g] fp32 tensor in [0, 1))
      'squash'      apply tanh(x/0.5)*0.5 before min/max (default True, as the reference does)
      'scale_dtype' torch.bfloat16 (default, as the reference) or torch.float32
      'seed'        Philox key (default 0); the Philox offset advances by one per call.
"""
from __future__ import annotations

import itertools

import torch
import torch.nn.functional as F

from .. import act_lib  # noqa: F401  (registers torch.ops.act_lib.*)
from .tensor_act_reshape_utils import (
    default_act_tensor_reshape,
    spatical_aware_act_tensor_reshape,
    spatical_aware_act_tensor_reshape_back,
    tile_layout_applies,
)

_philox_offsets = itertools.count()


def next_philox_offset() -> int:
    """Per-process Philox offset: a fresh noise stream for every stochastic quantize call."""
    return next(_philox_offsets)


def quantize(input, bits, pack_only, group_size, act_padding, N, avg_alam, alam_bits, clamp, clamp_alpha, *,
             rounding="nearest", squash=True, scale_dtype=torch.bfloat16, seed=0, offset=None, noise=None):
    """-> ((packed, scale, min), meta tuple); reference module_utils.py:28-55."""
    rn = act_lib.rounding_code(rounding)
    if rn == act_lib.ROUND_STOCH_PHILOX and offset is None:
        offset = next_philox_offset()
    offset = offset or 0

    if not act_padding and tile_layout_applies(input, group_size, act_padding) and not pack_only:
        n, c, h, w = input.shape
        s = int(round(group_size ** 0.5))
        out, scaler, xmin = torch.ops.act_lib.quant_pack_tiles(
            input, bits, group_size, clamp, clamp_alpha, squash, rn, noise, seed, offset, scale_dtype)
        G = scaler.shape[1]
        return (out, scaler, xmin), (bits, pack_only, group_size, act_padding, n, G, h // s, w // s, False, True,
                                     False, avg_alam, alam_bits, input.shape)

    groups, N, G, new_H, new_W, ori_shape, pad_elig, reshape_elig, channel_mean = spatical_aware_act_tensor_reshape(
        input, Group_Size=group_size, act_padding=act_padding, pack_only=pack_only)
    if pack_only:
        # the meta keeps the tile flags: the reference's pack-only meta (module_utils.py:40,55) drops them,
        # so a mask grouped into spatial tiles came back in flat order wherever H x W holds several tiles
        out = torch.ops.act_lib.pack_triton(groups, bits, group_size)
        return (out, None, None), (bits, pack_only, group_size, act_padding, N, G, new_H, new_W, pad_elig,
                                   reshape_elig, channel_mean, None, None, ori_shape)
    if avg_alam:
        out, scaler, xmin = torch.ops.act_lib.quant_pack_triton(groups, bits, group_size, avg_alam, alam_bits, clamp,
                                                                clamp_alpha)
    else:
        out, scaler, xmin = torch.ops.act_lib.quant_pack(groups, bits, group_size, clamp, clamp_alpha, squash, rn,
                                                         noise, seed, offset, scale_dtype)
    return (out, scaler, xmin), (bits, pack_only, group_size, act_padding, N, G, new_H, new_W, pad_elig,
                                 reshape_elig, channel_mean, avg_alam, alam_bits, ori_shape)


def unified_quantize(input, input_l, target_name, meta, clamp, clamp_alpha):
    """Reference module_utils.py:58-62, reading the optional rounding keys from meta."""
    m = meta[f"{target_name}"]
    q_tensor, q_meta = quantize(
        input, m["bits"], m["pack_only"], m["group_size"], m["act_padding"], m["N"], m["AVG_ALAM"], m["ALAM_BITS"],
        clamp, clamp_alpha, rounding=m.get("rounding", "nearest"), squash=m.get("squash", True),
        scale_dtype=m.get("scale_dtype", torch.bfloat16), seed=m.get("seed", 0), noise=m.get("noise"))
    return q_tensor, q_meta, input_l


def dequantize(quantized_tensor, quantized_meta):
    """Reference module_utils.py:65-83: bf16 activations in the original shape."""
    q_input, q_scale, q_min = quantized_tensor
    (bits, pack_only, group_size, act_padding, N, G, new_H, new_W, pad_elig, reshape_elig, channel_mean, avg_alam,
     alam_bits, input_shape) = quantized_meta
    if pack_only:
        unpack = torch.ops.act_lib.unpack_triton(q_input, bits, N, G, group_size)
    elif reshape_elig and not channel_mean and not avg_alam:
        n, c, h, w = input_shape
        return torch.ops.act_lib.dequant_unpack_tiles(q_input, q_scale, q_min, bits, group_size, n, c, h, w,
                                                      torch.bfloat16)
    else:
        unpack = torch.ops.act_lib.dequant_unpack_triton(q_input, q_scale, q_min, bits, group_size, bool(avg_alam),
                                                         alam_bits or 0)
    return spatical_aware_act_tensor_reshape_back(unpack, input_shape, group_size, new_H, new_W, act_padding,
                                                  pad_elig, reshape_elig, channel_mean)


def unified_dequantize(ori_quantized_tensor, ori_quantized_meta, input_l):
    """Reference module_utils.py:86-102: adds back the nearest-upsampled low-pass when present."""
    input_shape = ori_quantized_meta[-1]
    x = dequantize(ori_quantized_tensor, ori_quantized_meta)
    if input_l is None:
        return x
    if len(input_shape) == 4:
        size = (input_shape[-2], input_shape[-1])
    elif len(input_shape) == 3:
        size = input_shape[2]
    else:
        size = input_shape[0]
    return x + F.interpolate(input_l, size=size, scale_factor=None, mode="nearest").to(torch.bfloat16)


__all__ = ["quantize", "unified_quantize", "dequantize", "unified_dequantize", "default_act_tensor_reshape"]
