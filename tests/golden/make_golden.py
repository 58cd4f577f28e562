"""Generates the committed golden fixtures (tests/golden/cases.npz) with the CPU oracle.

The reference has no fixtures for this path, so these are the build's own: seeded inputs and the
oracle's packed words, scale, min and dequantized output for a handful of small configurations,
including the reference's CPU case (fp32 [8, 64, 32, 32] ~ N(0,1), seed 0, g = 256, 2-bit, nearest,
16 x 16 spatial tiles, fp32 min + scale; the input is regenerated from the seed, not stored).
GPU tests compare the HIP kernels to these arrays; tests/test_oracle.py checks that the oracle
still reproduces them.

Run: python -m tests.golden.make_golden
"""
from __future__ import annotations

import os

import numpy as np
import torch

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "cases.npz")


def c1_input() -> np.ndarray:
    g = torch.Generator().manual_seed(0)
    return torch.randn(8, 64, 32, 32, generator=g, dtype=torch.float32).numpy()


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


# name -> (input builder, kwargs); inputs are numpy arrays (bf16 as uint16 bit patterns)
def _cases():
    def bf16_noise(bits, seed):
        def build():
            gen = torch.Generator().manual_seed(seed)
            x = torch.randn(4, 24, 256, generator=gen).abs_()
            u = torch.rand(4, 24, 256, generator=gen)
            return {"x": _bf16_bits(x), "noise": u.numpy()}
        return build, dict(group_size=256, bits=bits, rounding=oracle.STOCH_NOISE, meta_dtype=oracle.F32,
                           y_dtype=oracle.BF16)

    cases = {
        "c1_cpu_config": (lambda: {}, dict(group_size=256, bits=2, rounding=oracle.NEAREST, meta_dtype=oracle.F32,
                                           tile=(8, 64, 32, 32), y_dtype=oracle.F32, store_input=False)),
        "f16_g128_philox_b4": (
            lambda: {"x": torch.randn(3, 10, 128, generator=torch.Generator().manual_seed(11)).half().numpy()},
            dict(group_size=128, bits=4, rounding=oracle.STOCH_PHILOX, seed=1, offset=0, meta_dtype=oracle.F32,
                 y_dtype=oracle.F32)),
        "bf16_tiles_g64_b2_bf16meta": (
            lambda: {"x": _bf16_bits(torch.randn(2, 3, 16, 24, generator=torch.Generator().manual_seed(12)))},
            dict(group_size=64, bits=2, rounding=oracle.NEAREST, meta_dtype=oracle.BF16, tile=(2, 3, 16, 24),
                 y_dtype=oracle.BF16)),
        "f32_g1024_squash_clamp_b8": (
            lambda: {"x": (torch.randn(2, 3, 1024, generator=torch.Generator().manual_seed(13)) * 2).numpy()},
            dict(group_size=1024, bits=8, rounding=oracle.NEAREST, meta_dtype=oracle.BF16, flags=3,
                 clamp_alpha=3.0, y_dtype=oracle.BF16)),
    }
    for bits in (1, 2, 4, 8):
        cases[f"bf16_noise_b{bits}"] = bf16_noise(bits, 100 + bits)
    return cases


CASES = _cases()


def compute_case(name: str) -> dict:
    build, kw = CASES[name]
    arrays = build()
    if name == "c1_cpu_config":
        x = c1_input()
    else:
        x = arrays["x"]
    g, bits = kw["group_size"], kw["bits"]
    tile = kw.get("tile")
    packed, scale, mn = oracle.quant_pack(
        x.reshape(-1) if tile is None else x, g, bits, tile_nchw=tile, rounding=kw["rounding"],
        noise=arrays.get("noise"), seed=kw.get("seed", 0), offset=kw.get("offset", 0), flags=kw.get("flags", 0),
        clamp_alpha=kw.get("clamp_alpha", 0.0), meta_dtype=kw["meta_dtype"])
    y = oracle.dequant_unpack(packed, scale, mn, g, bits, tile_nchw=tile, y_dtype=kw["y_dtype"])
    out = {"packed": packed, "scale": scale, "min": mn}
    if name != "c1_cpu_config":
        out.update(arrays)
        out["y"] = y
    return out


def load_all() -> dict:
    data = np.load(PATH, allow_pickle=False)
    out: dict = {}
    for key in data.files:
        name, field = key.split(".", 1)
        out.setdefault(name, {})[field] = data[key]
    return out


def main() -> None:
    flat = {}
    for name in CASES:
        for field, arr in compute_case(name).items():
            flat[f"{name}.{field}"] = arr
    np.savez_compressed(PATH, **flat)
    print(f"wrote {PATH} ({os.path.getsize(PATH)} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
