"""Pins the CPU oracle (oracle/dopt_oracle.c) before it is used to check the HIP kernels.

The reference ships no tests, golden vectors or fixtures for this path (its Triton kernels need an
NVIDIA GPU), so each oracle function is pinned by something independent of its own formula:
hand-computed known-answer groups, a library routine the format reduces to (numpy.packbits,
torch's bf16 rounding), published Philox known-answer vectors, an independent vectorised numpy
restatement, brute-force index maps for the tile layout, and error bounds / unbiasedness that
any correct quantizer must satisfy. A planted mistake (dropped +0.5 bias, swapped shift order,
transposed tile index, RNE instead of truncation) fails at least one test here.
"""
import numpy as np
import pytest
import torch

import oracle
from tests.restate import (_ulp32, f64_pretransform, fma32, numpy_quant, packbits_reference, squash_inputs,  # noqa: F401
                           squash_mismatch)

F32, BF16 = oracle.F32, oracle.BF16
NEAREST, NOISE, PHILOX = oracle.NEAREST, oracle.STOCH_NOISE, oracle.STOCH_PHILOX


@pytest.fixture(autouse=True)
def _lib(oracle_lib):
    return oracle_lib


def words_to_bytes(packed):
    return np.ascontiguousarray(packed, dtype="<u4").view(np.uint8)


# ----------------------------------------------------------------------------- Philox
# Known-answer vectors of the Random123 distribution (kat_vectors, "philox4x32 10" lines):
# counter, key -> output.
PHILOX_KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.mark.parametrize("ctr,key,want", PHILOX_KAT)
def test_philox_known_answers(ctr, key, want):
    assert list(oracle.philox4x32_10(ctr, key)) == want


def test_philox_noise_element_mapping():
    # block 0 (elements 0..15) of seed 0 / offset 0 is the first KAT vector; element k takes
    # byte (k & 3) of word k >> 2, u = (b + 0.5) / 256
    w = PHILOX_KAT[0][2]
    bts = [(w[k >> 2] >> (8 * (k & 3))) & 0xFF for k in range(16)]
    want = (np.array(bts, dtype=np.float64) + 0.5) / 256.0
    got = oracle.philox_noise(0, 16, 0, 0)
    np.testing.assert_array_equal(got.astype(np.float64), want)
    # block 1 (elements 16..31) is the call with counter {1, 0, 0, 0}: a different KAT-derived stream
    w1 = oracle.philox4x32_10([1, 0, 0, 0], [0, 0])
    bts1 = [(int(w1[k >> 2]) >> (8 * (k & 3))) & 0xFF for k in range(16)]
    np.testing.assert_array_equal(oracle.philox_noise(16, 16, 0, 0).astype(np.float64),
                                  (np.array(bts1, dtype=np.float64) + 0.5) / 256.0)
    # the offset is the high half of the counter, the seed the key
    w2 = oracle.philox4x32_10([3, 0, 7, 0], [5, 0])
    b2 = (int(w2[1]) >> 8) & 0xFF  # element 16*3 + 5 -> word 1, byte 1
    assert oracle.philox_noise(16 * 3 + 5, 1, 5, 7)[0] == np.float32((b2 + 0.5) / 256.0)


def test_philox_noise_statistics():
    u = oracle.philox_noise(0, 1 << 18, 1234, 7)
    assert u.min() > 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 3e-3
    assert abs(u.var() - 1.0 / 12.0) < 2e-3
    # different offsets give different streams
    v = oracle.philox_noise(0, 1 << 10, 1234, 8)
    assert np.mean(u[: 1 << 10] == v) < 0.01


# ----------------------------------------------------------------------------- known answers
def test_kat_ramp_nearest():
    # codes 0,1,2,3 repeating: min 0, max 3 -> step 1, word 0b11100100 per byte
    x = np.tile(np.arange(4, dtype=np.float32), 16)[None, :]
    packed, scale, mn = oracle.quant_pack(x, 64, 2)
    assert scale[0] == 1.0 and mn[0] == 0.0
    assert np.all(packed == 0xE4E4E4E4)
    y = oracle.dequant_unpack(packed, scale, mn, 64, 2)
    np.testing.assert_array_equal(y, x)


def test_kat_half_steps_round_down():
    # (x - min) * inv lands exactly on k + 0.5: + (0.5 - 1e-6) truncates to k (not RNE, not up)
    base = np.array([0, 0.5, 1, 1.5, 2, 2.5, 3, 3], dtype=np.float32)
    x = np.tile(base, 8)[None, :]
    packed, scale, mn = oracle.quant_pack(x, 64, 2)
    codes = oracle.unpack_codes(packed, 64, 2)[0]
    np.testing.assert_array_equal(codes[:8], [0, 0, 1, 1, 2, 2, 3, 3])


def test_kat_constant_group():
    x = np.full((3, 128), 5.25, dtype=np.float32)
    packed, scale, mn = oracle.quant_pack(x, 128, 4)
    assert np.all(scale == 1.0) and np.all(mn == 5.25) and np.all(packed == 0)
    np.testing.assert_array_equal(oracle.dequant_unpack(packed, scale, mn, 128, 4), x)


def test_kat_stochastic_with_noise():
    # min 0, max 3 -> step 1; q = rint((x + u) - 0.5), ties to even
    x = np.zeros((1, 64), dtype=np.float32)
    u = np.zeros((1, 64), dtype=np.float32)
    x[0, 1] = 3.0
    cases = [(1.25, 0.3, 1), (1.25, 0.8, 2), (2.5, 0.0, 2), (2.5, 0.5, 2), (1.5, 0.5, 2),
             (0.0, 0.99, 0), (3.0, 0.99, 3), (3.0, 0.0, 2), (0.75, 0.25, 0), (0.75, 0.26, 1)]
    for i, (xv, uv, _) in enumerate(cases):
        x[0, 2 + i] = xv
        u[0, 2 + i] = uv
    packed, scale, mn = oracle.quant_pack(x, 64, 2, rounding=NOISE, noise=u)
    assert scale[0] == 1.0 and mn[0] == 0.0
    codes = oracle.unpack_codes(packed, 64, 2)[0]
    np.testing.assert_array_equal(codes[2:2 + len(cases)], [c[2] for c in cases])


def test_kat_negative_zero_min_is_canonical():
    x = np.full((1, 64), 1.0, dtype=np.float32)
    x[0, :8] = -0.0
    _, _, mn = oracle.quant_pack(x, 64, 1)
    assert mn.view(np.uint32)[0] == 0  # +0.0, not 0x80000000


def test_nan_codes_are_zero_and_ignored_by_minmax():
    x = np.linspace(-1, 1, 64, dtype=np.float32)[None, :].copy()
    x[0, 10] = np.nan
    packed, scale, mn = oracle.quant_pack(x, 64, 8)
    codes = oracle.unpack_codes(packed, 64, 8)[0]
    assert codes[10] == 0
    assert mn[0] == np.float32(-1.0) and scale[0] == np.float32(2.0) / np.float32(255.0)


# ----------------------------------------------------------------------------- library routines
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("g", [64, 256, 1024])
def test_pack_codes_equals_numpy_packbits(bits, g):
    rng = np.random.default_rng(bits * 1000 + g)
    # int8 codes: at 8 bits only 0..127 are non-negative (the sign-extension case is tested below)
    codes = rng.integers(0, min(1 << bits, 128), size=(5, g)).astype(np.int8)
    packed = oracle.pack_codes(codes, g, bits)
    np.testing.assert_array_equal(words_to_bytes(packed), packbits_reference(codes, bits))
    np.testing.assert_array_equal(oracle.unpack_codes(packed, g, bits), codes)


def test_pack_codes_wraps_like_int32_sum():
    # the reference sums int32(int8 code) << shift; negative codes sign-extend and carry
    codes = np.zeros((1, 64), dtype=np.int8)
    codes[0, 0] = -1
    codes[0, 1] = 1
    packed = oracle.pack_codes(codes, 64, 2)
    assert packed[0, 0] == np.uint32((0xFFFFFFFF + (1 << 2)) & 0xFFFFFFFF)


def test_bf16_meta_matches_torch_rounding():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 256)) * 3).astype(np.float32)
    _, s32, m32 = oracle.quant_pack(x, 256, 2, meta_dtype=F32)
    _, s16, m16 = oracle.quant_pack(x, 256, 2, meta_dtype=BF16)
    torch_s = torch.from_numpy(s32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    torch_m = torch.from_numpy(m32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(s16, torch_s)
    np.testing.assert_array_equal(m16, torch_m)


def test_bf16_output_matches_torch_rounding():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((32, 128)).astype(np.float32)
    p, s, m = oracle.quant_pack(x, 128, 8)
    y32 = oracle.dequant_unpack(p, s, m, 128, 8, y_dtype=F32)
    y16 = oracle.dequant_unpack(p, s, m, 128, 8, y_dtype=BF16)
    want = torch.from_numpy(y32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(y16, want)


def test_input_widening_bf16_f16():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 256)).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    xb_bits = xb.view(torch.int16).numpy().view(np.uint16)
    a = oracle.quant_pack(xb_bits, 256, 4)
    b = oracle.quant_pack(xb.float().numpy(), 256, 4)
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u, v)
    xh = x.astype(np.float16)
    a = oracle.quant_pack(xh, 256, 4)
    b = oracle.quant_pack(xh.astype(np.float32), 256, 4)
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u, v)


# ----------------------------------------------------------------------------- independent restatement
def test_fma32_emulation_is_exact():
    from fractions import Fraction
    rng = np.random.default_rng(99)
    a = (rng.standard_normal(4000) * np.exp2(rng.integers(-30, 30, 4000))).astype(np.float32)
    b = (rng.standard_normal(4000) * np.exp2(rng.integers(-30, 30, 4000))).astype(np.float32)
    c = (rng.standard_normal(4000) * np.exp2(rng.integers(-60, 60, 4000))).astype(np.float32)
    got = fma32(a, b, c)
    for i in range(4000):
        exact = Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i]))
        r = np.float32(float(exact))  # float(Fraction) is correctly rounded to f64 ...
        # ... so check the f32 neighbours directly: the result must be the nearest (ties to even)
        lo, hi = (np.nextafter(r, np.float32(-np.inf)), np.nextafter(r, np.float32(np.inf)))
        cands = sorted([lo, r, hi], key=lambda v: (abs(Fraction(float(v)) - exact),
                                                   int(np.float32(v).view(np.uint32)) & 1))
        assert got[i] == cands[0], (a[i], b[i], c[i])


def _fma_boundary_values(step_target, bits, per_boundary=2):
    """Values t in [0, QMAX*step] just around the code boundaries of a group with min 0, where
    fma(t, inv, 0.5-1e-6) and the separately rounded (t * inv) + (0.5-1e-6) truncate differently."""
    f = np.float32
    qmax = (1 << bits) - 1
    mx = f(step_target * qmax)
    step = f(mx / f(qmax))
    inv = f(f(1) / step)
    found = []
    for k in range(1, qmax + 1):
        target = f((k - f(0.5 - 1e-6)) / inv)
        cand = np.nextafter(np.full(401, target, dtype=f), np.inf if target >= 0 else -np.inf)
        ladder = target.view(np.uint32) + np.arange(-200, 201).astype(np.int64)
        cand = ladder.astype(np.uint32).view(f)
        cand = cand[(cand >= 0) & (cand <= mx)]
        fused = fma32(cand, np.full(cand.shape, inv), np.full(cand.shape, f(0.5 - 1e-6)))
        unfused = ((cand * inv).astype(f) + f(0.5 - 1e-6)).astype(f)
        hit = cand[np.floor(fused) != np.floor(unfused)]
        found.extend(hit[:per_boundary].tolist())
    return mx, np.array(found, dtype=f), inv


def test_nearest_uses_the_fused_multiply_add():
    # values where fma(t, inv, c) and the separately rounded (t * inv) + c truncate to different
    # codes: the oracle must follow the fused form (the reference's compiled arithmetic)
    bits, g = 8, 256
    rows = []
    for st in (0.013, 0.37, 1.9, 7.25):
        mx, vals, inv = _fma_boundary_values(st, bits)
        if len(vals) == 0:
            continue
        for i in range(0, len(vals), g - 2):
            chunk = vals[i:i + g - 2]
            row = np.full(g, mx / 2, dtype=np.float32)
            row[0], row[1] = 0.0, mx
            row[2:2 + len(chunk)] = chunk
            rows.append(row)
    x = np.array(rows, dtype=np.float32)
    assert len(x) > 0
    p, sc, mnv = oracle.quant_pack(x, g, bits)
    codes = oracle.unpack_codes(p, g, bits).view(np.uint8).astype(np.int64)
    inv = (np.float32(1) / sc).astype(np.float32)
    t = (x - mnv[:, None]).astype(np.float32)
    fused = fma32(t, np.broadcast_to(inv[:, None], t.shape), np.full(t.shape, np.float32(0.5 - 1e-6)))
    unfused = ((t * inv[:, None]).astype(np.float32) + np.float32(0.5 - 1e-6)).astype(np.float32)
    differ = np.floor(fused) != np.floor(unfused)
    assert differ.sum() >= 20, "too few distinguishing inputs"
    np.testing.assert_array_equal(codes, np.clip(np.floor(fused), 0, 255).astype(np.int64))


def test_dequant_uses_the_fused_multiply_add():
    rng = np.random.default_rng(321)
    q = rng.integers(0, 256, size=(64, 256)).astype(np.uint8)
    packed = q.view("<u4").reshape(64, -1).copy()
    sc = (rng.random(64) * 3).astype(np.float32)
    mn = rng.standard_normal(64).astype(np.float32)
    y = oracle.dequant_unpack(packed, sc, mn, 256, 8)
    want = fma32(q.astype(np.float32), np.broadcast_to(sc[:, None], q.shape), np.broadcast_to(mn[:, None], q.shape))
    np.testing.assert_array_equal(y, want)
    unfused = ((q.astype(np.float32) * sc[:, None]).astype(np.float32) + mn[:, None]).astype(np.float32)
    assert np.any(unfused != want)  # the check above can tell the two forms apart


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("rounding", [NEAREST, NOISE])
def test_oracle_equals_numpy_restatement(bits, rounding):
    rng = np.random.default_rng(10 + bits)
    g = 256
    x = (rng.standard_normal((200, g)) * rng.uniform(0.01, 10, (200, 1))).astype(np.float32)
    x[7] = 2.0  # a constant group
    u = rng.random((200, g), dtype=np.float32) if rounding == NOISE else None
    p, s, m = oracle.quant_pack(x, g, bits, rounding=rounding, noise=u)
    p2, s2, m2 = numpy_quant(x, bits, rounding, u)
    np.testing.assert_array_equal(s, s2)
    np.testing.assert_array_equal(m, m2)
    np.testing.assert_array_equal(p, p2)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_philox_mode_equals_noise_mode_with_the_philox_stream(bits):
    # Philox rounding is noise-tensor rounding with u = the element's Philox byte (pinned above by
    # the KAT vectors and the element mapping)
    rng = np.random.default_rng(50 + bits)
    g = 128
    x = rng.standard_normal((37, g)).astype(np.float32)
    u = oracle.philox_noise(0, x.size, 77, 5).reshape(x.shape)
    p, s, m = oracle.quant_pack(x, g, bits, rounding=PHILOX, seed=77, offset=5)
    p2, s2, m2 = numpy_quant(x, bits, NOISE, u)
    np.testing.assert_array_equal(p, p2)
    np.testing.assert_array_equal(s, s2)


# ----------------------------------------------------------------------------- layout
def test_tile_layout_equals_torch_permute():
    rng = np.random.default_rng(6)
    N, C, H, W, g = 2, 3, 32, 48, 256
    s = 16
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    tiles = (torch.from_numpy(x).view(N, C, H // s, s, W // s, s).permute(0, 1, 2, 4, 3, 5)
             .reshape(N, -1, g).contiguous().numpy())
    a = oracle.quant_pack(x, g, 2, tile_nchw=(N, C, H, W))
    b = oracle.quant_pack(tiles.reshape(-1, g), g, 2)
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u, v)
    y = oracle.dequant_unpack(*a, g, 2, tile_nchw=(N, C, H, W))
    yflat = oracle.dequant_unpack(*b, g, 2)
    back = (torch.from_numpy(yflat).view(N, C, H // s, W // s, s, s).permute(0, 1, 2, 4, 3, 5)
            .reshape(N, C, H, W).numpy())
    np.testing.assert_array_equal(y, back)


def test_tile_layout_brute_force_small():
    # g = 64 -> 8 x 8 tiles; group r = (c, th, tw) holds x[n, c, th*8 + i, tw*8 + j] at element
    # i*8 + j. The groups are built by explicit loops and quantised flat; the tile path must agree.
    N, C, H, W = 2, 2, 16, 24
    rng = np.random.default_rng(7)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    groups = []
    for n in range(N):
        for c in range(C):
            for th in range(H // 8):
                for tw in range(W // 8):
                    groups.append([x[n, c, th * 8 + i, tw * 8 + j] for i in range(8) for j in range(8)])
    flat = np.array(groups, dtype=np.float32)
    a = oracle.quant_pack(x, 64, 4, tile_nchw=(N, C, H, W))
    b = oracle.quant_pack(flat, 64, 4)
    for u, v in zip(a, b):
        np.testing.assert_array_equal(u, v)
    y_tiles = oracle.dequant_unpack(*a, 64, 4, tile_nchw=(N, C, H, W))
    y_flat = oracle.dequant_unpack(*b, 64, 4)
    r = 0
    for n in range(N):
        for c in range(C):
            for th in range(H // 8):
                for tw in range(W // 8):
                    np.testing.assert_array_equal(
                        y_tiles[n, c, th * 8:(th + 1) * 8, tw * 8:(tw + 1) * 8].reshape(-1), y_flat[r])
                    r += 1


# ----------------------------------------------------------------------------- bounds / statistics
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_nearest_error_bound(bits):
    rng = np.random.default_rng(20 + bits)
    x = rng.standard_normal((512, 256)).astype(np.float32)
    p, s, m = oracle.quant_pack(x, 256, bits)
    y = oracle.dequant_unpack(p, s, m, 256, bits)
    err = np.abs(y - x)
    step = s[:, None]
    # the reference's +(0.5 - 1e-6) bias allows step*(0.5 + 1e-6), plus fp32 rounding of q*step + min
    assert np.all(err <= step * 0.500002 + 1e-6 * (1 + np.abs(x)))
    assert np.mean(err > step / 2 + 1e-6) < 1e-4


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_stochastic_error_bound(bits):
    rng = np.random.default_rng(30 + bits)
    x = rng.standard_normal((256, 128)).astype(np.float32)
    p, s, m = oracle.quant_pack(x, 128, bits, rounding=PHILOX, seed=9, offset=3)
    y = oracle.dequant_unpack(p, s, m, 128, bits)
    assert np.all(np.abs(y - x) < s[:, None] * (1 + 1e-5))


def test_stochastic_is_unbiased():
    rng = np.random.default_rng(40)
    x = rng.standard_normal((1, 64)).astype(np.float32)
    n = 3000
    acc = np.zeros(64, dtype=np.float64)
    for off in range(n):
        p, s, m = oracle.quant_pack(x, 64, 2, rounding=PHILOX, seed=5, offset=off)
        acc += oracle.dequant_unpack(p, s, m, 64, 2)[0]
    mean = acc / n
    step = float(s[0])
    # std of one sample <= step/2; 8-bit noise quantisation adds at most step/2^9 of bias
    assert np.all(np.abs(mean - x[0]) < 5 * (step / 2) / np.sqrt(n) + step / 2 ** 9)


# ----------------------------------------------------------------------------- validation
def test_errors():
    x = np.zeros((1, 64), dtype=np.float32)
    with pytest.raises(ValueError):
        oracle.quant_pack(x, 64, 3)
    with pytest.raises(oracle.OracleError):
        oracle.quant_pack(np.zeros((1, 96), dtype=np.float32), 96, 2)
    with pytest.raises(oracle.OracleError):  # g = 128 is not a square: no tile layout
        oracle.quant_pack(np.zeros((1, 1, 22, 22), dtype=np.float32), 128, 2, tile_nchw=(1, 1, 22, 22))


# ----------------------------------------------------------------------------- committed fixtures
def test_golden_fixtures_regenerate():
    from tests.golden import make_golden

    for name, case in make_golden.load_all().items():
        fresh = make_golden.compute_case(name)
        for key in case:
            np.testing.assert_array_equal(case[key], fresh[key], err_msg=f"{name}:{key}")


# ----------------------------------------------------------------------------- fused activation layers
def _bf16(a):
    return oracle.f32_to_bf16_bits(np.asarray(a, dtype=np.float32))


def _f32(b):
    return oracle.bf16_bits_to_f32(b)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("relu6", [False, True])
@pytest.mark.parametrize("storage", ["f32", "bf16"])
def test_relu_pack_known_answers(bits, relu6, storage):
    rng = np.random.default_rng(60 + bits)
    x = (rng.standard_normal(1024) * 4).astype(np.float32)
    x[:8] = [0.0, -0.0, 6.0, 5.999, 1e-30, -1e-30, np.inf, -np.inf]
    xin = x if storage == "f32" else _bf16(x)
    xv = x if storage == "f32" else _f32(xin)
    y, packed = oracle.relu_pack(xin, bits, relu6)
    mask = ((xv > 0) & (xv < 6)) if relu6 else (xv > 0)
    want_y = np.where(mask, _f32(_bf16(xv)), 0.0).astype(np.float32)  # bf16-rounded as the reference stores it
    got_y = y if storage == "f32" else _f32(y)
    np.testing.assert_array_equal(got_y, want_y)
    assert np.all(got_y.view(np.uint32)[~mask] == 0)  # +0.0, not -0.0
    codes = mask.astype(np.int64).reshape(1, -1)
    np.testing.assert_array_equal(words_to_bytes(packed), packbits_reference(codes, bits)[0])


@pytest.mark.parametrize("bits", [1, 4])
def test_relu_unpack_closed_form(bits):
    rng = np.random.default_rng(70 + bits)
    mask = rng.random(512) < 0.5
    packed = packbits_reference(mask.astype(np.int64).reshape(1, -1), bits)[0].view("<u4")
    dy = (rng.standard_normal(512) * 3).astype(np.float32)
    dy[:3] = [-2.0, np.inf, -np.inf]
    mask[:3] = False
    packed = packbits_reference(mask.astype(np.int64).reshape(1, -1), bits)[0].view("<u4")
    dx = oracle.relu_unpack(packed, dy, bits)
    with np.errstate(invalid="ignore"):
        want = _bf16((dy * mask.astype(np.float32)).astype(np.float32))  # -2*0 = -0.0, inf*0 = NaN
    np.testing.assert_array_equal(dx[3:], want[3:])
    assert dx[0] == 0x8000 and np.isnan(_f32(dx[1:3])).all()


def _torch_act_and_grad(x, act):
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    y = torch.nn.functional.gelu(xt, approximate="tanh") if act == oracle.ACT_GELU else torch.nn.functional.silu(xt)
    (g,) = torch.autograd.grad(y.sum(), xt)
    return y.detach().numpy(), g.numpy()


@pytest.mark.parametrize("act", [oracle.ACT_GELU, oracle.ACT_SILU])
def test_act_forward_matches_torch_float64(act):
    rng = np.random.default_rng(80 + act)
    x = np.concatenate([rng.standard_normal(4000) * 3, [0.0, -0.0, 10.0, -10.0, 30.0, -30.0]]).astype(np.float32)
    y, d = oracle.act_forward(x, act)
    ty, td = _torch_act_and_grad(x.astype(np.float64), act)
    # fp32 evaluation then one bf16 rounding: within one bf16 ulp of the float64 value
    for got, want in ((_f32(y), ty), (_f32(d), td)):
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= np.abs(want) * 2 ** -8 + 1e-6), float(err.max())


@pytest.mark.parametrize("act", [oracle.ACT_GELU, oracle.ACT_SILU])
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_act_quant_pack_is_the_quantizer_of_the_squashed_derivative(act, bits):
    rng = np.random.default_rng(90 + bits + 10 * act)
    g = 128
    x = (rng.standard_normal((40, g)) * 2).astype(np.float32)
    y, packed, scale, mn = oracle.act_quant_pack(x, act, g, bits, meta_dtype=oracle.F32)
    y0, _ = oracle.act_forward(x, act)
    np.testing.assert_array_equal(y, y0)  # the activation output is the unfused one
    # the squashed derivative, float64: dequantized codes must lie within step/2 (+fp32 slack) of it
    _, td = _torch_act_and_grad(x.astype(np.float64), act)
    sq = np.tanh(np.clip(td, -3, 3) / 0.5) * 0.5
    deq = oracle.dequant_unpack(packed, scale, mn, g, bits)
    assert np.all(np.abs(deq - sq) <= scale[:, None] * 0.5 + 1e-5)
    # the range floor: max(mx - mn, 1e-4) / QMAX
    assert np.all(scale >= np.float32(1e-4) / np.float32((1 << bits) - 1))


def test_act_quant_pack_range_floor_known_answer():
    # a constant group has mx == mn: the range is floored at 1e-4, so step = 1e-4/QMAX and every code is 0
    x = np.full((2, 64), 0.7, dtype=np.float32)
    for act in (oracle.ACT_GELU, oracle.ACT_SILU):
        _, packed, scale, mn = oracle.act_quant_pack(x, act, 64, 2, meta_dtype=oracle.F32)
        assert np.all(packed == 0)
        assert np.all(scale == np.float32(np.float32(1e-4) / np.float32(3)))


@pytest.mark.parametrize("bits", [2, 8])
def test_act_dequant_mul_closed_form(bits):
    rng = np.random.default_rng(100 + bits)
    g, ng = 256, 24
    q = rng.integers(0, 1 << bits, size=(ng, g))
    packed = packbits_reference(q, bits).view("<u4").reshape(ng, -1)
    sc = _bf16(rng.random(ng) * 0.1)
    mn = _bf16(rng.standard_normal(ng) * 0.2)
    dy = _bf16(rng.standard_normal((ng, g)))
    dx = oracle.act_dequant_mul(packed, sc, mn, g, bits, dy)
    act = fma32(q.astype(np.float32), np.broadcast_to(_f32(sc)[:, None], q.shape), np.broadcast_to(_f32(mn)[:, None], q.shape))
    np.testing.assert_array_equal(dx, _bf16((_f32(dy) * act).astype(np.float32)))


# ----------------------------------------------------------------------------- clamp + tanh squash
@pytest.mark.parametrize("alpha", [3.0, 0.3])
@pytest.mark.parametrize("bits", [2, 8])
def test_clamp_squash_equals_float64(bits, alpha):
    x = squash_inputs(bits + int(alpha * 10))
    got = oracle.quant_pack(x, 256, bits, flags=oracle.FLAG_CLAMP | oracle.FLAG_SQUASH, clamp_alpha=alpha)
    assert squash_mismatch(got, x, bits, alpha) == []


@pytest.mark.parametrize("plant", [{"form": "2tanh(x/2)"}, {"clamp_first": False}])
def test_clamp_squash_check_catches_planted_mistakes(plant):
    """The comparison above must reject a restatement with BatchNorm's squash 2 tanh(x/2) in place of
    tanh(2x)/2, and one that clamps after squashing (which clamps nothing at alpha = 3 but lets
    values beyond alpha move the group's extremes)."""
    x = squash_inputs(5)
    alpha = 3.0
    got = oracle.quant_pack(x, 256, 2, flags=oracle.FLAG_CLAMP | oracle.FLAG_SQUASH, clamp_alpha=alpha)
    assert squash_mismatch(got, x, 2, alpha, **plant) != []


def test_clamp_alone_is_bit_exact_against_numpy():
    x = squash_inputs(6)
    for bits in (1, 4):
        got = oracle.quant_pack(x, 256, bits, flags=oracle.FLAG_CLAMP, clamp_alpha=0.75)
        want = numpy_quant(np.clip(x, np.float32(-0.75), np.float32(0.75)), bits)
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b)


def test_noise_near_one_is_clamped_to_qmax():
    """u = 1 - 2^-24 (torch.rand's largest value) on a group's maximum: fma(t, inv, u) rounds up to
    QMAX + 1 and rint(QMAX + 1/2) is QMAX + 1, so only the clamp keeps the code in range."""
    rng = np.random.default_rng(8)
    for bits in (1, 2, 4, 8):
        qmax = (1 << bits) - 1
        x = rng.standard_normal((64, 128)).astype(np.float32)
        u = rng.random((64, 128), dtype=np.float32)
        imax = x.argmax(axis=1)
        u[np.arange(64), imax] = np.float32(1 - 2 ** -24)
        p, s, m = oracle.quant_pack(x, 128, bits, rounding=NOISE, noise=u)
        codes = oracle.unpack_codes(p, 128, bits).view(np.uint8 if bits == 8 else np.int8).astype(np.int64)
        assert (codes[np.arange(64), imax] == qmax).all()
        # the case is real: before the clamp a good share of these maxima round to QMAX + 1
        inv = (np.float32(1) / s).astype(np.float32)
        t = (x[np.arange(64), imax] - m).astype(np.float32)
        pre = np.rint((fma32(t, inv, u[np.arange(64), imax]) - np.float32(0.5)).astype(np.float32))
        assert (pre == qmax + 1).mean() > 0.3
        np.testing.assert_array_equal(p, numpy_quant(x, bits, NOISE, u)[0])


# ----------------------------------------------------------------------------- ALAM averaging
SQ_CL = oracle.FLAG_SQUASH | oracle.FLAG_CLAMP


def _bf16_to_f32(bits_u16):
    return (np.asarray(bits_u16, dtype=np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_alam_one_equals_the_quantizer(bits):
    """alam_bits = 1 averages runs of one value: the plain quantizer with bf16 meta."""
    x = np.random.default_rng(bits).standard_normal((6, 256)).astype(np.float32)
    p, s, m = oracle.alam_quant_pack(x, 256, bits, 1, flags=SQ_CL, clamp_alpha=3.0)
    rp, rs, rm = oracle.quant_pack(x, 256, bits, flags=SQ_CL, clamp_alpha=3.0, meta_dtype=BF16)
    np.testing.assert_array_equal(p, rp)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(m, rm)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_alam_two_on_pairs_of_equal_values(bits):
    """With every run of 2 holding one value twice, the run's mean is that value's code argument
    exactly (qf + qf and the halving are exact), so the ALAM codes are the plain codes of the
    even elements."""
    base = np.random.default_rng(10 + bits).standard_normal((5, 128)).astype(np.float32)
    x = np.repeat(base, 2, axis=1)  # [5, 256], x[2c] == x[2c + 1]
    p, s, m = oracle.alam_quant_pack(x, 256, bits, 2, flags=oracle.FLAG_SQUASH)
    rp, rs, rm = oracle.quant_pack(x, 256, bits, flags=oracle.FLAG_SQUASH, meta_dtype=BF16)
    codes = oracle.unpack_codes(p, 128, bits).view(np.uint8)
    plain = oracle.unpack_codes(rp, 256, bits).view(np.uint8)
    np.testing.assert_array_equal(codes, plain[:, 0::2])
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(m, rm)


@pytest.mark.parametrize("bits,alam", [(2, 2), (2, 4), (4, 4), (8, 8), (1, 8)])
def test_alam_codes_are_the_truncated_run_means(bits, alam):
    """Each code is trunc(mean of the run's nearest-code arguments), with the arguments taken from
    the plain quantizer's own step and min (pinned above) and the mean in float64: equal except
    where summation order decides a boundary, and never off by more than one."""
    rng = np.random.default_rng(bits * 31 + alam)
    x = rng.standard_normal((8, 512)).astype(np.float32)
    p, s, m = oracle.alam_quant_pack(x, 512, bits, alam, flags=oracle.FLAG_SQUASH)
    # squashed values and the plain quantizer's fp32 step / min for the same groups
    xs = np.tanh(x.astype(np.float64) / 0.5) * 0.5
    _, s32, m32 = oracle.quant_pack(x, 512, bits, flags=oracle.FLAG_SQUASH, meta_dtype=F32)
    np.testing.assert_array_equal(_bf16_to_f32(s), _bf16_to_f32(oracle.quant_pack(
        x, 512, bits, flags=oracle.FLAG_SQUASH, meta_dtype=BF16)[1]))
    qf = (xs - m32[:, None].astype(np.float64)) / s32[:, None].astype(np.float64) + (0.5 - 1e-6)
    want = np.clip(np.floor(qf.reshape(8, 512 // alam, alam).mean(axis=2)), 0, (1 << bits) - 1)
    got = oracle.unpack_codes(p, 512 // alam, bits).view(np.uint8).astype(np.float64)
    assert np.max(np.abs(got - want)) <= 1
    assert np.mean(got != want) < 0.002


def test_alam_rejects_shapes_the_reference_cannot_reshape():
    x = np.zeros((1, 64), np.float32)
    with pytest.raises(oracle.OracleError):
        oracle.alam_quant_pack(x, 64, 2, 8)  # 4 words of codes: 8 does not divide them
    with pytest.raises(oracle.OracleError):
        oracle.alam_quant_pack(x, 64, 2, 3)  # not a power of two


def test_triton_randn_box_muller_from_the_philox_words():
    """Triton's randn: the first two Philox words (pinned by the known-answer vectors) -> uniforms
    (int32 folded to non-negative, times fp32(4.6566127342e-10)) -> Box-Muller's first output.
    Checked against float64 from the same words, to fp32 rounding of log / cos / sqrt."""
    for seed, off in [(42, 0), (42, 1), (43, 7), (42 + 100000, 255), (2**33 + 5, 1023)]:
        ctr = np.array([off, 0, 0, 0], np.uint32)
        key = np.array([seed & 0xFFFFFFFF, seed >> 32], np.uint32)
        out = np.zeros(4, np.uint32)
        oracle.lib().oracle_philox4x32_10(ctr.ctypes.data, key.ctypes.data, out.ctypes.data)

        def uni(w):
            i = int(np.array(w, np.uint32).view(np.int32))
            i = ~i if i < 0 else i
            return float(np.float32(i) * np.float32(4.6566127342e-10))
        u1, u2 = max(uni(out[0]), float(np.float32(1e-7))), uni(out[1])
        want = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        got = oracle.triton_randn(seed, off)
        assert abs(got - want) <= 8e-6 * max(1.0, abs(want)), (seed, off, got, want)


def test_triton_randn_is_standard_normal():
    vals = np.array([oracle.triton_randn(42 + r, e) for r in range(64) for e in range(512)])
    assert abs(vals.mean()) < 0.01
    assert abs(vals.std() - 1.0) < 0.01
    # two-sided tail frequencies of a standard normal
    assert abs(np.mean(np.abs(vals) > 1.0) - 0.3173) < 0.01
    assert abs(np.mean(np.abs(vals) > 2.0) - 0.0455) < 0.005


@pytest.mark.parametrize("bits,alam", [(2, 2), (4, 4), (8, 2)])
def test_alam_dequant_is_code_plus_centred_noise(bits, alam):
    """y = bf16(fma(code + n - 0.5, scale, min)) with n the noise above: given the codes, the
    residual (y - min) / scale - code has the noise's distribution shifted by -0.5, and element e
    of group r carries randn(42 + r, e)."""
    x = np.random.default_rng(7).standard_normal((64, 256)).astype(np.float32)
    p, s, m = oracle.alam_quant_pack(x, 256, bits, alam, flags=oracle.FLAG_SQUASH)
    y = _bf16_to_f32(oracle.alam_dequant_unpack(p, s, m, 256, bits, alam)).astype(np.float64)
    sc, mn = _bf16_to_f32(s).astype(np.float64), _bf16_to_f32(m).astype(np.float64)
    codes = np.repeat(oracle.unpack_codes(p, 256 // alam, bits).view(np.uint8).astype(np.float64), alam, axis=1)
    resid = (y - mn[:, None]) / sc[:, None] - codes
    assert abs(resid.mean() + 0.5) < 0.03
    assert abs(resid.std() - 1.0) < 0.03
    for r, e in [(0, 0), (3, 17), (63, 255)]:
        n = oracle.triton_randn(42 + r, e)
        want = (codes[r, e] + (n - 0.5)) * sc[r] + mn[r]
        assert abs(y[r, e] - want) <= 2 ** -7 * abs(want) + 1e-30


def _tl_rand(seed, off):
    """tl.rand(seed, off) from the Philox words (pinned by the known-answer vectors above)"""
    ctr = np.array([off, 0, 0, 0], np.uint32)
    key = np.array([seed & 0xFFFFFFFF, seed >> 32], np.uint32)
    out = np.zeros(4, np.uint32)
    oracle.lib().oracle_philox4x32_10(ctr.ctypes.data, key.ctypes.data, out.ctypes.data)
    i = int(out[:1].view(np.int32)[0])
    i = ~i if i < 0 else i
    return np.float32(i) * np.float32(4.6566127342e-10)


def test_silu_alam_backward_adds_the_rand_noise():
    """The SiLU backward with avg_alam at alam_bits = 1: dx = bf16(dy * fma(q + (u - 1/2), scale,
    min)) with u = tl.rand(42 + group, element), against float64 from the Philox words (one bf16
    ulp: the float64 form rounds twice); without the seed it is the plain dx."""
    g, bits, ng = 64, 2, 8
    x = np.random.default_rng(3).standard_normal((ng, g)).astype(np.float32)
    p, s, m = oracle.quant_pack(x, g, bits, meta_dtype=oracle.BF16)
    dy = np.random.default_rng(4).standard_normal((ng, g)).astype(np.float32)
    got = _bf16_to_f32(oracle.act_dequant_mul(p, s, m, g, bits, dy, alam_seed=42)).astype(np.float64)
    codes = oracle.unpack_codes(p, g, bits).view(np.uint8).astype(np.float32).reshape(ng, g)
    sc, mn = _bf16_to_f32(s).astype(np.float64), _bf16_to_f32(m).astype(np.float64)
    u = np.array([[_tl_rand(42 + r, e) for e in range(g)] for r in range(ng)], dtype=np.float32)
    qn = (codes + (u - np.float32(0.5))).astype(np.float64)
    want = dy.astype(np.float64) * (qn * sc[:, None] + mn[:, None])
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)
    plain = _bf16_to_f32(oracle.act_dequant_mul(p, s, m, g, bits, dy)).astype(np.float64)
    np.testing.assert_allclose(plain, dy * (codes * sc[:, None] + mn[:, None]), rtol=2.0 ** -7, atol=1e-30)
    assert np.mean(got != plain) > 0.5


# ----------------------------------------------------------------------------- PACT clamp
def _torch_bf16_bits(a):
    """torch's own fp32 -> bf16 rounding (RNE), as uint16 bit patterns"""
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("alpha", [3.0, 0.5, 1e-3, float("inf")])
def test_pact_clamp_forward_closed_form(dtype, alpha):
    """y = torch's bf16 of numpy clip(x, -alpha, alpha) and mask = |x| <= alpha, element for element;
    inputs at exactly +-alpha, +-0, past alpha and large; a NaN x gives -alpha and mask 0 (fmax then
    fmin)."""
    rng = np.random.default_rng(int(alpha * 1000) if np.isfinite(alpha) else 99)
    vals = np.concatenate([rng.standard_normal(4096) * 4, [alpha, -alpha, 0.0, -0.0, 1e30, -1e30]])
    vals = vals[np.isfinite(vals)].astype(np.float32)
    if dtype == "bf16":
        x = _torch_bf16_bits(vals)
        xf = oracle.bf16_bits_to_f32(x)
    elif dtype == "f16":
        x = vals.astype(np.float16)
        xf = x.astype(np.float32)
    else:
        x = vals
        xf = x
    y, mask = oracle.pact_clamp_fwd(x, alpha)
    np.testing.assert_array_equal(y, _torch_bf16_bits(np.clip(xf, np.float32(-alpha), np.float32(alpha))))
    np.testing.assert_array_equal(mask, (np.abs(xf) <= np.float32(alpha)).astype(np.int8))
    if np.isfinite(alpha):
        assert mask[np.abs(xf) == np.float32(alpha)].all()  # the boundary is inside (<=, not <)
    yn, mn = oracle.pact_clamp_fwd(np.array([np.nan], dtype=np.float32), alpha)
    assert yn[0] == _torch_bf16_bits(np.array([-alpha]))[0] and mn[0] == 0  # bf16(-alpha)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_pact_clamp_backward_closed_form(dtype):
    """dx = torch's bf16 of where(mask != 0, dy, +0): any non-zero mask byte passes dy."""
    rng = np.random.default_rng(5)
    dyf = (rng.standard_normal(1031) * 3).astype(np.float32)
    mask = rng.integers(-3, 3, size=1031).astype(np.int8)
    if dtype == "bf16":
        dy = _torch_bf16_bits(dyf)
        dyv = oracle.bf16_bits_to_f32(dy)
    elif dtype == "f16":
        dy = dyf.astype(np.float16)
        dyv = dy.astype(np.float32)
    else:
        dy, dyv = dyf, dyf
    got = oracle.pact_clamp_bwd(mask, dy)
    np.testing.assert_array_equal(got, _torch_bf16_bits(np.where(mask != 0, dyv, np.float32(0.0))))
    assert not (got[mask == 0] & 0x8000).any()  # +0, never -0, where the mask is clear


def test_pact_clamp_rejects_non_positive_or_nan_alpha():
    for bad in (-1.0, 0.0, float("nan")):
        with pytest.raises(oracle.OracleError):
            oracle.pact_clamp_fwd(np.zeros(4, dtype=np.float32), bad)
