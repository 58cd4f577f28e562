"""GPU parity: the gfx950 kernels (through act_lib -> C ABI) against the CPU oracle.

Bar: bit-exact packed words, scale, min and dequantized values for nearest rounding and for
stochastic rounding with a given noise tensor or the Philox stream (the oracle implements the
same generator). The tanh squash of the reference's pre-transform is the one tolerance: the
kernel evaluates tanh(2x)/2 with its own polynomial / exp form and the oracle with the C
library's tanhf, so both are compared with float64 (min within 2 fp32 ulps, scale within what
that gives, codes equal away from rounding boundaries). Small ragged sizes sweep every (dtype,
bits, group size, rounding) kernel; the full ResNet activation (bf16 [256,256,56,56]) is checked
bit-exact against the oracle and through size-independent bounds.
"""
import numpy as np
import pytest
import torch

import deep_optimization_amd  # noqa: F401
import oracle
from deep_optimization_amd import _lib
from tests.golden import make_golden
from tests.restate import squash_inputs, squash_mismatch

pytestmark = pytest.mark.gpu
DEV = "cuda"

TORCH_TO_ORACLE = {torch.float32: oracle.F32, torch.float16: oracle.F16, torch.bfloat16: oracle.BF16}
ROUNDINGS = {"nearest": oracle.NEAREST, "noise": oracle.STOCH_NOISE, "philox": oracle.STOCH_PHILOX}


def np_view(t: torch.Tensor) -> np.ndarray:
    """CPU numpy view with the oracle's storage convention (bf16 as uint16 bit patterns)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.int32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def make_input(shape, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=gen)
    # vary the dynamic range across the leading rows so steps differ per group
    scale = torch.exp(torch.randn(shape[:-1] + (1,), generator=gen) * 2)
    return (x * scale).to(dtype)


def gpu_quant(x, bits, g, rounding, noise=None, seed=0, offset=0, scale_dtype=torch.float32, clamp=False,
              alpha=0.0, squash=False, tile=False):
    op = torch.ops.act_lib.quant_pack_tiles if tile else torch.ops.act_lib.quant_pack
    out = op(x.to(DEV), bits, g, clamp, alpha, squash, ROUNDINGS[rounding], None if noise is None else noise.to(DEV),
             seed, offset, scale_dtype)
    torch.cuda.synchronize()
    return out


def oracle_quant(x, bits, g, rounding, noise=None, seed=0, offset=0, meta=oracle.F32, flags=0, alpha=0.0,
                 tile=None):
    xn = np_view(x)
    return oracle.quant_pack(xn if tile else xn.reshape(-1, g), g, bits, tile_nchw=tile, rounding=ROUNDINGS[rounding],
                             noise=None if noise is None else noise.numpy(), seed=seed, offset=offset, flags=flags,
                             clamp_alpha=alpha, meta_dtype=meta)


def assert_quant_equal(gpu, ref, what=""):
    p, s, m = gpu
    rp, rs, rm = ref
    np.testing.assert_array_equal(np_view(p).reshape(rp.shape), rp, err_msg=f"packed {what}")
    np.testing.assert_array_equal(np_view(s).reshape(-1), rs, err_msg=f"scale {what}")
    np.testing.assert_array_equal(np_view(m).reshape(-1), rm, err_msg=f"min {what}")


# ----------------------------------------------------------------------------- flat quant-pack sweep
@pytest.mark.parametrize("rounding", ["nearest", "noise", "philox"])
@pytest.mark.parametrize("g", [64, 128, 256, 512, 1024])
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
def test_quant_pack_flat_parity(dtype, bits, g, rounding):
    NG = 1 + 67 * (1024 // g)  # ragged: not a multiple of any groups-per-wave count
    x = make_input((1, NG, g), dtype, seed=bits * 100 + g)
    noise = torch.rand((1, NG, g), generator=torch.Generator().manual_seed(7)) if rounding == "noise" else None
    gpu = gpu_quant(x, bits, g, rounding, noise, seed=77, offset=5)
    ref = oracle_quant(x, bits, g, rounding, noise, seed=77, offset=5)
    assert_quant_equal(gpu, ref, f"{dtype} b{bits} g{g} {rounding}")


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("g", [64, 128, 256, 512, 1024])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("meta", [torch.float32, torch.bfloat16], ids=["meta32", "meta16"])
def test_dequant_flat_parity(bits, g, out_dtype, meta):
    NG = 3 + 41 * (1024 // g)
    x = make_input((1, NG, g), torch.bfloat16, seed=bits + g)
    mo = oracle.F32 if meta == torch.float32 else oracle.BF16
    rp, rs, rm = oracle_quant(x, bits, g, "nearest", meta=mo)
    yo = oracle.dequant_unpack(rp, rs, rm, g, bits, y_dtype=TORCH_TO_ORACLE[out_dtype])
    p = torch.from_numpy(rp.view(np.int32)).to(DEV)
    if meta == torch.bfloat16:
        s = torch.from_numpy(rs.view(np.int16)).view(torch.bfloat16).to(DEV).view(1, NG)
        m = torch.from_numpy(rm.view(np.int16)).view(torch.bfloat16).to(DEV).view(1, NG)
    else:
        s = torch.from_numpy(rs).to(DEV).view(1, NG)
        m = torch.from_numpy(rm).to(DEV).view(1, NG)
    y = torch.ops.act_lib.dequant_unpack(p, s, m, bits, g, out_dtype)
    np.testing.assert_array_equal(np_view(y).reshape(yo.shape), yo)


# ----------------------------------------------------------------------------- tile layout
TILE_CASES = [((2, 3, 32, 48), 256), ((1, 4, 16, 40), 64), ((1, 2, 64, 32), 1024), ((3, 5, 8, 8), 64),
              ((2, 2, 48, 16), 256)]


@pytest.mark.parametrize("shape,g", TILE_CASES)
@pytest.mark.parametrize("rounding", ["nearest", "noise", "philox"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_quant_pack_tiles_parity(shape, g, rounding, dtype):
    bits = 2 if g == 256 else 4
    x = make_input(shape, dtype, seed=sum(shape) + g)
    n_groups = shape[0] * shape[1] * (shape[2] * shape[3] // g)
    noise = torch.rand(n_groups * g, generator=torch.Generator().manual_seed(3)) if rounding == "noise" else None
    gpu = gpu_quant(x, bits, g, rounding, noise, seed=3, offset=11, tile=True)
    ref = oracle_quant(x, bits, g, rounding, noise, seed=3, offset=11, tile=shape)
    assert_quant_equal(gpu, ref, f"tiles {shape} g{g}")
    y = torch.ops.act_lib.dequant_unpack_tiles(*gpu, bits, g, *shape, torch.bfloat16)
    yo = oracle.dequant_unpack(*ref, g, bits, tile_nchw=shape, y_dtype=oracle.BF16)
    np.testing.assert_array_equal(np_view(y), yo)


# ----------------------------------------------------------------------------- committed fixtures
@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_golden_fixtures(name):
    case = make_golden.load_all()[name]
    _, kw = make_golden.CASES[name]
    g, bits = kw["group_size"], kw["bits"]
    tile = kw.get("tile")
    if name == "c1_cpu_config":
        x = torch.from_numpy(make_golden.c1_input())
    elif case["x"].dtype == np.uint16:
        x = torch.from_numpy(case["x"].view(np.int16)).view(torch.bfloat16)
    else:
        x = torch.from_numpy(case["x"])
    noise = torch.from_numpy(case["noise"]) if "noise" in case else None
    rounding = {oracle.NEAREST: "nearest", oracle.STOCH_NOISE: "noise", oracle.STOCH_PHILOX: "philox"}[kw["rounding"]]
    meta = torch.float32 if kw["meta_dtype"] == oracle.F32 else torch.bfloat16
    flags = kw.get("flags", 0)
    xin = x if tile else x.reshape(1, -1, g)
    gpu = gpu_quant(xin, bits, g, rounding, noise, seed=kw.get("seed", 0), offset=kw.get("offset", 0),
                    scale_dtype=meta, clamp=bool(flags & 1), alpha=kw.get("clamp_alpha", 0.0),
                    squash=bool(flags & 2), tile=tile is not None)
    if flags & 2:
        # tanh squash: the kernel's tanh(2x)/2 and the C library's tanhf differ by up to a few ulps
        codes_gpu = oracle.unpack_codes(np_view(gpu[0]), g, bits).astype(int)
        codes_ref = oracle.unpack_codes(case["packed"], g, bits).astype(int)
        assert np.max(np.abs(codes_gpu - codes_ref)) <= 1 and np.mean(codes_gpu != codes_ref) < 1e-3
        return
    np.testing.assert_array_equal(np_view(gpu[0]).reshape(case["packed"].shape), case["packed"])
    np.testing.assert_array_equal(np_view(gpu[1]).reshape(-1), case["scale"])
    np.testing.assert_array_equal(np_view(gpu[2]).reshape(-1), case["min"])
    out_dtype = torch.float32 if kw["y_dtype"] == oracle.F32 else torch.bfloat16
    if tile:
        y = torch.ops.act_lib.dequant_unpack_tiles(*gpu, bits, g, *tile, out_dtype)
    else:
        y = torch.ops.act_lib.dequant_unpack(*gpu, bits, g, out_dtype)
    want = case["y"] if "y" in case else oracle.dequant_unpack(case["packed"], case["scale"], case["min"], g, bits,
                                                                 tile_nchw=tile, y_dtype=kw["y_dtype"])
    np.testing.assert_array_equal(np_view(y).reshape(want.shape), want)


# ----------------------------------------------------------------------------- code-only pack
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("g", [64, 256, 1024])
def test_pack_unpack_codes_parity(bits, g):
    gen = torch.Generator().manual_seed(bits + g)
    codes = torch.randint(-128, 128, (3, 37, g), generator=gen, dtype=torch.int8)
    if bits == 1:
        codes = (codes > 0).to(torch.int8)  # the masks the reference packs
    w = torch.ops.act_lib.pack_triton(codes.to(DEV), bits, g)
    want = oracle.pack_codes(codes.numpy().reshape(-1, g), g, bits)
    np.testing.assert_array_equal(np_view(w), want)
    back = torch.ops.act_lib.unpack_triton(w, bits, 3, 37, g)
    np.testing.assert_array_equal(back.cpu().numpy().reshape(-1, g), oracle.unpack_codes(want, g, bits))


# ----------------------------------------------------------------------------- reference-schema ops
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_reference_schema_ops(bits):
    g = 256
    x = make_input((4, 50, g), torch.bfloat16, seed=bits)
    p, s, m = torch.ops.act_lib.quant_pack_triton(x.to(DEV), bits, g, False, 0, True, 3.0)
    assert s.dtype == torch.bfloat16 and s.shape == (4, 50) and p.shape == (200, g * bits // 32)
    rp, rs, rm = oracle_quant(x, bits, g, "nearest", meta=oracle.BF16, flags=3, alpha=3.0)
    # squash (tanh) is tolerance-only: scale/min within 1 bf16 ulp, codes within 1 and rarely off
    rs32 = oracle.bf16_bits_to_f32(rs)
    np.testing.assert_allclose(s.float().cpu().numpy().reshape(-1), rs32, rtol=2 ** -7, atol=0)
    np.testing.assert_allclose(m.float().cpu().numpy().reshape(-1), oracle.bf16_bits_to_f32(rm), rtol=2 ** -7,
                               atol=1e-30)
    cg = oracle.unpack_codes(np_view(p), g, bits).astype(int)
    cr = oracle.unpack_codes(rp, g, bits).astype(int)
    assert np.max(np.abs(cg - cr)) <= 1 and np.mean(cg != cr) < 1e-3
    # dequant of the GPU's own packed data is bit-exact against the oracle
    y = torch.ops.act_lib.dequant_unpack_triton(p, s, m, bits, g, False, 0)
    assert y.dtype == torch.bfloat16 and y.shape == (4, 50, g)
    yo = oracle.dequant_unpack(np_view(p), np_view(s).reshape(-1), np_view(m).reshape(-1), g, bits,
                               y_dtype=oracle.BF16)
    np.testing.assert_array_equal(np_view(y).reshape(yo.shape), yo)


# ----------------------------------------------------------------------------- ALAM averaging
def _codes(packed, bits):
    """Little-endian b-bit fields of uint32 words -> [rows, words * 32 / b] (any code count)."""
    w = np.ascontiguousarray(packed).view(np.uint32).reshape(packed.shape[0], -1).astype(np.uint64)
    sh = np.arange(32 // bits, dtype=np.uint64) * np.uint64(bits)
    return ((w[:, :, None] >> sh) & np.uint64((1 << bits) - 1)).reshape(w.shape[0], -1).astype(np.int64)


def _alam_gpu_raw(x, bits, g, alam, flags=0, alpha=0.0):
    """dopt_alam_quant_pack through the C ABI on a [NG, g] tensor -> (packed, scale, min) on the CPU."""
    L = _lib.lib()
    xd = x.to(DEV).contiguous()
    ng = xd.numel() // g
    p = torch.empty((ng, g * bits // 32 // alam), dtype=torch.int32, device=DEV)
    s = torch.empty(ng, dtype=torch.bfloat16, device=DEV)
    m = torch.empty(ng, dtype=torch.bfloat16, device=DEV)
    code = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}[xd.dtype]
    rc = L.dopt_alam_quant_pack(xd.data_ptr(), code, ng, g, bits, alam, flags, alpha, p.data_ptr(), s.data_ptr(),
                                m.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, L.dopt_last_error()
    torch.cuda.synchronize()
    return np_view(p), np_view(s), np_view(m)


# alam_bits must divide the group's words (1 bit at g = 64 has 2 words, so no runs of 8: rejected,
# test_alam_rejects_bad_run_lengths)
ALAM_CASES = [(g, bits, alam) for g in (64, 256, 1024)
              for bits, alam in [(1, 1), (1, 8), (2, 2), (2, 4), (4, 4), (8, 2), (8, 8)] if (g * bits // 32) % alam == 0]


@pytest.mark.parametrize("g,bits,alam", ALAM_CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16], ids=["bf16", "f32", "f16"])
def test_alam_quant_pack_bit_exact_without_squash(dtype, g, bits, alam):
    """Without the squash (a C-ABI option; the operator always squashes) the codes, scale and min
    are bit-exact against the oracle: min/max, step, the fma code arguments, the left-to-right
    run sums and the truncation."""
    x = make_input((3, 37, g), dtype, seed=bits * 7 + alam)
    p, s, m = _alam_gpu_raw(x, bits, g, alam)
    rp, rs, rm = oracle.alam_quant_pack(np_view(x).reshape(-1, g), g, bits, alam)
    np.testing.assert_array_equal(p.view(np.uint32).reshape(rp.shape), rp)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(m, rm)
    # the clamp alone (NaN and +-inf included) is exact as well
    x.view(-1)[:3] = torch.tensor([float("nan"), float("inf"), -float("inf")]).to(dtype)
    p, s, m = _alam_gpu_raw(x, bits, g, alam, flags=oracle.FLAG_CLAMP, alpha=2.5)
    rp, rs, rm = oracle.alam_quant_pack(np_view(x).reshape(-1, g), g, bits, alam, flags=oracle.FLAG_CLAMP,
                                        clamp_alpha=2.5)
    np.testing.assert_array_equal(p.view(np.uint32).reshape(rp.shape), rp)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(m, rm)


@pytest.mark.parametrize("bits,alam", [(2, 2), (4, 4), (8, 8), (1, 8)])
def test_alam_reference_operators(bits, alam):
    """quant_pack_triton / dequant_unpack_triton with avg_alam=True (the reference's clamp 3 +
    squash): packed [NG, NW / alam_bits], scale/min within 1 bf16 ulp of the oracle (the squash is
    tolerance-only) and codes within one; the dequant of the GPU's own codes equals the oracle's
    within one bf16 ulp (the noise's log / cos differ by fp32 ulps between the libraries), with
    the element-to-noise mapping of Triton's randn(42 + group, element)."""
    g = 256
    x = make_input((4, 50, g), torch.bfloat16, seed=bits + alam)
    p, s, m = torch.ops.act_lib.quant_pack_triton(x.to(DEV), bits, g, True, alam, True, 3.0)
    assert p.shape == (200, g * bits // 32 // alam) and s.shape == (4, 50) and s.dtype == torch.bfloat16
    rp, rs, rm = oracle.alam_quant_pack(np_view(x).reshape(-1, g), g, bits, alam, flags=3, clamp_alpha=3.0)
    np.testing.assert_allclose(s.float().cpu().numpy().reshape(-1), oracle.bf16_bits_to_f32(rs), rtol=2 ** -7)
    np.testing.assert_allclose(m.float().cpu().numpy().reshape(-1), oracle.bf16_bits_to_f32(rm), rtol=2 ** -7,
                               atol=1e-30)
    cg, cr = _codes(np_view(p), bits), _codes(rp, bits)
    assert np.max(np.abs(cg - cr)) <= 1 and np.mean(cg != cr) < 2e-3
    y = torch.ops.act_lib.dequant_unpack_triton(p, s, m, bits, g, True, alam)
    torch.cuda.synchronize()
    assert y.shape == (4, 50, g) and y.dtype == torch.bfloat16
    yo = oracle.alam_dequant_unpack(np_view(p), np_view(s).reshape(-1), np_view(m).reshape(-1), g, bits, alam)
    yg = np_view(y).reshape(yo.shape).astype(np.int64)
    diff = np.abs(yg - yo.astype(np.int64))  # bf16 bit patterns: same sign, so ulp distance
    assert diff.max() <= 1 and np.mean(diff != 0) < 0.01


def test_alam_rejects_bad_run_lengths():
    x = torch.zeros(1, 1, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError):
        torch.ops.act_lib.quant_pack_triton(x, 2, 64, True, 8, False, 0.0)  # 4 words per group
    with pytest.raises(RuntimeError):
        torch.ops.act_lib.quant_pack_triton(x, 2, 64, True, 3, False, 0.0)


def test_mismatched_sizes_are_rejected_before_launch():
    """Inputs whose sizes disagree with the group geometry raise instead of reaching a kernel that
    would read past them: a last dim other than group_size (the reference's x.view(N*G, g)
    raises), packed words short of N*G groups' worth."""
    x = torch.randn((2, 4, 128), device=DEV).to(torch.bfloat16)
    with pytest.raises(RuntimeError):
        torch.ops.act_lib.quant_pack_triton(x, 2, 256, False, 0, True, 3.0)
    with pytest.raises(RuntimeError):
        torch.ops.act_lib.quant_pack(x, 2, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
    packed = torch.zeros((8, 4), dtype=torch.int32, device=DEV)  # 2-bit g=256 needs 16 words per group
    with pytest.raises(RuntimeError):
        torch.ops.act_lib.unpack_triton(packed, 2, 2, 4, 256)
    with pytest.raises(RuntimeError):
        torch.ops.act_lib.dequant_unpack_triton(packed, torch.ones((2, 4), dtype=torch.bfloat16, device=DEV),
                                                torch.zeros((2, 4), dtype=torch.bfloat16, device=DEV), 2, 256, False, 0)


def test_tensors_off_the_current_device_are_rejected(monkeypatch):
    """The C ABI launches on the current device; an operator implemented in Python raises for a
    tensor elsewhere (simulated by making the current-device query answer another index). The
    native operators (csrc/torch_ops.cpp) make the tensor's device current instead."""
    x = torch.randint(0, 4, (2, 4, 256), dtype=torch.int8, device=DEV)
    monkeypatch.setattr(torch.cuda, "current_device", lambda: x.get_device() + 1)
    with pytest.raises(RuntimeError, match="current device"):
        torch.ops.act_lib.pack_triton(x, 2, 256)


def test_bad_bits_raise_value_error_on_device():
    x = torch.zeros(1, 1, 256, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        torch.ops.act_lib.quant_pack_triton(x, 3, 256, False, 0, False, 0.0)


# ----------------------------------------------------------------------------- edge cases
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_special_values_bit_exact(bits):
    g = 256
    x = make_input((1, 9, g), torch.float32, seed=5)
    x[0, 0, 3] = float("inf")
    x[0, 1, 7] = float("-inf")
    x[0, 2, 11] = float("nan")
    x[0, 3, :] = -0.0
    x[0, 3, 5] = 0.0
    x[0, 4, :] = 1e-40  # subnormal group
    x[0, 4, 9] = 3e-40
    x[0, 5, :] = 7.0  # constant
    x[0, 6, :] = 3e38  # range overflows to inf
    x[0, 6, 1] = -3e38
    noise = torch.rand(x.shape, generator=torch.Generator().manual_seed(3))
    noise[0, :, :4] = torch.tensor([0.0, 1.0 - 2.0**-24, 0.5, 2.0**-24])
    for rounding in ("nearest", "philox", "noise"):
        nz = noise if rounding == "noise" else None
        gpu = gpu_quant(x, bits, g, rounding, noise=nz, seed=1, offset=2)
        ref = oracle_quant(x, bits, g, rounding, noise=nz, seed=1, offset=2)
        assert_quant_equal(gpu, ref, rounding)


@pytest.mark.parametrize("alpha", [3.0, 0.0, -1.0])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_special_values_clamped_bit_exact(alpha, dtype):
    """The clamp pre-transform (clamp(x, -alpha, alpha), then nearest codes) on NaN, +-inf,
    signed zeros, subnormals and values beyond alpha: bit-exact against the oracle's
    fminf(fmaxf(x, -alpha), alpha), which sends NaN to -alpha (the kernel's v_med3 path for
    alpha >= 0, its min/max path for a negative alpha)."""
    g = 256
    x = make_input((1, 8, g), torch.float32, seed=6) * 4
    x[0, 0, 3] = float("inf")
    x[0, 1, 7] = float("-inf")
    x[0, 2, 11] = float("nan")
    x[0, 2, 12] = float("nan")
    x[0, 3, :] = -0.0
    x[0, 3, 5] = 0.0
    x[0, 4, :] = 1e-40
    x[0, 4, 9] = -3e-40
    x[0, 5, :] = float("nan")  # a group of NaN only: every value becomes -alpha
    x = x.to(dtype)
    for bits in (2, 8):
        gpu = gpu_quant(x, bits, g, "nearest", clamp=True, alpha=alpha)
        ref = oracle_quant(x, bits, g, "nearest", flags=1, alpha=alpha)
        assert_quant_equal(gpu, ref, f"{bits}-bit alpha={alpha}")


# ----------------------------------------------------------------------------- squash accuracy
def quant_np(out):
    """(packed [NG, W] uint32, scale fp32 [NG], min fp32 [NG]) numpy arrays of a GPU result."""
    p, s, m = out
    return np_view(p).reshape(s.numel(), -1), np_view(s).reshape(-1), np_view(m).reshape(-1)


def test_squash_elementwise_within_two_ulps():
    """Every group's minimum is the squash of one chosen value v (its 63 other values are larger by
    at least 0.05), so the stored fp32 minimum reads back the kernel's tanh(2v)/2 for 188,416 values:
    uniform over [-2.5, 2.5], dense around |v| = 1/16 and around the kernel's branch point 0.45,
    and log-uniform down to 1e-30. Each must be within 2 fp32 ulps of float64 tanh(2v)/2."""
    rng = np.random.default_rng(12)
    v = np.concatenate([rng.uniform(-2.5, 2.5, 1 << 16), rng.uniform(-0.07, 0.07, 1 << 15),
                        rng.uniform(-0.5, -0.4, 1 << 14), rng.uniform(0.4, 0.5, 1 << 14),
                        -(10.0 ** rng.uniform(-30, -1, 1 << 14)), 10.0 ** rng.uniform(-30, -1, 1 << 14)])
    v = v.astype(np.float32)
    g = 64
    x = (v[:, None] + np.float32(0.05) + np.abs(rng.standard_normal((v.size, g)))).astype(np.float32)
    x[:, 0] = v
    _, _, mn = quant_np(gpu_quant(torch.from_numpy(x).view(1, -1, g), 2, g, "nearest", squash=True))
    want = (np.tanh(2.0 * v.astype(np.float64)) / 2.0).astype(np.float32)
    ulp = np.abs(np.nextafter(np.abs(want), np.float32(np.inf)) - np.abs(want)).astype(np.float64)
    err = np.abs(mn.astype(np.float64) - want.astype(np.float64)) / ulp
    print(f"squash max error {err.max():.3f} ulp at v={v[np.argmax(err)]!r}")
    assert err.max() <= 2.0


@pytest.mark.parametrize("alpha", [3.0, 0.3])
@pytest.mark.parametrize("bits", [2, 8])
def test_clamp_squash_against_float64(bits, alpha):
    """act_lib::quant_pack with clamp + squash and fp32 scale/min against the float64 restatement
    (numpy clip, then tanh(2x)/2, rounded once): groups inside |x| < 1/16, straddling it,
    straddling 0.45, N(0, 1) and beyond alpha."""
    x = squash_inputs(bits + int(alpha * 10))
    got = gpu_quant(torch.from_numpy(x).view(1, -1, 256), bits, 256, "nearest", clamp=True, alpha=alpha, squash=True)
    assert squash_mismatch(quant_np(got), x, bits, alpha) == []


@pytest.mark.parametrize("g", [64, 256, 1024])
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_noise_near_one_on_group_max(dtype, bits, g):
    """Noise u = 1 - 2^-24 (torch.rand's largest value) and 1 - 2^-23 on each group's maximum, and
    whole groups of u = 1 - 2^-24: fma(t, inv, u) rounds up to QMAX + 1 for many of these maxima,
    and only the reference's clamp keeps the code at QMAX. Bit-exact against the oracle."""
    NG = 97 * (1024 // g)
    x = make_input((1, NG, g), dtype, seed=bits * 7 + g)
    noise = torch.rand((NG, g), generator=torch.Generator().manual_seed(g + bits))
    imax = x.float().view(NG, g).argmax(dim=1)
    rows = torch.arange(NG)
    noise[rows, imax] = torch.where(rows % 2 == 0, torch.tensor(1 - 2 ** -24), torch.tensor(1 - 2 ** -23))
    noise[::7] = 1 - 2 ** -24
    noise = noise.view(1, NG, g)
    assert_quant_equal(gpu_quant(x, bits, g, "noise", noise), oracle_quant(x, bits, g, "noise", noise),
                       f"{dtype} b{bits} g{g}")
    # the clamp pre-transform is bit-exact too
    assert_quant_equal(gpu_quant(x, bits, g, "noise", noise, clamp=True, alpha=1.0),
                       oracle_quant(x, bits, g, "noise", noise, flags=1, alpha=1.0), f"clamped {dtype} b{bits} g{g}")


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("rounding", ["noise", "philox"])
def test_pretransform_with_stochastic_rounding(rounding, bits):
    """The reference's clamp / squash pre-transform combined with stochastic rounding (what a layer
    whose meta asks for 'stochastic' or 'stochastic_noise' runs): clamp alone bit-exact against
    the oracle; clamp + squash against the float64 restatement with the same noise."""
    g = 256
    x = (make_input((1, 130, g), torch.float32, seed=bits + 40) * 2).to(torch.bfloat16)
    noise = torch.rand((1, 130, g), generator=torch.Generator().manual_seed(bits)) if rounding == "noise" else None
    assert_quant_equal(gpu_quant(x, bits, g, rounding, noise, seed=9, offset=4, clamp=True, alpha=1.5),
                       oracle_quant(x, bits, g, rounding, noise, seed=9, offset=4, flags=1, alpha=1.5))
    got = gpu_quant(x, bits, g, rounding, noise, seed=9, offset=4, clamp=True, alpha=3.0, squash=True)
    u = noise.numpy().reshape(-1, g) if noise is not None else oracle.philox_noise(0, x.numel(), 9, 4).reshape(-1, g)
    assert squash_mismatch(quant_np(got), x.float().numpy().reshape(-1, g), bits, 3.0, u=u) == []


def test_empty_and_single_group():
    x = torch.zeros((0, 4, 256), dtype=torch.bfloat16, device=DEV)
    p, s, m = torch.ops.act_lib.quant_pack(x, 2, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
    assert p.shape == (0, 16) and s.shape == (0, 4)
    y = torch.ops.act_lib.dequant_unpack(p, s, m, 2, 256, torch.bfloat16)
    assert y.shape == (0, 4, 256)
    x1 = make_input((1, 1, 1024), torch.float32, seed=9)
    assert_quant_equal(gpu_quant(x1, 8, 1024, "nearest"), oracle_quant(x1, 8, 1024, "nearest"))


def test_misaligned_input_view():
    base = make_input((1, 40 * 256 + 3), torch.bfloat16, seed=2)
    x = base[:, 3:].reshape(1, 40, 256)  # storage offset of 6 bytes
    gpu = gpu_quant(x, 2, 256, "nearest")
    ref = oracle_quant(x.contiguous(), 2, 256, "nearest")
    assert_quant_equal(gpu, ref)


def test_stream_ordering_on_side_stream():
    x = make_input((2, 300, 256), torch.bfloat16, seed=4).to(DEV)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        p, sc, m = torch.ops.act_lib.quant_pack(x, 4, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
        y = torch.ops.act_lib.dequant_unpack(p, sc, m, 4, 256, torch.float32)
    s.synchronize()
    ref = oracle_quant(x.cpu(), 4, 256, "nearest")
    assert_quant_equal((p, sc, m), ref)
    yo = oracle.dequant_unpack(*ref, 256, 4)
    np.testing.assert_array_equal(y.cpu().numpy().reshape(yo.shape), yo)


# ----------------------------------------------------------------------------- full workload sizes
@pytest.fixture(scope="module")
def resnet_act():
    """The ResNet-50 conv2 activation: bf16 [256, 256, 56, 56] post-ReLU |N(0,1)|, g = 256, 2-bit."""
    gen = torch.Generator(device=DEV).manual_seed(0)
    x = torch.randn((256, 256, 56, 56), generator=gen, device=DEV, dtype=torch.float32).abs_().to(torch.bfloat16)
    return x


def test_resnet_full_size_nearest_bit_exact(resnet_act):
    g = 256
    x = resnet_act.view(256, -1, g)
    p, s, m = torch.ops.act_lib.quant_pack(x, 2, g, False, 0.0, False, 0, None, 0, 0, torch.float32)
    torch.cuda.synchronize()
    ref = oracle.quant_pack(np_view(x).reshape(-1, g), g, 2)
    assert_quant_equal((p, s, m), ref, "resnet nearest")
    # round trip bound (size independent): |deq - x| <= step * (0.5 + 1e-6) + fp32 rounding
    y = torch.ops.act_lib.dequant_unpack(p, s, m, 2, g, torch.float32)
    err = (y - x.float()).abs()
    step = s.view(256, -1, 1)
    assert bool((err <= step * 0.500002 + 1e-6 * (1 + x.float().abs())).all())


def test_resnet_full_size_stochastic(resnet_act):
    g = 256
    x = resnet_act.view(256, -1, g)
    noise = torch.rand(x.shape, generator=torch.Generator(device=DEV).manual_seed(1), device=DEV)
    p, s, m = torch.ops.act_lib.quant_pack(x, 2, g, False, 0.0, False, ROUNDINGS["noise"], noise, 0, 0,
                                           torch.float32)
    y = torch.ops.act_lib.dequant_unpack(p, s, m, 2, g, torch.float32)
    step = s.view(256, -1, 1)
    assert bool(((y - x.float()).abs() < step * (1 + 1e-5)).all())
    # bit-exact on all 802,816 groups against the oracle with the same noise
    ref = oracle.quant_pack(np_view(x).reshape(-1, g), g, 2, rounding=oracle.STOCH_NOISE,
                            noise=noise.cpu().numpy().reshape(-1, g))
    assert_quant_equal((p, s, m), ref, "resnet noise tensor")
    del ref
    # Philox: unbiased in aggregate (mean dequant error ~ 0 over 205M elements)
    p2, s2, m2 = torch.ops.act_lib.quant_pack(x, 2, g, False, 0.0, False, ROUNDINGS["philox"], None, 1, 0,
                                              torch.float32)
    y2 = torch.ops.act_lib.dequant_unpack(p2, s2, m2, 2, g, torch.float32)
    rel = float((y2.double() - x.double()).mean() / s2.double().mean())
    assert abs(rel) < 1e-3


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_vit_mlp_full_size_philox(bits):
    """The ViT-B/16 MLP activation at its size: GELU(N(0,1)) bf16 [256, 197, 3072] (1,210,368 groups of
    g = 128), Philox stochastic rounding (seed 1, offset 0), quant-pack then unpack to bf16, as
    the benchmark runs it. Three windows of 64 groups (the first, the middle, the last) match the
    oracle bit for bit (codes, scale, min, dequantized bf16), the Philox stream taken from the
    oracle's generator at those element indices; over the whole tensor every value comes back
    within one step of the input, plus half a bf16 ulp for the output rounding."""
    g = 128
    x = torch.nn.functional.gelu(torch.randn((256, 197, 3072), generator=torch.Generator(device=DEV).manual_seed(2),
                                             device=DEV)).to(torch.bfloat16)
    xg = x.view(256, -1, g)
    ng = x.numel() // g
    print(f"[config 3] {bits}-bit, {ng} groups", flush=True)
    p, s, m = torch.ops.act_lib.quant_pack(xg, bits, g, False, 0.0, False, ROUNDINGS["philox"], None, 1, 0,
                                           torch.float32)
    y = torch.ops.act_lib.dequant_unpack(p, s, m, bits, g, torch.bfloat16)
    torch.cuda.synchronize()
    assert p.shape == (ng, g * bits // 32) and s.shape == (256, ng // 256) and y.shape == xg.shape
    xf = x.view(-1, g)
    for w in (slice(0, 64), slice(ng // 2 - 32, ng // 2 + 32), slice(ng - 64, ng)):
        u = oracle.philox_noise(w.start * g, (w.stop - w.start) * g, 1, 0).reshape(-1, g)
        ref = oracle.quant_pack(np_view(xf[w]), g, bits, rounding=oracle.STOCH_NOISE, noise=u)
        assert_quant_equal((p[w], s.view(-1)[w], m.view(-1)[w]), ref, f"{bits}-bit groups {w}")
        yo = oracle.dequant_unpack(*ref, g, bits, y_dtype=oracle.BF16)
        np.testing.assert_array_equal(np_view(y.view(-1, g)[w]), yo, err_msg=f"{bits}-bit dequant {w}")
    yf = y.view(-1, g).float()
    err = (yf - xf.float()).abs()
    step = s.view(-1, 1)
    assert bool((err <= step * (1 + 1e-6) + yf.abs() * 2.0 ** -8).all())


# ----------------------------------------------------------------------------- FP8 GEMM
def fp8_quantize(x):
    s = 448.0 / x.abs().max().clamp_min(1e-12)
    return (x * s).to(torch.float8_e4m3fn), s


@pytest.mark.parametrize("M,N,K", [(256, 256, 128), (512, 768, 1024), (1024, 256, 4096), (4096, 11008, 4096),
                                   (8192, 8192, 8192)])
def test_fp8_gemm_parity(M, N, K):
    gen = torch.Generator(device=DEV).manual_seed(M + N + K)
    a = torch.randn(M, K, generator=gen, device=DEV)
    b = torch.randn(N, K, generator=gen, device=DEV)
    a8, sa = fp8_quantize(a)
    b8, sb = fp8_quantize(b)
    out_scale = float(1.0 / (sa * sb))
    c = torch.ops.act_lib.fp8_gemm_nt(a8, b8, out_scale)
    ref = (a8.float() @ b8.float().t()) * out_scale
    rel = float((c.float() - ref).norm() / ref.norm())
    assert rel <= 1e-2, rel
    # elementwise: within bf16 rounding of the fp32 result
    assert bool(((c.float() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-3 * ref.abs().max()).all())


@pytest.mark.parametrize("M,N,K", [(1, 1, 16), (100, 300, 48), (257, 255, 144), (1000, 777, 1040), (33, 4099, 2064),
                                   (4095, 4097, 4112), (300, 200, 0), (257, 255, 8336), (600, 520, 8448)])
def test_fp8_gemm_ragged_shapes(M, N, K):
    """Edge tiles (M, N not multiples of 256, K a multiple of 16 but not of 64; K = 0 gives zeros),
    through the C ABI with padded row strides: lda, ldb > K, ldc > N (odd, so element stores), and a
    sentinel around the M x N block of C that must stay untouched. K = 8336 and 8448 (an even slab
    count from K = 8192) take the 16x16x128 persistent kernel's edge instance."""
    gen = torch.Generator(device=DEV).manual_seed(M * 7 + N + K)
    lda, ldb, ldc = K + 32, K + 48, N + 3
    a_buf = torch.randn(M, lda, generator=gen, device=DEV)
    b_buf = torch.randn(N, ldb, generator=gen, device=DEV)
    a8 = (a_buf * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    b8 = (b_buf * 40).clamp(-448, 448).to(torch.float8_e4m3fn)
    # the padding columns hold NaN encodings: a kernel that read past K would turn rows NaN
    a8.view(torch.uint8)[:, K:] = 0x7F
    b8.view(torch.uint8)[:, K:] = 0xFF
    c = torch.full((M + 2, ldc), 77.0, dtype=torch.bfloat16, device=DEV)
    out_scale = 1.0 / 1600.0
    rc = _lib.lib().dopt_fp8_gemm_nt(a8.data_ptr(), b8.data_ptr(), M, N, K, lda, ldb, out_scale, c.data_ptr(), ldc,
                                     torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "fp8_gemm_nt")
    torch.cuda.synchronize()
    ref = (a8[:, :K].float() @ b8[:, :K].float().t()) * out_scale
    got = c[:M, :N].float()
    assert bool(torch.isfinite(got).all())
    if K == 0:
        assert bool((got == 0).all())
    else:
        rel = float((got - ref).norm() / ref.norm())
        assert rel <= 1e-2, rel
        assert bool(((got - ref).abs() <= ref.abs() * 2 ** -7 + 1e-3 * ref.abs().max()).all())
    assert bool((c[:M, N:] == 77.0).all()) and bool((c[M:] == 77.0).all())


def test_fp8_gemm_operator_odd_n():
    """act_lib::fp8_gemm_nt with N % 8 != 0 (ldc = N: element stores) equals the fp32 matmul."""
    gen = torch.Generator(device=DEV).manual_seed(3)
    a8, sa = fp8_quantize(torch.randn(130, 96, generator=gen, device=DEV))
    b8, sb = fp8_quantize(torch.randn(67, 96, generator=gen, device=DEV))
    c = torch.ops.act_lib.fp8_gemm_nt(a8, b8, float(1.0 / (sa * sb)))
    ref = (a8.float() @ b8.float().t()) / (sa * sb)
    assert float((c.float() - ref).norm() / ref.norm()) <= 1e-2


@pytest.mark.parametrize("case", ["nn", "nn_ragged_k", "a_transposed", "b_colmajor", "both_views"])
def test_fp8_linear_any_strides(case):
    """act_lib::fp8_linear, Triton_Linear's contraction (linear.py:43-95: a [M, K] @ b [K, N] with any
    strides), against the fp32 matmul of the same e4m3 operands: b in its row-major [K, N] layout
    (the transposing pack), K not a multiple of 16 (zero-padded), a as a transposed view, b
    column-major (read in place), and both views at once."""
    M, K, N = {"nn": (1024, 2048, 768), "nn_ragged_k": (300, 100, 200), "a_transposed": (520, 272, 260),
               "b_colmajor": (512, 512, 1000), "both_views": (257, 1040, 129)}[case]
    gen = torch.Generator(device=DEV).manual_seed(M + K + N)
    a8, sa = fp8_quantize(torch.randn(M, K, generator=gen, device=DEV))
    b8, sb = fp8_quantize(torch.randn(K, N, generator=gen, device=DEV))
    a_in, b_in = a8, b8
    if case in ("a_transposed", "both_views"):
        a_in = a8.t().contiguous().t()  # strides (1, M)
    if case in ("b_colmajor", "both_views"):
        b_in = b8.t().contiguous().t()  # strides (1, K)
    assert torch.equal(a_in.view(torch.uint8), a8.view(torch.uint8)) and torch.equal(b_in.view(torch.uint8),
                                                                                       b8.view(torch.uint8))
    out_scale = float(1.0 / (sa * sb))
    c = torch.ops.act_lib.fp8_linear(a_in, b_in, out_scale)
    ref = (a8.float() @ b8.float()) * out_scale
    rel = float((c.float() - ref).norm() / ref.norm())
    assert c.shape == (M, N) and rel <= 1e-2, rel
    assert bool(((c.float() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-3 * ref.abs().max()).all())


def test_fp8_pack_kmajor_is_the_strided_copy():
    """dopt_fp8_pack_kmajor against torch's strided indexing: the transposing path (stride_r == 1) and
    the gather path, ragged extents, a destination row stride past cols."""
    L = _lib.lib()
    gen = torch.Generator(device=DEV).manual_seed(9)
    for rows, cols, transposed in ((300, 130, True), (77, 1000, True), (64, 64, True), (45, 33, False)):
        src_store = torch.randint(0, 256, (cols, rows) if transposed else (rows, cols * 2), generator=gen,
                                  device=DEV, dtype=torch.int32).to(torch.uint8)
        view = src_store.t() if transposed else src_store[:, ::2]
        dst = torch.full((rows, cols + 5), 0xAB, dtype=torch.uint8, device=DEV)
        rc = L.dopt_fp8_pack_kmajor(view.data_ptr(), rows, cols, view.stride(0), view.stride(1), dst.data_ptr(),
                                    cols + 5, torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "fp8_pack_kmajor")
        assert torch.equal(dst[:, :cols], view), (rows, cols, transposed)
        assert bool((dst[:, cols:] == 0xAB).all())


def test_fp8_gemm_rejects_bad_shapes():
    a = torch.zeros(100, 120, dtype=torch.float8_e4m3fn, device=DEV)
    b = torch.zeros(256, 120, dtype=torch.float8_e4m3fn, device=DEV)
    with pytest.raises(RuntimeError, match="fp8 GEMM"):
        torch.ops.act_lib.fp8_gemm_nt(a, b, 1.0)


def test_native_library_is_loaded():
    import ctypes  # noqa: F401

    assert _lib.lib().dopt_abi_version() == 1
    with open("/proc/self/maps") as f:
        assert "libdopt.so" in f.read()


def test_beyond_2pow32_elements():
    """A bf16 activation of 2^32 + 2^24 elements (8.6 GB; g = 1024, 4,210,688 groups): element
    offsets past 2^32 take the kernels' 64-bit address arithmetic, and the Philox counter (the
    element index / 16) passes 2^28. Three windows of groups (the first, the 64 on either side of
    element 2^32, the last) match the oracle bit for bit, nearest and Philox, packed codes,
    scale, min and the dequantized bf16 values."""
    g, bits = 1024, 2
    n_el = (1 << 32) + (1 << 24)
    ng = n_el // g
    x = torch.randn((n_el,), generator=torch.Generator(device=DEV).manual_seed(11), device=DEV,
                    dtype=torch.bfloat16).view(1, ng, g)
    b = (1 << 32) // g
    windows = [slice(0, 64), slice(b - 64, b + 64), slice(ng - 64, ng)]
    for rounding, seed, offset in (("nearest", 0, 0), ("philox", 7, 3)):
        print(f"[>2^32] {rounding}", flush=True)
        p, s, m = torch.ops.act_lib.quant_pack(x, bits, g, False, 0.0, False, ROUNDINGS[rounding], None, seed, offset,
                                               torch.float32)
        y = torch.ops.act_lib.dequant_unpack(p, s, m, bits, g, torch.bfloat16)
        torch.cuda.synchronize()
        for w in windows:
            xs = np_view(x[0, w])
            if rounding == "nearest":
                ref = oracle.quant_pack(xs, g, bits)
            else:  # the Philox stream at these element indices, through the oracle's noise-tensor path
                u = oracle.philox_noise(w.start * g, (w.stop - w.start) * g, seed, offset).reshape(-1, g)
                ref = oracle.quant_pack(xs, g, bits, rounding=oracle.STOCH_NOISE, noise=u)
            assert_quant_equal((p[w], s.view(-1)[w], m.view(-1)[w]), ref, f"{rounding} groups {w}")
            yo = oracle.dequant_unpack(*ref, g, bits, y_dtype=oracle.BF16)
            np.testing.assert_array_equal(np_view(y.view(-1, g)[w]), yo, err_msg=f"{rounding} dequant {w}")
        del p, s, m, y
    del x
    torch.cuda.empty_cache()
