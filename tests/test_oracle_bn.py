"""Pins the BatchNorm part of the CPU oracle (oracle_bn_*) before it is trusted as the checker
of the HIP kernels.

  * normalization: against torch's float64 batch_norm (training statistics: mean, biased
    variance, eps inside the square root, affine), and the backward against torch's float64
    autograd of batch_norm;
  * codes, ReLU mask and packing: known answers through the sync path (mean 0, invstd 1 makes
    x_hat = x exactly): integer ramps whose codes have the closed form round(x * QMAX / 31), no
    value lying near a rounding boundary; the packed words from numpy.packbits;
  * the squashed mode equals the already pinned quantizer (oracle_quant_pack, nearest, bf16
    scale/min) applied per channel to the values it quantizes;
  * the ReLU modes' division form keeps |x_hat' - x_hat| <= scale/2 and is monotone;
  * avg_alam: alam_bits = 1 keeps the plain codes, runs of equal values give the plain codes,
    codes are the floor of the runs' mean code argument (float64 from the pinned t), the input
    gradient is the plain one on repeated codes and the reduce adds the Philox-derived tl.rand
    noise.
"""
import numpy as np
import pytest
import torch

import oracle


def bf16(a):
    return oracle.bf16_bits_to_f32(a).astype(np.float64)


def rnd(shape, seed, scale=1.0, shift=0.0):
    r = np.random.default_rng(seed)
    return (r.standard_normal(shape) * scale + shift).astype(np.float32)


def stats32(x):
    s, q = oracle.bn_reduce(x)
    return s.astype(np.float32), q.astype(np.float32)


@pytest.mark.parametrize("shape", [(4, 8, 6, 6), (3, 5, 7, 9), (16, 4, 8, 8)])
def test_normalize_matches_torch_float64(shape):
    x = rnd(shape, 1, scale=2.0, shift=0.7)
    C = shape[1]
    w, b = rnd((C,), 2), rnd((C,), 3)
    s, q = oracle.bn_reduce(x)
    xd = x.astype(np.float64)
    np.testing.assert_allclose(s, xd.sum(axis=(0, 2, 3)), rtol=1e-12)
    np.testing.assert_allclose(q, (xd ** 2).sum(axis=(0, 2, 3)), rtol=1e-12)
    out = oracle.bn_norm_quant(x, w, b, mode=oracle.BN_NORM, eps=1e-5, sum=s.astype(np.float32),
                               sumsq=q.astype(np.float32))
    mean = xd.mean(axis=(0, 2, 3))
    var = xd.var(axis=(0, 2, 3))  # biased, as the kernels compute it
    np.testing.assert_allclose(out["mean"], mean, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(out["var"], var, rtol=1e-5, atol=1e-6)
    want = torch.nn.functional.batch_norm(torch.from_numpy(xd), None, None, torch.from_numpy(w.astype(np.float64)),
                                          torch.from_numpy(b.astype(np.float64)), training=True, eps=1e-5).numpy()
    y = bf16(out["y"])
    assert np.all(np.abs(y - want) <= 2.0 ** -8 * np.abs(want) + 2e-5)
    xh_want = (xd - mean[None, :, None, None]) / np.sqrt(var + 1e-5)[None, :, None, None]
    assert np.all(np.abs(bf16(out["x_hat"]) - xh_want) <= 2.0 ** -8 * np.abs(xh_want) + 2e-5)


def _sync(x, bits, mode, g, w=None, b=None):
    C = x.shape[1]
    w = np.ones(C, np.float32) if w is None else w
    b = np.zeros(C, np.float32) if b is None else b
    return oracle.bn_norm_quant(x, w, b, mode=mode, group_size=g, bits=bits, mean=np.zeros(C, np.float32),
                                invstd=np.ones(C, np.float32))


def _packbits(codes, bits):
    """little-endian bitstream of codes (numpy.packbits over the per-code bit planes)"""
    planes = ((codes[:, None] >> np.arange(bits)[None, :]) & 1).astype(np.uint8).reshape(-1)
    return np.packbits(planes, bitorder="little").view(np.uint32)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("mode", [oracle.BN_RELU_QUANT, oracle.BN_RELU6_QUANT])
def test_relu_modes_known_answer_ramp(bits, mode):
    # one channel, two groups of 32: the ramp 0..31 and the same ramp minus 16 (mask bits vary)
    ramp = np.arange(32, dtype=np.float32)
    x = np.concatenate([ramp, ramp - 16.0]).reshape(1, 1, 64)
    out = _sync(x, bits, mode, 32)
    qmax = (1 << bits) - 1
    want_q = np.floor(ramp.astype(np.float64) * qmax / 31 + 0.5).astype(np.uint32)
    codes = np.concatenate([want_q, want_q])
    np.testing.assert_array_equal(out["packed"].reshape(-1), _packbits(codes, bits))
    np.testing.assert_array_equal(bf16(out["scale"]).reshape(-1), bf16(oracle.f32_to_bf16_bits(
        np.full(2, np.float32(31.0) / np.float32(qmax)))))
    np.testing.assert_array_equal(bf16(out["min"]).reshape(-1), [0.0, -16.0])
    xv = x.reshape(-1).astype(np.float64)
    mask = (xv > 0) & ((xv < 6) if mode == oracle.BN_RELU6_QUANT else True)
    np.testing.assert_array_equal(out["relu_packed"].reshape(-1), _packbits(mask.astype(np.uint32), 1))
    y_want = np.minimum(np.maximum(xv, 0), 6) if mode == oracle.BN_RELU6_QUANT else np.where(mask, xv, 0)
    np.testing.assert_array_equal(bf16(out["y"]).reshape(-1), y_want)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_squash_mode_known_answer_ramp(bits):
    # x_hat on an evenly spaced ramp over [-3, 3]; codes of t = 2 tanh(x_hat / 2) worked out in
    # float64, each value at least 1e-4 (in code units) away from a rounding boundary
    xh = (-3.0 + 6.0 * np.arange(32) / 31).astype(np.float32)
    x = xh.reshape(1, 1, 32)
    out = _sync(x, bits, oracle.BN_QUANT, 32)
    t = 2.0 * np.tanh(xh.astype(np.float64) / 2.0)
    qmax = (1 << bits) - 1
    u = (t - t.min()) / (t.max() - t.min()) * qmax + 0.5
    assert np.all(np.abs(u - np.round(u)) > 1e-4)
    np.testing.assert_array_equal(out["packed"].reshape(-1), _packbits(np.floor(u).astype(np.uint32), bits))
    np.testing.assert_allclose(out["t"].reshape(-1), t, rtol=2e-7, atol=1e-7)


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
@pytest.mark.parametrize("g", [64, 128, 256])  # the pinned quantizer takes g >= 64; g = 32 is pinned by the ramps
def test_squash_mode_equals_pinned_quantizer(bits, g):
    x = rnd((4, 3, 8, 8), 10 + bits, scale=1.5, shift=0.3)
    C, M = 3, 4 * 64
    w, b = rnd((C,), 4), rnd((C,), 5)
    s, q = stats32(x)
    out = oracle.bn_norm_quant(x, w, b, mode=oracle.BN_QUANT, group_size=g, bits=bits, eps=1e-5, sum=s, sumsq=q)
    t = out["t"]  # [C, M], channel-major flat order n*HW + s
    xd = x.astype(np.float64)
    xh = (xd - out["mean"][None, :, None, None]) / np.sqrt(out["var"].astype(np.float64) + 1e-5)[None, :, None, None]
    t_want = 2.0 * np.tanh(np.clip(xh, -3, 3) / 2.0)
    np.testing.assert_allclose(t, t_want.transpose(1, 0, 2, 3).reshape(C, M), rtol=1e-5, atol=1e-6)
    rp, rs, rm = oracle.quant_pack(t.reshape(-1, g), g, bits, meta_dtype=oracle.BF16)
    np.testing.assert_array_equal(out["packed"].reshape(-1), rp.reshape(-1))
    np.testing.assert_array_equal(out["scale"].reshape(-1), rs)
    np.testing.assert_array_equal(out["min"].reshape(-1), rm)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_relu_mode_division_bound_and_monotone(bits):
    x = rnd((8, 2, 4, 8), 30 + bits, scale=1.0)
    C, M, g = 2, 8 * 32, 64
    w, b = rnd((C,), 6), rnd((C,), 7)
    s, q = stats32(x)
    out = oracle.bn_norm_quant(x, w, b, mode=oracle.BN_RELU_QUANT, group_size=g, bits=bits, eps=1e-5, sum=s, sumsq=q)
    t = out["t"].reshape(-1, g).astype(np.float64)
    codes = oracle.unpack_codes(out["packed"].reshape(-1, g * bits // 32), g, bits).view(np.uint8).astype(np.float64)
    # the step kept in fp32 by the kernel is the unrounded rng / QMAX; the stored bf16 is its rounding
    step = (t.max(axis=1) - t.min(axis=1)) / ((1 << bits) - 1)
    deq = codes * step[:, None] + t.min(axis=1)[:, None]
    assert np.all(np.abs(deq - t) <= step[:, None] * (0.5 + 1e-5))
    order = np.argsort(t, axis=1, kind="stable")
    assert np.all(np.diff(np.take_along_axis(codes, order, axis=1), axis=1) >= 0)


@pytest.mark.parametrize("eps", [1e-7, 1e-5])
def test_backward_matches_torch_autograd(eps):
    shape = (6, 4, 5, 8)
    x = rnd(shape, 40, scale=1.3, shift=-0.2)
    C = shape[1]
    w, b = rnd((C,), 8) + 1.0, rnd((C,), 9)
    dy = rnd(shape, 41)
    s, q = stats32(x)
    fw = oracle.bn_norm_quant(x, w, b, mode=oracle.BN_NORM, eps=eps, sum=s, sumsq=q)
    dw, db = oracle.bn_bwd_reduce(dy, mode=oracle.BN_NORM, x_hat=fw["x_hat"])
    dx = oracle.bn_bwd_dx(dy, dw.astype(np.float32), db.astype(np.float32), w, fw["var"], mode=oracle.BN_NORM,
                          eps=eps, x_hat=fw["x_hat"])
    xt = torch.from_numpy(x.astype(np.float64)).requires_grad_(True)
    wt = torch.from_numpy(w.astype(np.float64)).requires_grad_(True)
    bt = torch.from_numpy(b.astype(np.float64)).requires_grad_(True)
    torch.nn.functional.batch_norm(xt, None, None, wt, bt, training=True, eps=eps).backward(
        torch.from_numpy(dy.astype(np.float64)))
    # x_hat is kept in bf16 (relative error 2^-9), the sums and dx follow it
    np.testing.assert_allclose(db, bt.grad.numpy(), rtol=1e-6, atol=1e-6)
    xh = bf16(fw["x_hat"])
    assert np.all(np.abs(dw - wt.grad.numpy()) <= 2.0 ** -8 * np.abs(dy * xh).sum(axis=(0, 2, 3)) + 1e-6)
    got = bf16(dx)
    want = xt.grad.numpy()
    assert np.sqrt(((got - want) ** 2).mean()) <= 1e-2 * np.sqrt((want ** 2).mean())


def test_relu_backward_masks_dy():
    """With the ReLU mask all zero the reduce sums are zero and dx is -(0 + x_hat' * 0) * ... = 0."""
    x = -np.abs(rnd((2, 1, 8, 8), 50)) - 1.0
    C = 1
    w, b = np.ones(C, np.float32), np.zeros(C, np.float32)
    out = oracle.bn_norm_quant(x, w, b, mode=oracle.BN_RELU_QUANT, group_size=32, bits=2,
                               mean=np.zeros(C, np.float32), invstd=np.ones(C, np.float32))
    assert not out["relu_packed"].any()
    dy = rnd(x.shape, 51)
    dw, db = oracle.bn_bwd_reduce(dy, mode=oracle.BN_RELU_QUANT, packed=out["packed"],
                                  relu_packed=out["relu_packed"], scale=out["scale"], min=out["min"], group_size=32,
                                  bits=2)
    assert dw[0] == 0.0 and db[0] == 0.0
    dx = oracle.bn_bwd_dx(dy, dw.astype(np.float32), db.astype(np.float32), w, np.ones(C, np.float32),
                          mode=oracle.BN_RELU_QUANT, eps=1e-5, packed=out["packed"], relu_packed=out["relu_packed"],
                          scale=out["scale"], min=out["min"], group_size=32, bits=2)
    assert not np.any(bf16(dx))


# ----------------------------------------------------------------------------- avg_alam
def _codes(packed, bits):
    """codes of a little-endian code bitstream (numpy.unpackbits)"""
    b = np.unpackbits(np.ascontiguousarray(packed).reshape(-1).view(np.uint8), bitorder="little")
    return (b.reshape(-1, bits).astype(np.int64) << np.arange(bits)).sum(axis=1)


def _philox_uniform(seed, off):
    """tl.rand(seed, off) from the Philox words (pinned by the known-answer vectors): word 0 as
    int32, folded to non-negative, times fp32(4.6566127342e-10)"""
    ctr = np.array([off, 0, 0, 0], np.uint32)
    key = np.array([seed & 0xFFFFFFFF, seed >> 32], np.uint32)
    out = np.zeros(4, np.uint32)
    oracle.lib().oracle_philox4x32_10(ctr.ctypes.data, key.ctypes.data, out.ctypes.data)
    i = int(out[:1].view(np.int32)[0])
    i = ~i if i < 0 else i
    return float(np.float32(i) * np.float32(4.6566127342e-10))


def test_triton_rand_is_the_first_philox_word_as_a_uniform():
    for seed, off in [(42, 0), (42, 5), (43, 255), (42 + 7, 511), (2**33 + 1, 17)]:
        assert oracle.triton_rand(seed, off) == _philox_uniform(seed, off)
    u = np.array([oracle.triton_rand(42 + b, e) for b in range(16) for e in range(512)])
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1.0 / 12.0) < 0.005


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_alam_one_keeps_the_plain_codes(bits):
    x = rnd((4, 3, 8, 8), 60 + bits, scale=1.5)
    C = 3
    w, b = rnd((C,), 61), rnd((C,), 62)
    s, q = stats32(x)
    kw = dict(mode=oracle.BN_QUANT, group_size=64, bits=bits, eps=1e-5, sum=s, sumsq=q)
    plain = oracle.bn_norm_quant(x, w, b, **kw)
    one = oracle.bn_norm_quant(x, w, b, alam_bits=1, **kw)
    for k in ("y", "packed", "scale", "min"):
        np.testing.assert_array_equal(one[k], plain[k])


@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_alam_two_on_pairs_of_equal_values(bits):
    """Runs of two equal x_hat (sync path: x_hat = x): the mean of a pair of equal qf is that qf
    exactly, so the codes are the plain mode's codes of every other element."""
    x = np.repeat(rnd((1, 2, 128), 70 + bits, scale=1.2), 2, axis=2)  # [1, 2, 256], pairs of equal values
    plain = _sync(x, bits, oracle.BN_QUANT, 256)
    got = oracle.bn_norm_quant(x, np.ones(2, np.float32), np.zeros(2, np.float32), mode=oracle.BN_QUANT,
                               group_size=256, bits=bits, mean=np.zeros(2, np.float32), invstd=np.ones(2, np.float32),
                               alam_bits=2)
    want = _codes(plain["packed"], bits).reshape(2, -1)[:, ::2]
    np.testing.assert_array_equal(_codes(got["packed"], bits).reshape(2, -1), want)
    np.testing.assert_array_equal(got["scale"], plain["scale"])
    np.testing.assert_array_equal(got["min"], plain["min"])


def _alam_case(bits, alam, seed, g=256):
    x = rnd((4, 2, 16, 16), seed, scale=1.4, shift=0.2)
    C = 2
    w, b = rnd((C,), seed + 1) + 1.0, rnd((C,), seed + 2)
    s, q = stats32(x)
    kw = dict(mode=oracle.BN_QUANT, group_size=g, bits=bits, eps=1e-5, sum=s, sumsq=q)
    return x, w, b, oracle.bn_norm_quant(x, w, b, **kw), oracle.bn_norm_quant(x, w, b, alam_bits=alam, **kw)


@pytest.mark.parametrize("bits,alam", [(1, 2), (2, 2), (2, 4), (4, 8), (8, 16), (8, 64)])
def test_alam_codes_are_the_truncated_run_means(bits, alam):
    """Each code is floor of the mean of its run's code arguments qf = (t - min) / scale + 0.5 - 1e-6,
    worked out in float64 from the pinned t, min and scale; runs whose mean lies within 1e-4 of an
    integer are left out (fp32 summation order)."""
    g = 256
    _, _, _, plain, got = _alam_case(bits, alam, 80 + bits + alam, g)
    t = plain["t"].astype(np.float64).reshape(-1, g)
    mn = t.min(axis=1, keepdims=True)
    qmax = (1 << bits) - 1
    step = (t.max(axis=1, keepdims=True) - mn) / qmax
    qf = (t - mn) / step + (0.5 - 1e-6)
    mean = qf.reshape(-1, g // alam, alam).mean(axis=2)
    want = np.clip(np.floor(mean), 0, qmax)
    codes = _codes(got["packed"], bits).reshape(want.shape)
    far = np.abs(mean - np.round(mean)) > 1e-4
    assert far.mean() > 0.95
    np.testing.assert_array_equal(codes[far], want[far])
    np.testing.assert_array_equal(got["scale"], plain["scale"])
    np.testing.assert_array_equal(got["min"], plain["min"])
    assert got["packed"].shape == (2, 4 * 256 * bits // 32 // alam)


def _repeat_codes(packed, bits, alam):
    """the plain layout of avg_alam codes: every code written alam times"""
    return _packbits(np.repeat(_codes(packed, bits), alam).astype(np.uint32), bits).reshape(packed.shape[0], -1)


@pytest.mark.parametrize("bits,alam", [(2, 2), (4, 4), (8, 16)])
def test_alam_backward_is_the_plain_backward_of_repeated_codes(bits, alam):
    """dx with avg_alam is the plain mode's dx on the codes repeated alam times (no noise, bit for
    bit); the reduce adds q + (tl.rand(42 + e / (2 g), e mod g) - 0.5) per element: its dbias is the
    plain one and its dweight the float64 sum of dy * fma(q + noise, scale, min) with the noise
    from the Philox words."""
    g = 256
    x, w, b, _, fw = _alam_case(bits, alam, 90 + bits, g)
    dy = rnd(x.shape, 91 + bits)
    rep = _repeat_codes(fw["packed"], bits, alam)
    kw = dict(mode=oracle.BN_QUANT, scale=fw["scale"], min=fw["min"], group_size=g, bits=bits)
    dw_p, db_p = oracle.bn_bwd_reduce(dy, packed=rep, **kw)
    dw_a, db_a = oracle.bn_bwd_reduce(dy, packed=fw["packed"], alam_bits=alam, **kw)
    np.testing.assert_array_equal(db_a, db_p)
    C, M = 2, 4 * 256
    q = _codes(rep, bits).reshape(C, M).astype(np.float32)
    e = np.arange(M)
    u = np.array([_philox_uniform(42 + int(k) // (2 * g), int(k) % g) for k in e], dtype=np.float32)
    qn = q + (u - np.float32(0.5))[None, :]
    sc = np.repeat(bf16(fw["scale"]), g, axis=1)
    mn = np.repeat(bf16(fw["min"]), g, axis=1)
    xq = qn.astype(np.float64) * sc + mn
    dyc = dy.transpose(1, 0, 2, 3).reshape(C, M).astype(np.float64)
    want = (dyc * xq).sum(axis=1)
    assert np.all(np.abs(dw_a - want) <= 1e-6 * (np.abs(dyc) * np.abs(xq)).sum(axis=1))
    assert np.all(np.abs(dw_a - dw_p) > 0)  # the noise changes dweight
    args = (dw_a.astype(np.float32), db_a.astype(np.float32), w, fw["var"])
    dx_p = oracle.bn_bwd_dx(dy, *args, packed=rep, eps=1e-7, **kw)
    dx_a = oracle.bn_bwd_dx(dy, *args, packed=fw["packed"], alam_bits=alam, eps=1e-7, **kw)
    np.testing.assert_array_equal(dx_a, dx_p)


def test_alam_rejects_run_lengths_the_reference_cannot_reshape():
    x = rnd((2, 1, 8, 8), 99)
    w, b = np.ones(1, np.float32), np.zeros(1, np.float32)
    s, q = stats32(x)
    for alam in (3, 4):  # g = 64, 2 bits: 4 code words; 3 is no power of two, 4 divides them
        kw = dict(mode=oracle.BN_QUANT, group_size=64, bits=2, eps=1e-5, sum=s, sumsq=q, alam_bits=alam)
        if alam == 3:
            with pytest.raises(RuntimeError):
                oracle.bn_norm_quant(x, w, b, **kw)
        else:
            oracle.bn_norm_quant(x, w, b, **kw)
    with pytest.raises(RuntimeError):  # 8 does not divide 4 words
        oracle.bn_norm_quant(x, w, b, mode=oracle.BN_QUANT, group_size=64, bits=2, eps=1e-5, sum=s, sumsq=q,
                             alam_bits=8)
    with pytest.raises(RuntimeError):  # avg_alam is a squashed-mode option
        oracle.bn_norm_quant(x, w, b, mode=oracle.BN_RELU_QUANT, group_size=64, bits=2, eps=1e-5, sum=s, sumsq=q,
                             alam_bits=2)


def test_squash_code_bar_accepts_exact_ties_and_rejects_planted_mistakes():
    """The GPU tests' bar for the squashed mode's codes (tests/test_gpu_bn.py::squash_codes_close),
    checked on oracle codes: bf16 data with five distinct values, symmetric about a channel mean of
    exactly -3.0, puts every x = -3.0 element at x_hat = 0 and its code argument exactly at a half
    step, where the last ulp of the squash decides the rounding. A one-step flip of those elements
    passes; a one-step flip elsewhere, a two-step difference, and codes from a planted wrong eps
    (1e-2 in place of 1e-5) fail."""
    from tests.test_gpu_bn import codes_of, squash_codes_close

    vals = torch.tensor([-3.03125, -3.015625, -3.0, -2.984375, -2.96875])
    pattern = torch.tensor([0, 1, 2, 3, 4, 2, 2, 2])
    col = vals[pattern[torch.arange(256) % 8]]
    x = torch.stack([col, col.flip(0)], dim=1).view(256, 2, 1, 1).to(torch.bfloat16)
    xn = x.view(torch.int16).numpy().view(np.uint16)
    w, b = np.ones(2, np.float32), np.zeros(2, np.float32)
    s, q = oracle.bn_reduce(xn)

    def quant(eps):
        return oracle.bn_norm_quant(xn, w, b, mode=oracle.BN_QUANT, group_size=128, bits=8, eps=eps, sum=s, sumsq=q)

    ref = quant(1e-5)
    mean, var = torch.from_numpy(ref["mean"]), torch.from_numpy(ref["var"])
    assert float(mean[0]) == -3.0 and float(mean[1]) == -3.0
    codes = codes_of(ref["packed"], 8).reshape(2, 256)
    xc = x.float().view(256, 2).t().numpy()  # channel-major, like the codes
    tie = xc == -3.0

    def packed(c):
        return np.ascontiguousarray(c.astype(np.uint8)).view(np.uint32)

    flipped = codes.copy()
    flipped[tie] = np.where(codes[tie] >= 128, codes[tie] - 1, codes[tie] + 1)
    assert squash_codes_close(x, mean, var, packed(flipped), ref["packed"], 8, 128)[0]
    for e in np.flatnonzero(~tie[0])[:3]:  # one step off at an element far from a boundary
        c = codes.copy()
        c[0, e] += 1 if c[0, e] < 255 else -1
        assert not squash_codes_close(x, mean, var, packed(c), ref["packed"], 8, 128)[0]
    c = codes.copy()
    e = np.flatnonzero(tie[0])[0]
    c[0, e] += 2 if c[0, e] < 128 else -2
    assert not squash_codes_close(x, mean, var, packed(c), ref["packed"], 8, 128)[0]
    assert not squash_codes_close(x, mean, var, quant(1e-2)["packed"], ref["packed"], 8, 128)[0]
