"""float64 / numpy restatements shared by the oracle pins (tests/test_oracle.py) and the GPU
parity tests: an exact float32 fused multiply-add, the vectorised quantizer, numpy.packbits
packing, and the float64 clamp + tanh squash with its comparison.

Test infrastructure only.
"""
import numpy as np

import oracle

NEAREST, NOISE = oracle.NEAREST, oracle.STOCH_NOISE


def packbits_reference(codes, bits):
    """Little-endian bitstream of b-bit codes via numpy.packbits (library routine)."""
    codes = np.asarray(codes, dtype=np.int64)
    expanded = ((codes[..., None] >> np.arange(bits)) & 1).astype(np.uint8)
    flat = expanded.reshape(codes.shape[0], -1)
    return np.packbits(flat, axis=1, bitorder="little")


def fma32(a, b, c):
    """Correctly rounded float32 fused multiply-add in numpy, independent of any libm fmaf:
    a*b is exact in float64 (24 + 24 bits); TwoSum gives the exact error of the float64 sum;
    rounding that sum to odd at 53 bits and then to nearest at 24 bits is correctly rounded
    (53 >= 24 + 2, Boldo & Melquiond)."""
    a = np.asarray(a, dtype=np.float32).astype(np.float64)
    b = np.asarray(b, dtype=np.float32).astype(np.float64)
    c = np.asarray(c, dtype=np.float32).astype(np.float64)
    p = a * b
    with np.errstate(invalid="ignore", over="ignore"):
        s = p + c
        bp = s - c
        e = (p - (s - bp)) + (c - bp)  # exact: p + c == s + e (finite s)
        bits = s.view(np.int64).copy()
        inexact = np.isfinite(s) & (e != 0)
        # truncate toward zero: RN went away from zero when e and s have opposite signs
        away = inexact & (np.sign(e) != np.sign(s)) & (s != 0)
        bits[away] -= 1
        bits[inexact] |= 1  # round to odd
        odd = bits.view(np.float64)
        return odd.astype(np.float32)


def numpy_quant(x, bits, rounding=NEAREST, u=None):
    """Vectorised numpy float32 restatement: each array op rounds once, fma32 for the fused
    multiply-add of the reference's contracted `(x - mn) * inv + c`."""
    f = np.float32
    qmax = (1 << bits) - 1
    mn = x.min(axis=1) + f(0.0)
    mx = x.max(axis=1)
    rng = (mx - mn).astype(np.float32)
    step = np.where(rng > 0, rng / f(qmax), f(1.0)).astype(np.float32)
    inv = (f(1.0) / step).astype(np.float32)
    t = (x - mn[:, None]).astype(np.float32)
    if rounding == NEAREST:
        qf = fma32(t, np.broadcast_to(inv[:, None], t.shape), np.full(t.shape, f(0.5 - 1e-6)))
        q = np.clip(qf, 0, qmax).astype(np.int64)
    else:
        qf = (fma32(t, np.broadcast_to(inv[:, None], t.shape), u) - f(0.5)).astype(np.float32)
        q = np.rint(np.clip(qf, 0, qmax)).astype(np.int64)
    packed = packbits_reference(q, bits).view("<u4")
    return packed, step, mn


# The pre-transform every compressed Linear / Conv layer runs (AC/modules/ops.py:262-264, :472-474
# pass clamp=True, alpha=3 into AC/act_triton_kernel.py:55-58): x = clamp(x, -alpha, alpha), then
# x = tanh(x / 0.5) * 0.5, then the quantizer. It is pinned against float64: numpy's clip and
# tanh, rounded once to fp32, followed by the numpy quantizer restatement above.
def _ulp32(v):
    v = np.abs(np.asarray(v, dtype=np.float32))
    return (np.nextafter(v, np.float32(np.inf)) - v).astype(np.float64)


def f64_pretransform(x, alpha, clamp_first=True, form="tanh2x/2"):
    """float64 restatement of the clamp + squash, rounded once to fp32. `clamp_first` and `form`
    exist to plant mistakes: the squash applied before the clamp, or BatchNorm's 2 tanh(x/2)."""
    v = np.asarray(x, dtype=np.float32).astype(np.float64)
    sq = (lambda t: np.tanh(2.0 * t) / 2.0) if form == "tanh2x/2" else (lambda t: 2.0 * np.tanh(t / 2.0))
    if clamp_first:
        v = sq(np.clip(v, -alpha, alpha))
    else:
        v = np.clip(sq(v), -alpha, alpha)
    return v.astype(np.float32)


def squash_mismatch(got, x, bits, alpha, u=None, **plant):
    """Compares the oracle's (packed, scale, min) of the clamped + squashed quantizer with the float64
    restatement. Returns a list of failures: min beyond 2 fp32 ulps; scale beyond what 2 ulps on the
    group's max and min give after one subtraction and one division; codes that differ at an element
    whose restated code is not within 4 ulps of the squashed value of a rounding boundary. `u` (the
    noise per element) selects stochastic rounding, else nearest."""
    p, s, m = got
    qmax = (1 << bits) - 1
    sq = f64_pretransform(x, alpha, **plant)
    _, step_r, mn_r = numpy_quant(sq, bits)
    mx_r = sq.max(axis=1)
    fails = []
    if np.any(np.abs(m.astype(np.float64) - mn_r) > 2 * _ulp32(mn_r)):
        fails.append("min")
    tol = (2 * _ulp32(mx_r) + 2 * _ulp32(mn_r)) / qmax + 2 * _ulp32(step_r)
    if np.any(np.abs(s.astype(np.float64) - step_r) > tol):
        fails.append("scale")
    # codes of the restated squash with the oracle's own scale/min (isolates the squash from the
    # statistics), and a 4-ulp band around it that marks the rounding-boundary elements
    inv = (np.float32(1) / s).astype(np.float32)
    codes = oracle.unpack_codes(p, x.shape[1], bits).view(np.uint8 if bits == 8 else np.int8).astype(np.int64)

    def code_of(v):
        t = (v - m[:, None]).astype(np.float32)
        invb = np.broadcast_to(inv[:, None], t.shape)
        if u is None:
            qf = fma32(t, invb, np.full(t.shape, np.float32(0.5 - 1e-6)))
            return np.clip(np.floor(qf), 0, qmax).astype(np.int64)
        qf = (fma32(t, invb, u) - np.float32(0.5)).astype(np.float32)
        return np.rint(np.clip(qf, 0, qmax)).astype(np.int64)

    want = code_of(sq)
    band = (4 * _ulp32(sq)).astype(np.float32)
    boundary = (code_of((sq - band).astype(np.float32)) != code_of((sq + band).astype(np.float32)))
    off = (codes != want) & ~boundary
    if off.any():
        fails.append(f"codes ({int(off.sum())} off the boundaries)")
    if boundary.mean() > 0.01:
        fails.append("too many boundary elements")
    return fails


def squash_inputs(seed):
    """Groups inside |x| < 1/16, straddling it, straddling 0.45, of N(0, 1) and beyond alpha."""
    rng = np.random.default_rng(seed)
    g = 256
    rows = [rng.uniform(-1 / 16, 1 / 16, (16, g)), rng.uniform(-1 / 32, 3 / 32, (16, g)),
            rng.uniform(-1e-3, 1e-3, (8, g)), rng.uniform(0.3, 0.6, (16, g)), rng.standard_normal((32, g)),
            rng.standard_normal((32, g)) * 4]
    return np.concatenate(rows).astype(np.float32)
