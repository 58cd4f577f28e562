"""Inputs whose launches need more than 2^32 - 1 work-items, i.e. more than one row of a 1-D grid
(a dispatch's grid size is a 32-bit count of work-items per dimension). The launchers then use a
2-D grid of 65536-block rows and the kernels a 64-bit linear block index. Each test takes the
cheapest configuration that crosses the limit for one kernel family, compares windows of groups
bit for bit with the oracle (the first, the two sides of the first row boundary, the start of the
last, partial row and the end), and checks a size-independent property over the whole tensor.

Device memory: 18 to 142 GB per test (an MI355X holds 288 GB); each test frees what it allocated.
"""
import numpy as np
import pytest
import torch

import deep_optimization_amd  # noqa: F401
import oracle
from deep_optimization_amd import _lib
from tests.test_gpu_parity import assert_quant_equal, np_view

pytestmark = pytest.mark.gpu
DEV = "cuda"
ROW = 1 << 16  # blocks per row of a 2-D grid


def need_free(gb):
    free = torch.cuda.mem_get_info()[0]
    if free < gb * 1e9:
        pytest.skip(f"needs {gb} GB of free device memory, {free / 1e9:.0f} GB free")


def release():
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def windows(n, edges, half):
    """[0, 2 half), [e - half, e + half) for each edge, [n - 2 half, n)."""
    out = [slice(0, 2 * half)] + [slice(e - half, e + half) for e in edges] + [slice(n - 2 * half, n)]
    assert all(0 <= w.start < w.stop <= n for w in out)
    return out


def test_alam_quant_and_dequant_past_one_grid_row():
    """ALAM quantize (one wave per group) and dequantize (one lane per element) of bf16
    [2^26 + 2^16 groups of 64] (4.3e9 elements): 2^32 + 2^22 lanes each. Codes, scale and min bit
    for bit (no squash); the dequantized values within one bf16 ulp (the noise's log / cos)."""
    need_free(24)
    g, bits, alam = 64, 2, 2
    ng = (1 << 26) + (1 << 16)
    gen = torch.Generator(device=DEV).manual_seed(21)
    x = torch.randn((ng * g,), generator=gen, device=DEV, dtype=torch.bfloat16)
    p = torch.empty((ng, g * bits // 32 // alam), dtype=torch.int32, device=DEV)
    s = torch.empty(ng, dtype=torch.bfloat16, device=DEV)
    m = torch.empty(ng, dtype=torch.bfloat16, device=DEV)
    L, st = _lib.lib(), torch.cuda.current_stream().cuda_stream
    print("[large] alam quant", flush=True)
    rc = L.dopt_alam_quant_pack(x.data_ptr(), _lib.BF16, ng, g, bits, alam, 0, 0.0, p.data_ptr(), s.data_ptr(),
                                m.data_ptr(), st)
    assert rc == 0, L.dopt_last_error()
    y = torch.empty((ng, g), dtype=torch.bfloat16, device=DEV)
    print("[large] alam dequant", flush=True)
    rc = L.dopt_alam_dequant_unpack(p.data_ptr(), s.data_ptr(), m.data_ptr(), ng, g, bits, alam, oracle.ALAM_SEED,
                                    y.data_ptr(), st)
    assert rc == 0, L.dopt_last_error()
    torch.cuda.synchronize()
    # both grids: 4 groups per quant block and 4 groups of 64 lanes per dequant block, so row r
    # starts at group 4 r ROW in both
    for w in windows(ng, [4 * ROW, 4 * 256 * ROW], 32):
        rp, rs, rm = oracle.alam_quant_pack(np_view(x.view(ng, g)[w]), g, bits, alam)
        np.testing.assert_array_equal(np_view(p[w]).view(np.uint32), rp, err_msg=f"codes {w}")
        np.testing.assert_array_equal(np_view(s[w]), rs, err_msg=f"scale {w}")
        np.testing.assert_array_equal(np_view(m[w]), rm, err_msg=f"min {w}")
        yo = oracle.alam_dequant_unpack(rp, rs, rm, g, bits, alam, seed=oracle.ALAM_SEED + w.start)
        diff = np.abs(np_view(y[w]).astype(np.int64) - yo.reshape(-1, g).astype(np.int64))
        assert diff.max() <= 1 and np.mean(diff != 0) < 0.01, f"dequant {w}"
    del x, p, s, m, y
    release()


def test_pack_and_unpack_codes_past_one_grid_row():
    """8-bit code pack / unpack (one lane per word) of 2^34 + 2^20 int8 codes: 2^32 + 2^18 lanes.
    At 8 bits, codes 0..127 pack to their bytes in little-endian order (the word is the int32 sum
    of the shifted, sign-extended codes, as the reference's sum computes it, so a code of 128 or
    more would borrow from the next byte), so the whole packed tensor equals the codes
    reinterpreted as int32, and the unpack returns the codes."""
    need_free(75)
    g, bits = 256, 8
    ng = (1 << 26) + (1 << 12)
    gen = torch.Generator(device=DEV).manual_seed(22)
    codes = torch.randint(0, 128, (1, ng, g), generator=gen, device=DEV, dtype=torch.int8)
    print("[large] pack codes", flush=True)
    packed = torch.ops.act_lib.pack_triton(codes, bits, g)
    torch.cuda.synchronize()
    assert torch.equal(packed.view(-1), codes.view(-1).view(torch.int32))
    for w in windows(ng, [ROW * 256 // 64, 256 * ROW * 256 // 64], 32):  # 64 words per group
        np.testing.assert_array_equal(np_view(packed[w]).view(np.uint32),
                                      oracle.pack_codes(np_view(codes[0, w]), g, bits), err_msg=f"{w}")
    print("[large] unpack codes", flush=True)
    back = torch.ops.act_lib.unpack_triton(packed, bits, 1, ng, g)
    del packed
    assert torch.equal(back, codes)
    del codes, back
    release()


def test_quant_pack_noise_tensor_past_one_grid_row():
    """fp32 [2^26 + 2^12 groups of 256] with a caller's noise tensor (2-bit, fp32 scale/min):
    4 elements per lane, 2^32 + 2^18 lanes. Windows bit for bit against the oracle; then the bf16
    dequantization of all 1.7e10 elements (64-bit offsets throughout) lies within one step of x
    (stochastic codes round to a neighbouring level) plus the bf16 rounding, chunk by chunk."""
    need_free(150)
    g, bits = 256, 2
    ng = (1 << 26) + (1 << 12)
    n = ng * g
    gen = torch.Generator(device=DEV).manual_seed(23)
    x = torch.randn((1, ng, g), generator=gen, device=DEV, dtype=torch.float32)
    u = torch.rand((1, ng, g), generator=gen, device=DEV, dtype=torch.float32)
    print("[large] quant_pack noise", flush=True)
    p, s, m = torch.ops.act_lib.quant_pack(x, bits, g, False, 0.0, False, oracle.STOCH_NOISE, u, 0, 0, torch.float32)
    torch.cuda.synchronize()
    # one group per wave, 4 waves per block: row r starts at group 4 r ROW
    for w in windows(ng, [4 * ROW, 4 * 256 * ROW], 32):
        ref = oracle.quant_pack(np_view(x[0, w]), g, bits, rounding=oracle.STOCH_NOISE, noise=np_view(u[0, w]))
        assert_quant_equal((p[w], s.view(-1)[w], m.view(-1)[w]), ref, f"groups {w}")
    del u
    release()
    print("[large] dequant_unpack", flush=True)
    y = torch.ops.act_lib.dequant_unpack(p, s, m, bits, g, torch.bfloat16)
    torch.cuda.synchronize()
    for w in windows(ng, [4 * ROW, 4 * 256 * ROW], 32):
        ref = (np_view(p[w]).view(np.uint32), np_view(s.view(-1)[w]), np_view(m.view(-1)[w]))
        np.testing.assert_array_equal(np_view(y.view(ng, g)[w]), oracle.dequant_unpack(*ref, g, bits, y_dtype=oracle.BF16),
                                      err_msg=f"dequant {w}")
    sv = s.view(-1)
    yv = y.view(ng, g)
    step = 1 << 20  # groups per chunk (1 GB of x)
    for c in range(0, ng, step):
        xs, ys = x[0, c:c + step], yv[c:c + step].float()
        bound = sv[c:c + step, None] * (1 + 1e-6) + ys.abs() * 2.0 ** -8 + 1e-30
        assert bool(((ys - xs).abs() <= bound).all()), f"groups {c}.."
    assert n == y.numel()
    del x, p, s, m, y, xs, ys, bound
    release()


def test_relu_unpack_past_one_grid_row():
    """The flat elementwise kernels (here the 1-bit ReLU backward: dx = bf16(dy * mask)) over
    2^35 + 2^21 elements: 8 per lane, 2^32 + 2^18 lanes. Windows bit for bit against the oracle,
    and every element, chunk by chunk, equal to dy where its mask bit is set and 0 elsewhere."""
    need_free(150)
    bits = 1
    n = (1 << 35) + (1 << 21)
    gen = torch.Generator(device=DEV).manual_seed(24)
    packed = torch.randint(-(1 << 31), 1 << 31, (n // 32,), generator=gen, device=DEV, dtype=torch.int32)
    dy = torch.randn((n,), generator=gen, device=DEV, dtype=torch.bfloat16)
    print("[large] relu_bwd_fused_unpack", flush=True)
    # the operator's layout arguments: N = 1 row of G groups of 64
    dx = torch.ops.act_lib.relu_bwd_fused_unpack(packed.view(n // 64, 2), dy.view(1, n), bits, 1, n // 64, 64)
    torch.cuda.synchronize()
    # 2048 elements per block: row r starts at element 2048 r ROW
    for w in windows(n, [2048 * ROW, 2048 * 256 * ROW], 2048):
        want = oracle.relu_unpack(np_view(packed[w.start // 32:w.stop // 32]).view(np.uint32), np_view(dy[w]), bits)
        np.testing.assert_array_equal(np_view(dx.view(-1)[w]), want, err_msg=f"elements {w}")
    shifts = torch.arange(32, device=DEV, dtype=torch.int32)
    dxv = dx.view(-1)
    step = 1 << 28
    for c in range(0, n, step):
        bit = ((packed[c // 32:(c + step) // 32, None] >> shifts) & 1).view(-1).bool()
        want = torch.where(bit, dy[c:c + step], torch.zeros((), dtype=dy.dtype, device=DEV))
        assert torch.equal(dxv[c:c + step], want), f"elements {c}.."
    del packed, dy, dx, dxv, bit, want
    release()
