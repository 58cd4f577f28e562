"""The measurement probes (libdopt_probe.so, probes/dopt_probe.h) on the GPU: the same-mix
bandwidth probe reads what it claims to, the instruction-cost probe runs every kind, and its
kind 8 checks the quantizer's fast exact-division helpers against the IEEE division on every
non-negative fp32 bit pattern."""
import numpy as np
import pytest
import torch

import probes

pytestmark = pytest.mark.gpu
EINVAL = -2


@pytest.mark.parametrize("bits", [0, 1, 2, 4, 8])
@pytest.mark.parametrize("with_noise", [True, False])
def test_stream_probe_writes_hash_of_reads(bits, with_noise):
    """dopt_stream_probe (the same-mix bandwidth ceiling the benchmark reports) reads every byte
    it claims to: its outputs are the XOR of each unit's 16 x bytes (and 32 noise bytes) as
    documented, checked against numpy, for a unit count that ends mid-group."""
    L = probes.lib()
    n = 1000
    gen = torch.Generator().manual_seed(bits * 2 + with_noise)
    x = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, 4), generator=gen, dtype=torch.int64).to(torch.int32)
    nz = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, 8), generator=gen, dtype=torch.int64).to(torch.int32)
    h = np.bitwise_xor.reduce(x.numpy().view(np.uint32), axis=1)
    if with_noise:
        h = h ^ np.bitwise_xor.reduce(nz.numpy().view(np.uint32), axis=1)
    codes = torch.full((max(bits, 1) * n,), 0x5A, dtype=torch.uint8, device="cuda")
    meta = torch.zeros(2 * ((n + 31) // 32), dtype=torch.int32, device="cuda")
    xd, nd = x.cuda(), nz.cuda()
    rc = L.dopt_stream_probe(xd.data_ptr(), nd.data_ptr() if with_noise else None, codes.data_ptr(), meta.data_ptr(),
                             n, bits, torch.cuda.current_stream().cuda_stream)
    probes.check(rc, "stream_probe")
    got = codes.cpu().numpy()
    if bits == 0:
        assert (got[1:] == 0x5A).all() and got[0] in (0x5A, 1)
        assert (got[0] == 1) == bool((h == 0x9E3779B9).any())
        return
    want = {1: h.astype(np.uint8), 2: h.astype(np.uint16), 4: h,
            8: np.stack([h, h >> np.uint32(7)], axis=1).reshape(-1)}[bits]
    np.testing.assert_array_equal(got.view(want.dtype), want)
    want_meta = np.stack([h[::32], h[::32] >> np.uint32(3)], axis=1).reshape(-1)
    np.testing.assert_array_equal(meta.cpu().numpy().view(np.uint32), want_meta)


def test_stream_probe_rejects_bad_arguments():
    L = probes.lib()
    buf = torch.zeros(64, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert L.dopt_stream_probe(buf.data_ptr(), None, buf.data_ptr(), buf.data_ptr(), 4, 3, s) == EINVAL
    assert L.dopt_stream_probe(buf.data_ptr() + 4, None, buf.data_ptr(), buf.data_ptr(), 4, 2, s) == EINVAL
    assert L.dopt_stream_probe(buf.data_ptr(), None, buf.data_ptr(), buf.data_ptr(), -1, 2, s) == EINVAL


@pytest.mark.parametrize("kind", [0, 1, 2, 3, 4, 5, 6, 7])
def test_valu_probe_runs(kind):
    """dopt_valu_probe (the instruction-cost probe the benchmark reports) launches, finishes and
    writes every output element."""
    L = probes.lib()
    sentinel = 0x7FC0DEAD  # a NaN payload the probe's chains do not produce
    out = torch.full((8 * 256,), sentinel, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert L.dopt_valu_probe(kind, out.data_ptr(), 8, s) == 0
    torch.cuda.synchronize()
    assert not (out == sentinel).any()
    if kind != 3:  # float chains and MFMA sums of values in (-1, 1) stay finite; kind 3 hashes bits
        assert torch.isfinite(out.view(torch.float32)).all()


def test_fast_exact_division_matches_ieee():
    """The quantizer's step = range / QMAX (multiply by the rounded reciprocal, one fma correction)
    and inv = 1 / step (v_rcp_f32 and one fma Newton step, the IEEE division for waves holding a
    subnormal or huge step) give the correctly rounded fp32 result for every non-negative fp32
    input: dopt_valu_probe kind 8 compares them with the division on all 2^31 + 1 bit patterns."""
    L = probes.lib()
    out = torch.full((4096 * 256,), -1.0, dtype=torch.float32, device="cuda")
    assert L.dopt_valu_probe(8, out.data_ptr(), 4096, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert not (out < 0).any()  # every thread reported
    assert int(out.sum().item()) == 0
