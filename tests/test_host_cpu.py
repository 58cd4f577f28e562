"""CPU-only tests of the boundary and the host logic (no kernel is launched).

* libdopt.so loads and exports exactly the functions include/dopt.h declares;
* argument validation runs before any HIP call and maps to the reference's exception types;
* the act_lib operators have correct fake (meta) implementations;
* module_utils reproduces the reference's 14-field meta tuple and output shapes (run under
  FakeTensorMode, so the operators resolve to their fake kernels);
* the group-layout helpers round-trip and match a brute-force restatement.
"""
import ctypes
import os
import re

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import deep_optimization_amd  # noqa: F401
from deep_optimization_amd import _lib, act_lib
from deep_optimization_amd.modules import module_utils as mu
from deep_optimization_amd.modules import tensor_act_reshape_utils as tr

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dopt.h")

needs_lib = pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="libdopt.so not built")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(dopt_\w+)\s*\(", text, re.M)))


def test_header_declares_the_binding_exports():
    assert header_functions() == sorted(_lib.EXPORTS)


@needs_lib
def test_library_exports_every_declared_symbol():
    L = ctypes.CDLL(_lib.LIB_PATH)
    for name in header_functions():
        assert hasattr(L, name), name
    assert _lib.lib().dopt_abi_version() == 1


@needs_lib
class TestValidationWithoutDevice:
    """Every check below fails before the library touches HIP, so it runs without a GPU."""

    def qp(self, **kw):
        a = dict(x=16, x_dtype=_lib.BF16, n=4, g=256, bits=2, tile=None, rn=0, noise=None, seed=0, off=0,
                 flags=0, alpha=0.0, packed=16, scale=16, minv=16, meta=_lib.F32, stream=None)
        a.update(kw)
        return _lib.lib().dopt_quant_pack(a["x"], a["x_dtype"], a["n"], a["g"], a["bits"], a["tile"], a["rn"],
                                          a["noise"], a["seed"], a["off"], a["flags"], a["alpha"], a["packed"],
                                          a["scale"], a["minv"], a["meta"], a["stream"])

    def test_bad_bits_is_value_error(self):
        assert self.qp(bits=3) == _lib.EBITS
        with pytest.raises(ValueError, match="bits must be one of"):
            _lib.check(self.qp(bits=3), "quant_pack")

    @pytest.mark.parametrize("g", [0, 32, 100, 2048])
    def test_bad_group_size(self, g):
        assert self.qp(g=g) == _lib.EINVAL
        assert "group_size" in _lib.lib().dopt_last_error().decode()

    def test_bad_dtype_meta_rounding_flags(self):
        assert self.qp(x_dtype=7) == _lib.EINVAL
        assert self.qp(meta=_lib.F16) == _lib.EINVAL
        assert self.qp(rn=5) == _lib.EINVAL
        assert self.qp(flags=8) == _lib.EINVAL

    def test_noise_mode_needs_noise(self):
        assert self.qp(rn=_lib.ROUND_STOCH_NOISE) == _lib.EINVAL

    def test_alignment_and_nulls(self):
        assert self.qp(x=None) == _lib.EINVAL
        assert self.qp(x=8) == _lib.EINVAL
        assert self.qp(packed=4) == _lib.EINVAL

    def test_tile_checks(self):
        T = ctypes.c_int64 * 4
        assert self.qp(g=128, tile=T(1, 1, 22, 22), n=4) == _lib.EINVAL  # not a square group
        assert self.qp(g=256, tile=T(1, 1, 24, 32), n=2) == _lib.EINVAL  # H % 16 != 0
        assert self.qp(g=256, tile=T(1, 2, 32, 32), n=3) == _lib.EINVAL  # wrong n_groups
        assert "n_groups" in _lib.lib().dopt_last_error().decode()

    def test_empty_is_a_no_op(self):
        assert self.qp(n=0, x=None, packed=None) == _lib.OK
        L = _lib.lib()
        assert L.dopt_dequant_unpack(None, None, None, _lib.F32, 0, 256, 2, None, None, _lib.BF16, None) == 0
        assert L.dopt_pack_codes(None, 0, 64, 1, None, None) == 0
        assert L.dopt_fp8_gemm_nt(None, None, 0, 256, 128, 128, 128, 1.0, None, 256, None) == 0

    def test_dequant_and_codes_validation(self):
        L = _lib.lib()
        assert L.dopt_dequant_unpack(16, 16, 16, _lib.F32, 4, 256, 3, None, 16, _lib.BF16, None) == _lib.EBITS
        assert L.dopt_dequant_unpack(16, 16, 16, _lib.F32, 4, 256, 2, None, 16, _lib.F16, None) == _lib.EINVAL
        assert L.dopt_pack_codes(16, 4, 64, 5, 16, None) == _lib.EBITS
        assert L.dopt_unpack_codes(16, 4, 48, 2, 16, None) == _lib.EINVAL

    def test_bn_noalloc_rejects_shapes_beyond_the_scratch(self):
        L = _lib.lib()
        N, C, HW = 1024, 2048, 56 * 56  # 2 * 2048 * 392 partials: more than the 2^20 floats of scratch
        assert L.dopt_bn_workspace_floats(N, C, HW) > (1 << 20)
        assert L.dopt_bn_workspace_floats(128, C, HW) <= (1 << 20)
        rc = L.dopt_bn_train_forward_noalloc(16, _lib.BF16, N, C, HW, C * HW, HW, 16, 16, 1e-5, _lib.BN_QUANT, 256, 2,
                                             16, None, 16, None, 16, 16, 16, 16, None, None, 0.1, None)
        assert rc == _lib.EINVAL
        msg = L.dopt_last_error().decode()
        assert "scratch" in msg and "1048576" in msg, msg

    def test_bn_alam_rejects_run_lengths_the_reference_cannot_reshape(self):
        L = _lib.lib()
        N, C, HW = 4, 2, 64  # groups of 64 at 2 bits: 4 code words per group
        for alam in (0, 3, 8):  # not a power of two dividing 4
            rc = L.dopt_bn_norm_quant_alam(16, _lib.BF16, N, C, HW, C * HW, HW, 16, 16, None, None, 0, 16, 16, 1e-5,
                                           64, 2, alam, 16, 16, 16, 16, 16, 16, None)
            assert rc == _lib.EINVAL and "alam_bits" in L.dopt_last_error().decode()
            assert L.dopt_bn_bwd_reduce_alam(16, 16, 16, 16, _lib.BF16, N, C, HW, C * HW, HW, 64, 2, alam, 16, 16,
                                             16, None) == _lib.EINVAL
            assert L.dopt_bn_bwd_dx_alam(16, 16, 16, 16, _lib.BF16, N, C, HW, C * HW, HW, 64, 2, alam, 16, 16, 16,
                                         16, 1e-7, 0, 16, None) == _lib.EINVAL
        assert L.dopt_bn_norm_quant_alam(16, _lib.BF16, N, C, HW, C * HW, HW, 16, 16, None, None, 0, 16, 16, 1e-5,
                                         64, 3, 2, 16, 16, 16, 16, 16, 16, None) == _lib.EBITS

    def test_act_dequant_mul_alam_argument_checks(self):
        L = _lib.lib()
        assert L.dopt_act_dequant_mul_alam(16, 16, 16, _lib.BF16, 4, 256, 3, None, 16, _lib.BF16, 42, 16,
                                           None) == _lib.EBITS
        assert L.dopt_act_dequant_mul_alam(16, 16, 16, _lib.BF16, 4, 256, 2, None, 16, _lib.F16, 42, 16,
                                           None) == _lib.EINVAL  # dy must be F32 or BF16
        assert L.dopt_act_dequant_mul_alam(16, 16, 16, _lib.F16, 4, 256, 2, None, 16, _lib.BF16, 42, 16,
                                           None) == _lib.EINVAL  # scale / min F32 or BF16
        assert L.dopt_act_dequant_mul_alam(None, 16, 16, _lib.BF16, 4, 256, 2, None, 16, _lib.BF16, 42, 16,
                                           None) == _lib.EINVAL  # null codes
        assert L.dopt_act_dequant_mul_alam(16, 16, 16, _lib.BF16, 0, 256, 2, None, 16, _lib.BF16, 42, 16,
                                           None) == _lib.OK  # nothing to do

    def test_gemm_shape_checks(self):
        L = _lib.lib()
        assert L.dopt_fp8_gemm_nt(16, 16, 100, 256, 120, 128, 128, 1.0, 16, 256, None) == _lib.EUNSUPPORTED  # K % 16
        assert L.dopt_fp8_gemm_nt(16, 16, 256, 256, 128, 64, 128, 1.0, 16, 256, None) == _lib.EINVAL  # lda < K
        assert L.dopt_fp8_gemm_nt(16, 16, 256, 256, 128, 136, 128, 1.0, 16, 256, None) == _lib.EINVAL  # lda % 16
        assert L.dopt_fp8_gemm_nt(8, 16, 256, 256, 128, 128, 128, 1.0, 16, 256, None) == _lib.EINVAL  # A unaligned
        assert L.dopt_fp8_gemm_nt(16, 16, 256, 250, 128, 128, 128, 1.0, 16, 249, None) == _lib.EINVAL  # ldc < N
        assert L.dopt_fp8_gemm_nt(16, 16, 256, 256, 128, 1 << 24, 128, 1.0, 16, 256, None) == _lib.EINVAL  # lda > 2^23
        # a 256-row tile at lda = 2^23 would reach offset 2^31 - 1, past the buffer range
        assert L.dopt_fp8_gemm_nt(16, 16, 256, 256, 128, 1 << 23, 128, 1.0, 16, 256, None) == _lib.EINVAL


def test_bits_consts_contract():
    assert act_lib._bits_consts(2, 256) == (16, 16, 3)
    assert act_lib._bits_consts(8, 64) == (4, 16, 255)
    with pytest.raises(ValueError):
        act_lib._bits_consts(3, 256)


def test_ops_reject_cpu_tensors():
    x = torch.zeros(1, 2, 256)
    with pytest.raises(NotImplementedError):
        torch.ops.act_lib.quant_pack_triton(x, 2, 256, False, 0, True, 3.0)


# ----------------------------------------------------------------------------- fake kernels
def test_fake_shapes():
    with FakeTensorMode():
        x = torch.empty(3, 5, 128, dtype=torch.bfloat16, device="cuda")
        p, s, m = torch.ops.act_lib.quant_pack_triton(x, 4, 128, False, 0, True, 3.0)
        assert p.shape == (15, 16) and p.dtype == torch.int32
        assert s.shape == (3, 5) and s.dtype == torch.bfloat16 and m.dtype == torch.bfloat16
        y = torch.ops.act_lib.dequant_unpack_triton(p, s, m, 4, 128, False, 0)
        assert y.shape == (3, 5, 128) and y.dtype == torch.bfloat16
        p, s, m = torch.ops.act_lib.quant_pack(x, 1, 128, False, 0.0, False, 2, None, 1, 2, torch.float32)
        assert p.shape == (15, 4) and s.dtype == torch.float32
        x4 = torch.empty(2, 3, 32, 48, dtype=torch.float32, device="cuda")
        p, s, m = torch.ops.act_lib.quant_pack_tiles(x4, 2, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
        assert p.shape == (2 * 3 * 2 * 3, 16) and s.shape == (2, 18)
        y = torch.ops.act_lib.dequant_unpack_tiles(p, s, m, 2, 256, 2, 3, 32, 48, torch.bfloat16)
        assert y.shape == (2, 3, 32, 48)
        c = torch.empty(2, 4, 64, dtype=torch.int8, device="cuda")
        w = torch.ops.act_lib.pack_triton(c, 1, 64)
        assert w.shape == (8, 2) and w.dtype == torch.int32
        assert torch.ops.act_lib.unpack_triton(w, 1, 2, 4, 64).shape == (2, 4, 64)
        a = torch.empty(256, 512, dtype=torch.float8_e4m3fn, device="cuda")
        b = torch.empty(768, 512, dtype=torch.float8_e4m3fn, device="cuda")
        assert torch.ops.act_lib.fp8_gemm_nt(a, b, 1.0).shape == (256, 768)


# ----------------------------------------------------------------------------- module_utils meta tuple
def _meta(bits, group_size, act_padding, N, pack_only=False):
    return {"layer": {"bits": bits, "pack_only": pack_only, "group_size": group_size, "act_padding": act_padding,
                      "N": N, "AVG_ALAM": False, "ALAM_BITS": 0}}


@pytest.mark.parametrize("shape,g,pad,expect", [
    # flat 4-D (56 % 16 != 0): reference meta (bits, False, g, False, N, G, 0, 0, False, False, False, ...)
    ((4, 8, 56, 56), 256, False, dict(G=8 * 56 * 56 // 256, nh=0, nw=0, pe=False, re=False)),
    # tiles (32 % 16 == 0): new_H = new_W = 2, reshape_eligibility True
    ((4, 8, 32, 32), 256, False, dict(G=8 * 4, nh=2, nw=2, pe=False, re=True)),
    # non-square tiles
    ((2, 3, 16, 48), 64, False, dict(G=3 * 2 * 6, nh=2, nw=6, pe=False, re=True)),
    # 3-D token activations: always flat
    ((2, 197, 768), 128, False, dict(G=197 * 768 // 128, nh=0, nw=0, pe=False, re=False)),
    # act_padding: zero-padded per sample to a multiple of g
    ((3, 5, 7, 7), 256, True, dict(G=(5 * 49 + 255) // 256, nh=0, nw=0, pe=False, re=False)),
])
def test_quantize_meta_tuple_matches_reference(shape, g, pad, expect):
    with FakeTensorMode():
        x = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
        meta = _meta(2, g, pad, shape[0])
        (p, s, m), qm, l = mu.unified_quantize(x, None, "layer", meta, True, 3.0)
        N = shape[0]
        assert qm == (2, False, g, pad, N, expect["G"], expect["nh"], expect["nw"], expect["pe"], expect["re"],
                      False, False, 0, x.shape)
        assert p.shape == (N * expect["G"], g * 2 // 32) and s.shape == (N, expect["G"])
        y = mu.unified_dequantize((p, s, m), qm, None)
        assert y.shape == x.shape and y.dtype == torch.bfloat16


def test_quantize_pack_only_meta():
    with FakeTensorMode():
        x = torch.empty(2, 3, 7, 7, dtype=torch.int8, device="cuda")
        meta = _meta(1, 64, True, 2, pack_only=True)
        (p, s, m), qm, _ = mu.unified_quantize(x, None, "layer", meta, False, 0.0)
        assert s is None and m is None
        G = (3 * 49 + 63) // 64
        assert qm == (1, True, 64, True, 2, G, 0, 0, False, False, False, None, None, x.shape)
        y = mu.unified_dequantize((p, s, m), qm, None)
        assert y.shape == x.shape and y.dtype == torch.int8


def test_quantize_pack_only_tile_meta_inverts_the_grouping():
    """A 1-bit mask grouped into spatial tiles (32x32 maps, 8x8 tiles) keeps its tile flags in the meta,
    so the restore puts every bit back at its element. The reference's pack-only meta
    (module_utils.py:40,55) records (0, 0, False, False) here, and its restore returns the tile-ordered
    codes in flat order: a deliberate deviation, pinned by the brute-force inverse below."""
    shape, g = (2, 3, 32, 32), 64
    with FakeTensorMode():
        x = torch.empty(shape, dtype=torch.int8, device="cuda")
        (p, s, m), qm, _ = mu.unified_quantize(x, None, "layer", _meta(1, g, False, 2, pack_only=True), False, 1.0)
        assert s is None and m is None and p.shape == (2 * 3 * 16, g // 32)
    assert qm[:11] == (1, True, g, False, 2, 3 * 16, 4, 4, False, True, False)
    x = (torch.rand(shape, generator=torch.Generator().manual_seed(0)) < 0.5).to(torch.int8)
    groups = tr.spatical_aware_act_tensor_reshape(x, g, False, True)[0]
    # group j of sample n holds the 8x8 tile (c, th, tw) = divmod over (C, 4, 4), row-major inside
    c, th, tw = 1, 2, 3
    assert torch.equal(groups[1, (c * 4 + th) * 4 + tw].view(8, 8), x[1, c, 8 * th:8 * th + 8, 8 * tw:8 * tw + 8])
    back = tr.spatical_aware_act_tensor_reshape_back(groups, shape, g, qm[6], qm[7], qm[3], qm[8], qm[9], qm[10])
    assert torch.equal(back, x)


def test_non_square_group_with_divisible_map_raises():
    x = torch.zeros(1, 2, 22, 22)
    with pytest.raises(RuntimeError, match="square group size"):
        tr.spatical_aware_act_tensor_reshape(x, 128, False, False)


# ----------------------------------------------------------------------------- layout helpers
@pytest.mark.parametrize("shape,g", [((2, 3, 16, 16), 64), ((2, 3, 32, 64), 256), ((1, 2, 8, 40), 64),
                                     ((2, 3, 10, 10), 64), ((4, 100), 64), ((2, 5, 33), 128)])
@pytest.mark.parametrize("pad", [False, True])
def test_layout_round_trip(shape, g, pad):
    x = torch.randn(shape)
    numel = x[0].numel()
    if not pad and numel % g:
        # the flat layout without padding needs g | features: the reference's reshape(N, -1, g)
        # (tensor_act_reshape_utils.py:46) raises, and so does this one
        with pytest.raises(RuntimeError, match="is invalid for input of size"):
            tr.spatical_aware_act_tensor_reshape(x, g, pad, False)
        return
    groups, N, G, nh, nw, ori, pe, re_, cm = tr.spatical_aware_act_tensor_reshape(x, g, pad, False)
    assert groups.shape == (N, G, g)
    back = tr.spatical_aware_act_tensor_reshape_back(groups, ori, g, nh, nw, pad, pe, re_, cm)
    assert torch.equal(back, x)


def test_tile_groups_brute_force():
    N, C, H, W, s = 1, 2, 16, 24, 8
    x = torch.arange(N * C * H * W, dtype=torch.float32).reshape(N, C, H, W)
    groups = tr.spatical_aware_act_tensor_reshape(x, s * s, False, False)[0][0]
    r = 0
    for c in range(C):
        for th in range(H // s):
            for tw in range(W // s):
                want = torch.tensor([float(x[0, c, th * s + i, tw * s + j]) for i in range(s) for j in range(s)])
                assert torch.equal(groups[r], want)
                r += 1


def test_padding_zero_fills():
    x = torch.ones(2, 3, 5)
    groups, N, G, *_ = tr.spatical_aware_act_tensor_reshape(x, 64, True, False)
    assert G == 1 and groups.shape == (2, 1, 64)
    assert torch.equal(groups[:, 0, :15], torch.ones(2, 15)) and torch.count_nonzero(groups[:, 0, 15:]) == 0


# ----------------------------------------------------------------------------- per-layer group meta
class TestLayerGroupMeta:
    """Known answers worked out by hand from the rule of controller.py:364-378 (first of
    [512, 256, 128, 64], or [1024, ...] for BatchNorm, dividing the grouped extent; else 256 with
    padding) and the N/G arithmetic of controller.py:127-177."""

    def test_find_group_size_known_answers(self):
        from deep_optimization_amd.controller import find_group_size

        assert find_group_size(256 * 56 * 56, 2) == (512, False)  # ResNet conv2 activation per sample
        assert find_group_size(197 * 3072, 2) == (512, False)  # ViT MLP activation per sample
        assert find_group_size(64 * 3 * 3 * 2, 4) == (128, False)  # 1152 = 2^7 * 9
        assert find_group_size(64 * 3, 8) == (64, False)
        assert find_group_size(100, 1) == (256, True)  # no power of two >= 64 divides 100
        assert find_group_size(1024 * 7, 2, special=True) == (1024, False)
        assert find_group_size(1024 * 7, 2) == (512, False)
        assert find_group_size(512, 3) == (256, True)  # bits outside {1,2,4,8} fall through

    def test_layer_group_meta_shapes(self):
        from deep_optimization_amd.controller import layer_group_meta

        m = layer_group_meta((256, 256, 56, 56), 2)
        assert m == {"group_size": 512, "act_padding": False, "N": 256, "NG": 256 * 1568}
        m = layer_group_meta((256, 197, 3072), 2)
        assert m == {"group_size": 512, "act_padding": False, "N": 256, "NG": 256 * 1182}
        m = layer_group_meta((256, 64, 56, 56), 2, batchnorm=True)  # per channel: N*H*W = 802816
        assert m == {"group_size": 1024, "act_padding": False, "N": 64, "NG": 64 * 784}
        m = layer_group_meta((32, 100), 1)
        assert m == {"group_size": 256, "act_padding": True, "N": 32, "NG": 32}
        m = layer_group_meta((8, 64, 32, 32), 2)  # the reference's CPU case's shape
        assert m["group_size"] == 512 and m["NG"] == 8 * 128

    def test_activation_size(self):
        from deep_optimization_amd.controller import compute_activation_size_in_bytes

        assert compute_activation_size_in_bytes((256, 256, 56, 56), torch.bfloat16) == 256 * 256 * 56 * 56 * 2 / 2 ** 20
