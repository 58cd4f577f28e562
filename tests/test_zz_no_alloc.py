"""dopt_bn_train_forward_noalloc (the allocation-free variant whose reduction partials live in a
static per-device scratch array) against dopt_bn_train_forward with a caller workspace, through
the C ABI: every output bit for bit, on two calls in a row, the second with a smaller input (it
reuses the scratch the first call left behind). The host-side rejection of shapes beyond the
scratch is tested without a GPU (tests/test_host_cpu.py)."""
import pytest
import torch

import deep_optimization_amd  # noqa: F401
from deep_optimization_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _outputs(N, C, HW, g, bits, mode):
    M = N * HW
    return {
        "y": torch.full((N, C, HW), 7, dtype=torch.int16, device=DEV),
        "packed": torch.full((C, M * bits // 32), -1, dtype=torch.int32, device=DEV),
        "relu": torch.full((C, M // 32 if mode != _lib.BN_QUANT else 1), -1, dtype=torch.int32, device=DEV),
        "scale": torch.full((C, M // g), 3, dtype=torch.int16, device=DEV),
        "min": torch.full((C, M // g), 3, dtype=torch.int16, device=DEV),
        "mean": torch.full((C,), float("nan"), device=DEV),
        "var": torch.full((C,), float("nan"), device=DEV),
    }


def _call(noalloc, x, N, C, HW, g, bits, mode, w, b, run_mean, run_var):
    L = _lib.lib()
    o = _outputs(N, C, HW, g, bits, mode)
    relu = o["relu"].data_ptr() if mode != _lib.BN_QUANT else None
    stream = torch.cuda.current_stream().cuda_stream
    common_tail = (o["y"].data_ptr(), None, o["packed"].data_ptr(), relu, o["scale"].data_ptr(), o["min"].data_ptr(),
                   o["mean"].data_ptr(), o["var"].data_ptr(), run_mean.data_ptr(), run_var.data_ptr(), 0.1, stream)
    if noalloc:
        rc = L.dopt_bn_train_forward_noalloc(x.data_ptr(), _lib.BF16, N, C, HW, C * HW, HW, w.data_ptr(), b.data_ptr(),
                                              1e-5, mode, g, bits, *common_tail)
    else:
        ws = torch.empty(L.dopt_bn_workspace_floats(N, C, HW), dtype=torch.float32, device=DEV)
        rc = L.dopt_bn_train_forward(x.data_ptr(), _lib.BF16, N, C, HW, C * HW, HW, ws.data_ptr(), w.data_ptr(),
                                     b.data_ptr(), 1e-5, mode, g, bits, *common_tail)
    _lib.check(rc, "bn_train_forward_noalloc" if noalloc else "bn_train_forward")
    torch.cuda.synchronize()
    return o


@pytest.mark.parametrize("mode", ["quant", "relu"])
def test_noalloc_equals_workspace_entry_point_twice(mode):
    m = _lib.BN_QUANT if mode == "quant" else _lib.BN_RELU_QUANT
    # first call ResNet-like (2 x 256 x 13 partials), second smaller with another group size
    for (N, C, H, W, g, bits) in ((32, 256, 56, 56, 256, 2), (4, 32, 28, 28, 64, 4)):
        print(f"[noalloc] mode={mode} N={N} C={C} HW={H * W} g={g} bits={bits}", flush=True)
        gen = torch.Generator(device=DEV).manual_seed(N + C)
        x = (torch.randn((N, C, H, W), generator=gen, device=DEV) * 2 + 0.5).to(torch.bfloat16)
        w = torch.rand((C,), generator=gen, device=DEV) + 0.5
        b = torch.randn((C,), generator=gen, device=DEV)
        rm0 = torch.randn((C,), generator=gen, device=DEV)
        rv0 = torch.rand((C,), generator=gen, device=DEV) + 0.5
        rm_a, rv_a, rm_b, rv_b = rm0.clone(), rv0.clone(), rm0.clone(), rv0.clone()
        want = _call(False, x, N, C, H * W, g, bits, m, w, b, rm_a, rv_a)
        got = _call(True, x, N, C, H * W, g, bits, m, w, b, rm_b, rv_b)
        for k in want:
            assert torch.equal(got[k], want[k]), k
        assert torch.equal(rm_a, rm_b) and torch.equal(rv_a, rv_b)
        assert bool(torch.isfinite(got["mean"]).all())

