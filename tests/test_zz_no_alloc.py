"""dopt_bn_train_forward_noalloc (the allocation-free variant whose reduction partials live in a
static per-device scratch array) against dopt_bn_train_forward with a caller workspace, through
the C ABI: every output bit for bit.

* The file's first test makes the entry point's first call in the process inside a HIP graph
  capture (where its one-time scratch-address lookup happens), then replays the graph three
  times, each replay checked against the eager workspace entry point.
* Two calls in a row, the second with a smaller input (it reuses the scratch the first call left
  behind), for every mode: normalize with x_hat, quant-pack, ReLU and ReLU6 + quant-pack; bf16,
  fp16 and fp32 inputs.
* A shape with 65,536 partial slots (4096 channels of 8 chunks), and one that fills the scratch
  exactly: 1024 channels of 512 chunks, 2 * 1024 * 512 = 2^20 partial slots (2^32 elements).
The host-side rejection of shapes beyond the scratch is tested without a GPU
(tests/test_host_cpu.py)."""
import pytest
import torch

import deep_optimization_amd  # noqa: F401
from deep_optimization_amd import _lib
from deep_optimization_amd.graph import finalize

pytestmark = pytest.mark.gpu
DEV = "cuda"
MODES = {"norm": _lib.BN_NORM, "quant": _lib.BN_QUANT, "relu": _lib.BN_RELU_QUANT, "relu6": _lib.BN_RELU6_QUANT}
DTYPES = {torch.bfloat16: _lib.BF16, torch.float16: _lib.F16, torch.float32: _lib.F32}


def _outputs(N, C, HW, g, bits, mode):
    M = N * HW
    quant = mode != _lib.BN_NORM
    return {
        "y": torch.full((N, C, HW), 7, dtype=torch.int16, device=DEV),
        "x_hat": torch.full((N, C, HW) if not quant else (1,), 5, dtype=torch.int16, device=DEV),
        "packed": torch.full((C, M * bits // 32) if quant else (2,), -1, dtype=torch.int32, device=DEV),
        "relu": torch.full((C, M // 32) if mode in (_lib.BN_RELU_QUANT, _lib.BN_RELU6_QUANT) else (1,), -1,
                           dtype=torch.int32, device=DEV),
        "scale": torch.full((C, M // g) if quant else (1,), 3, dtype=torch.int16, device=DEV),
        "min": torch.full((C, M // g) if quant else (1,), 3, dtype=torch.int16, device=DEV),
        "mean": torch.full((C,), float("nan"), device=DEV),
        "var": torch.full((C,), float("nan"), device=DEV),
    }


def _written(mode):
    keys = ["y", "mean", "var"]
    if mode == _lib.BN_NORM:
        return keys + ["x_hat"]
    keys += ["packed", "scale", "min"]
    return keys + (["relu"] if mode != _lib.BN_QUANT else [])


def _launch(noalloc, x, N, C, HW, g, bits, mode, w, b, run_mean, run_var, o, ws=None):
    L = _lib.lib()
    quant = mode != _lib.BN_NORM
    relu = o["relu"].data_ptr() if mode in (_lib.BN_RELU_QUANT, _lib.BN_RELU6_QUANT) else None
    stream = torch.cuda.current_stream().cuda_stream
    rm = None if run_mean is None else run_mean.data_ptr()
    rv = None if run_var is None else run_var.data_ptr()
    tail = (o["y"].data_ptr(), None if quant else o["x_hat"].data_ptr(), o["packed"].data_ptr() if quant else None,
            relu, o["scale"].data_ptr() if quant else None, o["min"].data_ptr() if quant else None,
            o["mean"].data_ptr(), o["var"].data_ptr(), rm, rv, 0.1, stream)
    dt = DTYPES[x.dtype]
    if noalloc:
        return L.dopt_bn_train_forward_noalloc(x.data_ptr(), dt, N, C, HW, C * HW, HW, w.data_ptr(), b.data_ptr(),
                                               1e-5, mode, g, bits, *tail)
    return L.dopt_bn_train_forward(x.data_ptr(), dt, N, C, HW, C * HW, HW, ws.data_ptr(), w.data_ptr(),
                                   b.data_ptr(), 1e-5, mode, g, bits, *tail)


def _call(noalloc, x, N, C, HW, g, bits, mode, w, b, run_mean, run_var):
    o = _outputs(N, C, HW, g, bits, mode)
    ws = None
    if not noalloc:
        ws = torch.empty(_lib.lib().dopt_bn_workspace_floats(N, C, HW), dtype=torch.float32, device=DEV)
    rc = _launch(noalloc, x, N, C, HW, g, bits, mode, w, b, run_mean, run_var, o, ws)
    _lib.check(rc, "bn_train_forward_noalloc" if noalloc else "bn_train_forward")
    torch.cuda.synchronize()
    return o


def _inputs(N, C, H, W, dtype=torch.bfloat16):
    gen = torch.Generator(device=DEV).manual_seed(N + C + H)
    x = (torch.randn((N, C, H, W), generator=gen, device=DEV) * 2 + 0.5).to(dtype)
    w = torch.rand((C,), generator=gen, device=DEV) + 0.5
    b = torch.randn((C,), generator=gen, device=DEV)
    rm = torch.randn((C,), generator=gen, device=DEV)
    rv = torch.rand((C,), generator=gen, device=DEV) + 0.5
    return x, w, b, rm, rv


def test_first_call_under_graph_capture_then_replays():
    N, C, H, W, g, bits, mode = 16, 128, 28, 28, 256, 2, _lib.BN_RELU_QUANT
    print(f"[noalloc] graph capture of the first call: N={N} C={C} HW={H * W}", flush=True)
    x, w, b, _, _ = _inputs(N, C, H, W)
    want = _call(False, x, N, C, H * W, g, bits, mode, w, b, None, None)
    o = _outputs(N, C, H * W, g, bits, mode)
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    rcs = []
    with torch.cuda.graph(graph):
        rcs.append(_launch(True, x, N, C, H * W, g, bits, mode, w, b, None, None, o))
    assert rcs == [0], _lib.lib().dopt_last_error()
    assert finalize(graph) == 0  # the entry point records no memset
    for r in range(3):
        for k in _written(mode):  # scribble over every output between replays
            o[k].fill_(-3 if o[k].dtype != torch.float32 else float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k in _written(mode):
            assert torch.equal(o[k], want[k]), (r, k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "f16", "f32"])
@pytest.mark.parametrize("mode", sorted(MODES))
def test_noalloc_equals_workspace_entry_point_twice(mode, dtype):
    m = MODES[mode]
    # first call ResNet-like (2 x 256 x 13 partials), second smaller with another group size
    for (N, C, H, W, g, bits) in ((32, 256, 56, 56, 256, 2), (4, 32, 28, 28, 64, 4)):
        print(f"[noalloc] mode={mode} {dtype} N={N} C={C} HW={H * W} g={g} bits={bits}", flush=True)
        x, w, b, rm0, rv0 = _inputs(N, C, H, W, dtype)
        rm_a, rv_a, rm_b, rv_b = rm0.clone(), rv0.clone(), rm0.clone(), rv0.clone()
        want = _call(False, x, N, C, H * W, g, bits, m, w, b, rm_a, rv_a)
        got = _call(True, x, N, C, H * W, g, bits, m, w, b, rm_b, rv_b)
        for k in want:
            assert torch.equal(got[k], want[k]), k
        assert torch.equal(rm_a, rm_b) and torch.equal(rv_a, rv_b)
        assert bool(torch.isfinite(got["mean"]).all())


def test_noalloc_many_partial_slots():
    """C = 4096 channels of 8 chunks each: 65,536 partial slots (1/16 of the scratch)."""
    N, C, H, W, g, bits = 16, 4096, 64, 64, 256, 2
    assert _lib.lib().dopt_bn_workspace_floats(N, C, H * W) == 2 * C * 8
    print(f"[noalloc] partial slots: N={N} C={C} HW={H * W}", flush=True)
    x, w, b, rm0, rv0 = _inputs(N, C, H, W)
    rm_a, rv_a, rm_b, rv_b = rm0.clone(), rv0.clone(), rm0.clone(), rv0.clone()
    want = _call(False, x, N, C, H * W, g, bits, _lib.BN_QUANT, w, b, rm_a, rv_a)
    got = _call(True, x, N, C, H * W, g, bits, _lib.BN_QUANT, w, b, rm_b, rv_b)
    for k in want:
        assert torch.equal(got[k], want[k]), k
    assert torch.equal(rm_a, rm_b) and torch.equal(rv_a, rv_b)
    torch.testing.assert_close(got["mean"], x.float().mean(dim=(0, 2, 3)), rtol=1e-5, atol=1e-5)


def test_noalloc_at_the_scratch_limit():
    """C = 1024 channels of N * HW = 1024 * 4096 elements, 512 chunks of 8192 each: the statistics
    partials take 2 * 1024 * 512 = DOPT_BN_SCRATCH_FLOATS slots, the whole scratch (the last
    channel's sums of squares in its last slots). 2^32 bf16 elements: 8 GiB of input and 9 GiB of
    outputs per call. Every output bit for bit against the workspace entry point."""
    N, C, H, W, g, bits = 1024, 1024, 64, 64, 256, 2
    L = _lib.lib()
    assert L.dopt_bn_workspace_floats(N, C, H * W) == 2 * C * 512 == 1 << 20  # DOPT_BN_SCRATCH_FLOATS
    print(f"[noalloc] scratch limit: N={N} C={C} HW={H * W} ({N * C * H * W} elements)", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(11)
    x = torch.randn((N, C, H, W), generator=gen, device=DEV, dtype=torch.bfloat16)
    x.mul_(2).add_(0.5)
    w = torch.rand((C,), generator=gen, device=DEV) + 0.5
    b = torch.randn((C,), generator=gen, device=DEV)
    want = _call(False, x, N, C, H * W, g, bits, _lib.BN_QUANT, w, b, None, None)
    got = _call(True, x, N, C, H * W, g, bits, _lib.BN_QUANT, w, b, None, None)
    for k in _written(_lib.BN_QUANT):
        assert torch.equal(got[k], want[k]), k
    del want, got
    torch.cuda.empty_cache()
