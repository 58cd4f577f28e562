"""Captured training steps on the GPU (deep_optimization_amd.graph).

What is pinned and how:
  * dopt_graph_replace_memsets: a graph that records memsets of every kind HIP captures
    (bytes at an odd address, 16- and 32-bit elements, a pitched 2-D fill, a large contiguous fill)
    followed by a kernel reading the filled buffer holds no memset node after the rewrite, and
    every replay (fresh garbage written eagerly in between) leaves exactly the bytes the memsets
    define, also as seen by the dependent kernel: the fill kernels keep the memsets' edges;
  * Graph.capture_cuda_graph_qdrop (Activation_Compression/cuda_graph_utils.py:82-120) on a
    Controller-rewritten 2-block ViT: the captured graph holds no memset node; on each of three
    replays the injected noise has norm alpha * |p| and is fresh, the loss and the clipped
    gradients equal an eager step at the same perturbed weights (relative error <= 1e-3: the
    same kernels run, up to non-deterministic reductions in libraries), and with lr = 0 the
    weights come back to their values (one fp32 add and subtract);
  * a Controller-rewritten ResNet (compressed Conv / BatchNorm / ReLU beside torch's layers)
    captured as forward + loss + backward: three replays give an eager step's loss and gradients
    within 1e-5 relative, with MIOpen's deterministic solvers;
  * a DOConv2d with the PACT clamp in front, captured as forward + backward: no memset node, and
    three replays equal eager steps to 1e-5.
"""
import ctypes

import pytest
import torch
import torch.nn as nn

import deep_optimization_amd  # noqa: F401
from deep_optimization_amd.controller import Controller
from deep_optimization_amd.graph import Graph, finalize, graph_node_counts
from deep_optimization_amd.vit import VisionTransformer

pytestmark = pytest.mark.gpu
DEV = "cuda"


def hip_runtime():
    """The HIP runtime this process already uses (torch's), not a second copy."""
    with open("/proc/self/maps") as f:
        paths = {line.split()[-1] for line in f if "libamdhip64.so" in line}
    assert len(paths) == 1, paths
    hip = ctypes.CDLL(paths.pop())
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    hip.hipMemsetAsync.argtypes = [vp, ctypes.c_int, sz, vp]
    hip.hipMemsetD16Async.argtypes = [vp, ctypes.c_ushort, sz, vp]
    hip.hipMemsetD32Async.argtypes = [vp, ctypes.c_int, sz, vp]
    hip.hipMemset2DAsync.argtypes = [vp, sz, ctypes.c_int, sz, sz, vp]
    return hip


def test_memset_nodes_become_fill_kernels():
    hip = hip_runtime()
    n = 1 << 20
    buf = torch.empty(n, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(buf)
    base = buf.data_ptr()
    # (kind, byte offset, value, count or (pitch, width, height))
    fills = [("b", 3, 0xAB, 1001), ("h", 2048, 0x1234, 777), ("w", 8192, 0x5EADBEEF, 5000),
             ("2d", 65536, 0x5A, (1000, 333, 70)), ("b", 200001, 0x7F, 300000)]
    g = torch.cuda.CUDAGraph(keep_graph=True)
    stream = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=stream):
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for kind, off, val, cnt in fills:
            p = ctypes.c_void_p(base + off)
            if kind == "b":
                rc = hip.hipMemsetAsync(p, val, cnt, st)
            elif kind == "h":
                rc = hip.hipMemsetD16Async(p, val, cnt, st)
            elif kind == "w":
                rc = hip.hipMemsetD32Async(p, ctypes.c_int(val).value, cnt, st)
            else:
                rc = hip.hipMemset2DAsync(p, cnt[0], val, cnt[1], cnt[2], st)
            assert rc == 0, (kind, rc)
        out.copy_(buf)
    before = graph_node_counts(g)
    print("captured nodes:", before, flush=True)
    assert before.get("memset", 0) >= 1
    replaced = finalize(g)
    after = graph_node_counts(g)
    assert after.get("memset", 0) == 0 and replaced == before["memset"], (before, after)
    assert after["kernel"] == before.get("kernel", 0) + replaced

    def expected(garbage):
        e = garbage.clone()
        for kind, off, val, cnt in fills:
            if kind == "b":
                e[off:off + cnt] = val
            elif kind == "h":
                e[off:off + 2 * cnt].view(torch.int16)[:] = val
            elif kind == "w":
                e[off:off + 4 * cnt].view(torch.int32)[:] = ctypes.c_int(val).value
            else:
                pitch, width, height = cnt
                for r in range(height):
                    e[off + r * pitch:off + r * pitch + width] = val
        return e

    gen = torch.Generator().manual_seed(1)
    for r in range(3):
        garbage = torch.randint(0, 256, (n,), generator=gen, dtype=torch.uint8)
        buf.copy_(garbage.to(DEV))
        out.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        want = expected(garbage)
        assert torch.equal(buf.cpu(), want), r
        assert torch.equal(out.cpu(), want), r


def rel_err(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def test_graph_qdrop_step_matches_eager():
    torch.manual_seed(3)
    B, alpha = 32, 0.0375
    base = VisionTransformer(depth=2, num_classes=100).to(DEV)
    model = Controller(base, {"batch_size": B, "default_bits": 2}, input_shape=(3, 224, 224)).warp_model(quantizer=True)
    x = torch.randn(B, 3, 224, 224, device=DEV)
    y = torch.randint(0, 100, (B,), device=DEV)
    crit = nn.CrossEntropyLoss()
    opt = torch.optim.AdamW(model.parameters(), lr=0.0, capturable=True)  # lr 0: the weights keep their values
    gr = Graph(model, crit, opt, [(x, y)], None, "qdrop", 1)
    graphs, stream, sx, sy, logits, loss = gr.capture_cuda_graph_qdrop()
    counts = graph_node_counts(graphs[0])
    print("qdrop step graph:", counts, "memsets rewritten:", gr.memsets_replaced, flush=True)
    assert counts.get("memset", 0) == 0 and counts["kernel"] > 100
    assert torch.equal(sx, x) and torch.equal(sy, y)
    params = list(model.parameters())
    p0 = [p.detach().clone() for p in params]
    prev = None
    for r in range(3):
        opt.zero_grad(set_to_none=False)
        graphs[0].replay()
        torch.cuda.synchronize()
        noise = [p._theta.clone() for p in params]  # the buffer holds this replay's scaled noise
        g_graph = [p.grad.clone() for p in params]
        loss_graph = float(loss.detach())
        for q, nz in zip(p0, noise):
            qn = q.double().norm().item()
            assert abs(nz.double().norm().item() - alpha * qn) <= 1e-4 * alpha * qn + 1e-12
        if prev is not None:
            assert any(not torch.equal(a, b) for a, b in zip(noise, prev))
        for p, q, nz in zip(params, p0, noise):
            ulp = 2 * torch.finfo(torch.float32).eps * (q.abs() + nz.abs())
            assert bool(((p.detach() - q).abs() <= ulp).all())
        # eager step at the same perturbed weights
        with torch.no_grad():
            for p, q, nz in zip(params, p0, noise):
                p.copy_(q)
                p.add_(nz)
        opt.zero_grad(set_to_none=False)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss_e = crit(model(sx), sy)
        loss_e.backward()
        torch.nn.utils.clip_grad_norm_(params, max_norm=1.0)
        assert abs(float(loss_e) - loss_graph) <= 1e-3 * abs(float(loss_e)), (r, float(loss_e), loss_graph)
        for i, (p, gg) in enumerate(zip(params, g_graph)):
            if gg.any():
                assert rel_err(gg, p.grad) <= 1e-3, (r, i, rel_err(gg, p.grad))
        with torch.no_grad():
            for p, q in zip(params, p0):
                p.copy_(q)
        torch.cuda.synchronize()
        prev = noise


@pytest.fixture
def deterministic_miopen():
    """MIOpen's default convolution solvers are not deterministic: two eager backward passes of
    the same ResNet step differ by 5-10% in most weight gradients (plain model alike); with
    deterministic solvers they agree exactly, so graph and eager can be compared closely."""
    old = torch.backends.cudnn.deterministic
    torch.backends.cudnn.deterministic = True
    yield
    torch.backends.cudnn.deterministic = old


def test_compressed_resnet_step_replays_like_eager(deterministic_miopen):
    """A Controller-rewritten ResNet (one bottleneck per stage, batch 16, 224 x 224: the stem and
    the wide stage-1 tensors pass the 10 MiB rule, so compressed Conv / BatchNorm / ReLU layers
    and torch's run side by side) captured as forward + loss + backward: no memset node is left,
    and each of three replays gives the loss and the gradients of an eager step at the same
    weights (relative error <= 1e-5)."""
    from deep_optimization_amd.modules.normalization import DOBatchNorm2d
    from deep_optimization_amd.resnet import ResNet

    torch.manual_seed(4)
    B = 16
    model = Controller(ResNet((1, 1, 1, 1), num_classes=100).to(DEV), {"batch_size": B, "default_bits": 2},
                       input_shape=(3, 224, 224)).warp_model(quantizer=True)
    assert sum(isinstance(m, DOBatchNorm2d) for m in model.modules()) >= 3
    x = torch.randn(B, 3, 224, 224, device=DEV)
    y = torch.randint(0, 100, (B,), device=DEV)
    crit = nn.CrossEntropyLoss()
    params = list(model.parameters())

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = crit(model(x), y)
        loss.backward()
        return loss

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for p in params:
            p.grad = torch.zeros_like(p)
        step()  # warm-up on the capture stream (MIOpen picks its solvers here)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph(keep_graph=True)
    for p in params:
        p.grad.zero_()
    with torch.cuda.graph(g, stream=side):
        loss_static = step().detach()
    finalize(g)
    counts = graph_node_counts(g)
    print("resnet step graph:", counts, flush=True)
    assert counts.get("memset", 0) == 0 and counts["kernel"] > 100
    for r in range(3):
        for p in params:
            p.grad.zero_()
        g.replay()
        torch.cuda.synchronize()
        g_graph = [p.grad.clone() for p in params]
        loss_graph = float(loss_static)
        for p in params:
            p.grad.zero_()
        loss_e = float(step().detach())
        torch.cuda.synchronize()
        assert abs(loss_e - loss_graph) <= 1e-5 * abs(loss_e), (r, loss_e, loss_graph)
        for i, (p, gg) in enumerate(zip(params, g_graph)):
            if gg.any():
                assert rel_err(gg, p.grad) <= 1e-5, (r, i, rel_err(gg, p.grad))


def test_pact_conv_layer_replays_like_eager(deterministic_miopen):
    """A DOConv2d with the PACT clamp in front (pact_alpha) captured as forward + backward under
    bf16 autocast: the clamp's operators and its 1-bit mask pack make no host synchronisation and
    no memset node; each of three replays gives the eager step's output and the input and weight
    gradients (relative error <= 1e-5)."""
    from deep_optimization_amd.controller import layer_group_meta
    from deep_optimization_amd.layers import DOConv2d

    torch.manual_seed(5)
    shape = (8, 32, 32, 32)
    meta = {"conv": {"pack_only": False, "bits": 2, "AVG_ALAM": False, "ALAM_BITS": 0, "DIVISION": None,
                     **layer_group_meta(shape, 2)}}
    layer = DOConv2d(32, 64, 3, padding=1, target_name="conv", meta=meta, pact_alpha=1.0).to(DEV).train()
    x = torch.randn(shape, device=DEV).requires_grad_(True)
    dy = torch.randn(8, 64, 32, 32, device=DEV).to(torch.bfloat16)
    leaves = [x, layer.weight]

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = layer(x)
        y.backward(dy)
        return y

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for t in leaves:
            t.grad = torch.zeros_like(t)
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph(keep_graph=True)
    for t in leaves:
        t.grad.zero_()
    with torch.cuda.graph(g, stream=side):
        y_static = step().detach()
    finalize(g)
    assert graph_node_counts(g).get("memset", 0) == 0
    for r in range(3):
        for t in leaves:
            t.grad.zero_()
        g.replay()
        torch.cuda.synchronize()
        y_graph, g_graph = y_static.clone(), [t.grad.clone() for t in leaves]
        for t in leaves:
            t.grad.zero_()
        y_e = step().detach()
        torch.cuda.synchronize()
        assert rel_err(y_graph, y_e) <= 1e-5, r
        for gg, t in zip(g_graph, leaves):
            assert rel_err(gg, t.grad) <= 1e-5, (r, rel_err(gg, t.grad))
