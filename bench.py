"""Benchmark of the activation-compression hot path on one MI355X.

A step is one forward save + backward restore of the benchmark's config 2, the ResNet-50 conv2
activation: bf16 [256, 256, 56, 56] post-ReLU |N(0,1)| (synthetic, seed 0), group size 256,
2-bit stochastic rounding with a seeded uniform [0, 1) noise tensor (seed 1) resident in HBM:
act_lib::quant_pack (pack) then act_lib::dequant_unpack back to bf16 (unpack), both through the
public torch operators. `value` is algorithmic bytes per step / wall time per step:
    pack   = 2 B (bf16 in) + 4 B (fp32 noise) + 2/8 B (codes) per element + 8 B per group
    unpack = 2/8 B + 8 B per group + 2 B (bf16 out) per element
The JSON line also carries the dominant kernel's roofline (quant-pack, HIP-event timed on the
stream it is launched on), the CPU oracle timed on the host cores (cpu_baseline), and extras:
the Philox and nearest rounding modes of the same step, a HIP-graph replay of the step, the ViT
MLP bit-width sweep (config 3), the fused activation layers, the FP8 GEMM (config 4) beside
hipBLASLt on the same data, the compressed Linear layers' weight-gradient GEMM at the ViT-B/16
shapes, the compressed BatchNorm layer, the ViT-B/16 train step (config 5): plain vs 2-bit,
the ResNet-50 train step (plain vs compressed Conv/BatchNorm/ReLU, eager and graph-replayed),
and the captured weight-noise step replayed from one HIP graph vs run eagerly.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras] [--no-cpu]
       python bench.py --pmc-probe   (one copy kernel + the dominant kernel, for rocprofv3 --pmc)
       python bench.py --fp8-probe random|constant   (the 8192^3 FP8 GEMM alone, for rocprofv3 --pmc)
       python bench.py --dw-probe [--dw-tokens K1,K2,...]   (three weight-gradient GEMMs at the ViT fc1
                   shape, for rocprofv3 --pmc; with --dw-tokens, five at each token count, a K sweep
                   under rocprofv3 --kernel-trace)
"""
from __future__ import annotations

import argparse
import json
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
SETTLE_S = 0.025  # sustained-load warm-up before every timed extra (seconds of wall time)
METRIC = "quant-pack+unpack GB/s (% HBM peak) at 2-bit; FP8 GEMM TFLOPS (% peak)"
PMC_SUMMARY = os.path.join(ROOT, "profiles", "quant_pack_resnet_noise_pmc.md")
N, C, H, W = 256, 256, 56, 56
G_SIZE, BITS = 256, 2
NEAREST, NOISE, PHILOX = 0, 1, 2


_T0 = time.perf_counter()


def progress(msg: str) -> None:
    """A progress line on stderr (the JSON result is the only stdout line), with the seconds elapsed."""
    print(f"[bench {time.perf_counter() - _T0:6.1f}s] {msg}", file=sys.stderr, flush=True)


def pack_bytes(n_elem, n_groups, in_bytes, bits, noise=False):
    return n_elem * in_bytes + n_elem * bits // 8 + n_groups * 8 + (n_elem * 4 if noise else 0)


def unpack_bytes(n_elem, n_groups, out_bytes, bits):
    return n_elem * bits // 8 + n_groups * 8 + n_elem * out_bytes


def read_traffic():
    """HBM bytes per quant-pack launch from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (each scaled by
    the same counter's reading for a copy kernel of known size), recorded in the committed summary."""
    try:
        text = open(PMC_SUMMARY).read()
    except OSError:
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", text)
    return int(m.group(1)) if m else None


def resnet_inputs(torch, dev):
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((N, C, H, W), generator=gen, device=dev, dtype=torch.float32).abs_().to(torch.bfloat16)
    noise = torch.rand((N, C * H * W // G_SIZE, G_SIZE), generator=torch.Generator(device=dev).manual_seed(1),
                       device=dev)
    return x, noise


def batchnorm_layer(torch, dev, event_avg, shape=(256, 256, 56, 56), block=1024, bits=2):
    """The compressed BatchNorm on a ResNet-50 stage-1 activation (bf16, per-channel groups of
    block // 2, 2-bit): statistics, normalize + quant-pack (squashed, and fused with ReLU), the
    backward reduce and input gradient, each against its algorithmic bytes; beside torch's
    BatchNorm (MIOpen) forward + backward on the same tensor, which saves the full input."""
    ops = torch.ops.act_lib
    N, C, H, W = shape
    HW, M = H * W, N * H * W
    E = N * C * HW
    g = dict(M=M, HW=HW, stride_n=C * HW, stride_c=HW)
    gen = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn((N, C, HW), generator=gen, device=dev).to(torch.bfloat16)
    dy = torch.randn((N, C, HW), generator=gen, device=dev).to(torch.bfloat16)
    w = torch.rand(C, generator=gen, device=dev) + 0.5
    b = torch.randn(C, generator=gen, device=dev)
    ng = E // (block // 2)
    frac = lambda nbytes, t: round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)  # noqa: E731
    s_, q_ = ops.bn_fwd_reduce(x, **g, BLOCK_M=block, num_warps=8, num_stages=5)
    t_st = event_avg(lambda: ops.bn_fwd_reduce(x, **g, BLOCK_M=block, num_warps=8, num_stages=5))
    res = {"shape": list(shape), "group": block // 2, "bits": bits,
           "stats": {"us": round(t_st * 1e6, 1), "frac": frac(2 * E, t_st)}}
    for mode in ("squash", "relu"):
        if mode == "squash":
            def fwd():
                return ops.bn_fwd_norm_quant_pack_fused(x, s_, q_, w, b, None, None, **g, BLOCK_M=block, bits=bits,
                                                        sync=False, avg_alam=False, alam_bits=0, num_warps=8,
                                                        num_stages=5)
            o = fwd()
            packed, scale, mn, var = o[1], o[2], o[3], o[5]

            def red():
                return ops.bn_bwd_reduce_dequant_unpack_fused(packed, dy, scale, mn, **g, BLOCK_M=block, bits=bits,
                                                              avg_alam=False, alam_bits=0)
            dw, db = red()

            def dx():
                return ops.bn_bwd_dx_dequant_unpack_fused(packed, dy, scale, mn, dw, db, w, var, **g, BLOCK_M=block,
                                                          bits=bits, sync=False, avg_alam=False, alam_bits=0)
            side = E * bits / 8 + ng * 4
        else:
            def fwd():
                return ops.bn_relu_fwd_norm_fused_quant_pack(x, s_, q_, w, b, None, None, **g, relu=True, relu6=False,
                                                             BLOCK_SIZE=block, BITS=bits, sync=False)
            o = fwd()
            packed, rp, scale, mn, var = o[1], o[2], o[3], o[4], o[6]

            def red():
                return ops.bn_relu_bwd_reduce_fused_dequant_unpack(packed, rp, dy, scale, mn, **g, BLOCK_SIZE=block,
                                                                   BITS=bits)
            dw, db = red()

            def dx():
                return ops.bn_relu_bwd_dx_fused_dequant_unpack(packed, rp, dy, dw, db, w, var, scale, mn, **g,
                                                               BLOCK_SIZE=block, BITS=bits)
            side = E * bits / 8 + E / 8 + ng * 4
        tf, tr, tx = event_avg(fwd), event_avg(red), event_avg(dx)
        res[mode] = {"fwd_us": round(tf * 1e6, 1), "fwd_frac": frac(4 * E + side, tf),
                     "bwd_reduce_us": round(tr * 1e6, 1), "bwd_reduce_frac": frac(2 * E + side, tr),
                     "bwd_dx_us": round(tx * 1e6, 1), "bwd_dx_frac": frac(4 * E + side, tx),
                     "layer_fwd_bwd_us": round((t_st + tf + tr + tx) * 1e6, 1)}
        del o
    xx = x.view(N, C, H, W).clone().requires_grad_(True)
    dy4 = dy.view(N, C, H, W)

    def torch_bn():
        torch.nn.functional.batch_norm(xx, None, None, w, b, True, 0.1, 1e-5).backward(dy4)
    res["torch_batchnorm_fwd_bwd_us"] = round(event_avg(torch_bn) * 1e6, 1)
    return res


def vit_train_step(torch, dev, batch=128, steps=6, warmup=3):
    """Config 5: one ViT-B/16 train step (forward, cross-entropy, backward, fused AdamW step)
    on a fixed synthetic batch (N(0,1) images 224x224x3, random labels over 1000 classes, bf16
    autocast, random-init weights), plain and rewritten by the Controller with every selected saved
    activation 2-bit. Reports ms per step and the peak HBM allocated during the timed steps."""
    import torch.nn.functional as F

    from deep_optimization_amd.controller import Controller
    from deep_optimization_amd.vit import vit_base_patch16_224

    res = {}
    g = torch.Generator(device=dev).manual_seed(5)
    xb = torch.randn((batch, 3, 224, 224), generator=g, device=dev)
    yb = torch.randint(0, 1000, (batch,), generator=g, device=dev)
    for name in ("plain", "compressed_2bit"):
        torch.manual_seed(0)
        model = vit_base_patch16_224().to(dev).train()
        if name != "plain":
            ctl = Controller(model, {"batch_size": batch, "default_bits": 2}, input_shape=(3, 224, 224))
            model = ctl.warp_model(quantizer=True)
        opt = torch.optim.AdamW(model.parameters(), lr=3e-3, fused=True)

        def one():
            opt.zero_grad(set_to_none=True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = F.cross_entropy(model(xb), yb)
            loss.backward()
            opt.step()
            return loss

        for _ in range(warmup):
            one()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base_alloc = torch.cuda.memory_allocated()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = one()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        res[name] = {"ms_per_step": round(dt * 1e3, 2), "samples_per_s": round(batch / dt, 1),
                     "peak_hbm_GiB": round(torch.cuda.max_memory_allocated() / 2 ** 30, 3),
                     "peak_above_resident_GiB": round((torch.cuda.max_memory_allocated() - base_alloc) / 2 ** 30, 3),
                     "loss": round(float(loss.detach()), 4)}
        if name != "plain":
            res[name]["layers_compressed"] = sum(1 for v in ctl.meta.values() if isinstance(v, dict))
        del model, opt
        torch.cuda.empty_cache()
    p, c = res["plain"], res["compressed_2bit"]
    res["compressed_vs_plain"] = {"step_time_ratio": round(c["ms_per_step"] / p["ms_per_step"], 3),
                                  "peak_hbm_ratio": round(c["peak_hbm_GiB"] / p["peak_hbm_GiB"], 3),
                                  "peak_above_resident_ratio": round(c["peak_above_resident_GiB"]
                                                                     / p["peak_above_resident_GiB"], 3)}
    return res


def vit_qdrop_graph_step(torch, dev, batch=128, steps=6, warmup=2):
    """The captured training step of Activation_Compression/cuda_graph_utils.py:82-120 (weight
    noise, forward, cross-entropy, backward, noise removal, gradient-norm clipping, AdamW) on the
    Controller-rewritten ViT-B/16 (all selected saved activations 2-bit, bf16 autocast, batch 128),
    replayed from one memset-free HIP graph, beside the same step run eagerly."""
    import torch.nn as nn

    from deep_optimization_amd.controller import Controller
    from deep_optimization_amd.graph import Graph, graph_node_counts
    from deep_optimization_amd.vit import vit_base_patch16_224

    g = torch.Generator(device=dev).manual_seed(5)
    xb = torch.randn((batch, 3, 224, 224), generator=g, device=dev)
    yb = torch.randint(0, 1000, (batch,), generator=g, device=dev)
    torch.manual_seed(0)
    model = vit_base_patch16_224().to(dev).train()
    model = Controller(model, {"batch_size": batch, "default_bits": 2}, input_shape=(3, 224, 224)).warp_model(quantizer=True)
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3, fused=True, capturable=True)
    gr = Graph(model, nn.CrossEntropyLoss(), opt, [(xb, yb)], None, "qdrop", 1)
    graphs, _, _, _, _, loss = gr.capture_cuda_graph_qdrop()
    counts = graph_node_counts(graphs[0])

    def eager():
        opt.zero_grad(set_to_none=False)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            gr._step(clip=True)

    def replay():
        opt.zero_grad(set_to_none=False)
        graphs[0].replay()

    res = {}
    for name, fn in (("eager", eager), ("graph_replay", replay)):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        res[f"{name}_ms_per_step"] = round((time.perf_counter() - t0) / steps * 1e3, 2)
    res["graph_speedup"] = round(res["eager_ms_per_step"] / res["graph_replay_ms_per_step"], 3)
    res["graph_nodes"] = counts
    res["memset_nodes_rewritten"] = gr.memsets_replaced[0]
    res["loss"] = round(float(loss.detach()), 4)
    del gr, graphs, model, opt
    return res


def resnet_train_step(torch, dev, batch=64, steps=6, warmup=3):
    """ResNet-50 train step (forward, cross-entropy, backward, SGD with momentum) on a fixed
    synthetic batch (N(0,1) 224x224x3 images, random labels over 1000 classes, bf16 autocast,
    random init), plain and rewritten by the Controller (every selected Conv / BatchNorm input 2-bit,
    ReLU masks 1-bit), each run eagerly and replayed from one memset-free HIP graph."""
    import torch.nn.functional as F

    from deep_optimization_amd.controller import Controller
    from deep_optimization_amd.graph import finalize
    from deep_optimization_amd.resnet import resnet50

    g = torch.Generator(device=dev).manual_seed(5)
    xb = torch.randn((batch, 3, 224, 224), generator=g, device=dev)
    yb = torch.randint(0, 1000, (batch,), generator=g, device=dev)
    res = {}
    for name in ("plain", "compressed_2bit"):
        torch.manual_seed(0)
        model = resnet50().to(dev).train()
        n_layers = None
        if name != "plain":
            ctl = Controller(model, {"batch_size": batch, "default_bits": 2}, input_shape=(3, 224, 224))
            model = ctl.warp_model(quantizer=True)
            n_layers = sum(1 for v in ctl.meta.values() if isinstance(v, dict))
        opt = torch.optim.SGD(model.parameters(), lr=0.01, momentum=0.9)

        def step():
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss = F.cross_entropy(model(xb), yb)
            loss.backward()
            opt.step()
            return loss

        def eager():
            opt.zero_grad(set_to_none=False)
            return step()

        first = float(eager().detach())
        for _ in range(warmup - 1):
            eager()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base_alloc = torch.cuda.memory_allocated()
        t0 = time.perf_counter()
        for _ in range(steps):
            eager()
        torch.cuda.synchronize()
        t_eager = (time.perf_counter() - t0) / steps
        peak = torch.cuda.max_memory_allocated() - base_alloc
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            eager()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        opt.zero_grad(set_to_none=False)
        with torch.cuda.graph(graph, stream=side):
            loss = step().detach()
        finalize(graph)
        for _ in range(warmup):
            opt.zero_grad(set_to_none=False)
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            opt.zero_grad(set_to_none=False)
            graph.replay()
        torch.cuda.synchronize()
        t_graph = (time.perf_counter() - t0) / steps
        res[name] = {"eager_ms_per_step": round(t_eager * 1e3, 2), "graph_replay_ms_per_step": round(t_graph * 1e3, 2),
                     "peak_above_resident_GiB": round(peak / 2 ** 30, 3), "loss_first_step": round(first, 4),
                     "loss_last_step": round(float(loss.detach()), 4)}
        if n_layers is not None:
            res[name]["layers_compressed"] = n_layers
        del graph, model, opt
        torch.cuda.empty_cache()
    p, c = res["plain"], res["compressed_2bit"]
    res["compressed_vs_plain"] = {
        "graph_step_time_ratio": round(c["graph_replay_ms_per_step"] / p["graph_replay_ms_per_step"], 3),
        "eager_step_time_ratio": round(c["eager_ms_per_step"] / p["eager_ms_per_step"], 3),
        "peak_above_resident_ratio": round(c["peak_above_resident_GiB"] / p["peak_above_resident_GiB"], 3)}
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # ~30 ms of warm-up and ~30 ms timed: long enough that the run-to-run spread of the step time
    # stays under 0.5%. The step takes ~12 us more than its two kernels timed apart, at any warm-up
    # length: the unpack's 411 MB of bf16 writes are written back while the next step's pack reads.
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--pmc-probe", action="store_true")
    ap.add_argument("--fp8-probe", choices=("random", "constant", "hipblaslt"))
    ap.add_argument("--dw-probe", action="store_true")
    ap.add_argument("--dw-tokens", default=None)
    ap.add_argument("--valu-probe", action="store_true")
    ap.add_argument("--host-probe", action="store_true")
    ap.add_argument("--counter-probe", choices=("philox", "nearest", "vit_philox", "vit_unpack", "vit_step", "gelu",
                                                "silu", "bn_squash", "bn_relu"))
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Activation compression shards with data parallelism and needs no exchange; run with --gpus 1.",
              file=sys.stderr)
        return 2
    if args.pmc_probe or args.fp8_probe or args.counter_probe or args.dw_probe or args.valu_probe or args.host_probe:
        from probes import modes

        if args.pmc_probe:
            return modes.pmc_probe()
        if args.fp8_probe:
            return modes.fp8_probe(args.fp8_probe)
        if args.counter_probe:
            return modes.counter_probe(args.counter_probe)
        if args.dw_probe:
            return modes.dw_probe(args.dw_tokens)
        if args.valu_probe:
            return modes.valu_probe()
        return modes.host_probe()

    import torch

    import deep_optimization_amd  # noqa: F401
    from deep_optimization_amd import _lib
    from deep_optimization_amd.graph import finalize as graph_finalize

    L = _lib.lib()
    dev = torch.device("cuda:0")
    ops = torch.ops.act_lib
    x, noise = resnet_inputs(torch, dev)
    xg = x.view(N, -1, G_SIZE)
    n_elem = x.numel()
    n_groups = n_elem // G_SIZE

    def step(rounding):
        p, s, m = ops.quant_pack(xg, BITS, G_SIZE, False, 0.0, False, rounding, noise if rounding == NOISE else None,
                                 1, 0, torch.float32)
        return ops.dequant_unpack(p, s, m, BITS, G_SIZE, torch.bfloat16)

    def settle(fn, seconds):
        """Run fn until `seconds` of wall time have passed, so that the part's clocks have left the
        state an idle gap leaves them in (the way Triton's do_bench warms up for 25 ms): a 2-5 ms
        timing window right after one measured a VALU-heavy pack up to 25% slower than the same
        kernel under sustained load."""
        t0 = time.perf_counter()
        while seconds > 0 and time.perf_counter() - t0 < seconds:
            for _ in range(4):
                fn()
            torch.cuda.synchronize()

    def time_steps(fn, steps, warmup, warm_s=SETTLE_S):
        for _ in range(warmup):
            fn()
        settle(fn, warm_s)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    sec = time_steps(lambda: step(NOISE), args.steps, args.warmup, warm_s=0.0)  # the contract: W warm-up steps
    pb_noise = pack_bytes(n_elem, n_groups, 2, BITS, noise=True)
    ub = unpack_bytes(n_elem, n_groups, 2, BITS)
    rt_bytes = pb_noise + ub
    value = rt_bytes / sec / 1e9

    # ---- dominant kernel: quant-pack (noise mode), launched through the C ABI on torch's current
    # stream and timed with HIP events recorded on that same stream (preallocated outputs).
    stream = torch.cuda.current_stream(dev)
    packed = torch.empty((n_groups, G_SIZE * BITS // 32), dtype=torch.int32, device=dev)
    scale = torch.empty(n_groups, dtype=torch.float32, device=dev)
    xmin = torch.empty(n_groups, dtype=torch.float32, device=dev)
    y = torch.empty_like(x)

    def launch_pack(rounding=NOISE):
        rc = L.dopt_quant_pack(xg.data_ptr(), _lib.BF16, n_groups, G_SIZE, BITS, None, rounding,
                               noise.data_ptr() if rounding == NOISE else None, 1, 0, 0, 0.0, packed.data_ptr(),
                               scale.data_ptr(), xmin.data_ptr(), _lib.F32, stream.cuda_stream)
        _lib.check(rc, "quant_pack")

    def launch_unpack():
        rc = L.dopt_dequant_unpack(packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), _lib.F32, n_groups, G_SIZE,
                                   BITS, None, y.data_ptr(), _lib.BF16, stream.cuda_stream)
        _lib.check(rc, "dequant_unpack")

    def event_avg(fn, reps=max(args.steps, 10)):
        for _ in range(3):
            fn()
        settle(fn, SETTLE_S)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / reps / 1e3  # seconds per launch

    t_pack = event_avg(launch_pack)
    t_unpack = event_avg(launch_unpack)
    # the memory system's ceiling for the same byte mix: dopt_stream_probe reads x and the noise
    # tensor and writes codes-sized and scale/min-sized outputs the way quant-pack does, with no
    # arithmetic; once with the writes and once reading only
    n_units = n_elem // 8
    probe_meta = torch.empty(2 * n_groups, dtype=torch.float32, device=dev)

    import probes

    PL = probes.lib()

    def launch_probe(bits):
        rc = PL.dopt_stream_probe(x.data_ptr(), noise.data_ptr(), packed.data_ptr(), probe_meta.data_ptr(), n_units,
                                  bits, stream.cuda_stream)
        probes.check(rc, "stream_probe")

    t_mix = event_avg(lambda: launch_probe(BITS))
    t_reads = event_avg(lambda: launch_probe(0))
    del probe_meta
    roofline = {"bound": "hbm", "kernel": "quant_pack_kernel<bf16, 2-bit, g256, noise tensor>",
                "achieved": round(pb_noise / t_pack / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(pb_noise / t_pack / 1e9 / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                "algorithmic_bytes_per_launch": pb_noise, "avg_launch_us": round(t_pack * 1e6, 2),
                "unpack_kernel": {"achieved": round(ub / t_unpack / 1e9, 1), "avg_launch_us": round(t_unpack * 1e6, 2),
                                  "frac": round(ub / t_unpack / 1e9 / HBM_PEAK_GBS, 4),
                                  "algorithmic_bytes_per_launch": ub},
                "same_mix_stream_ceiling": {"avg_launch_us": round(t_mix * 1e6, 2),
                                            "frac": round(pb_noise / t_mix / 1e9 / HBM_PEAK_GBS, 4),
                                            "kernel_time_vs_ceiling": round(t_pack / t_mix, 4),
                                            "reads_only_us": round(t_reads * 1e6, 2)}}

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(sec * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "config": {"workload": "BASELINE config 2: ResNet-50 conv2 activation bf16 [256,256,56,56] |N(0,1)|, "
                               "group 256, 2-bit stochastic rounding with a seeded uniform[0,1) noise tensor; "
                               "quant-pack fwd + unpack-dequant bwd (bf16 out)",
                   "bytes_per_step": rt_bytes, "group_size": G_SIZE, "bits": BITS, "rounding": "stochastic_noise",
                   "scale_dtype": "float32", "path": "torch.ops.act_lib (eager)"},
        "roofline": roofline,
    }

    if not args.no_extras:
        extras = {}
        pb_plain = pack_bytes(n_elem, n_groups, 2, BITS)
        for name, rn in (("stochastic_philox", PHILOX), ("nearest", NEAREST)):
            s_ = time_steps(lambda rn=rn: step(rn), args.steps, 2)
            b_ = pb_plain + ub
            t_k = event_avg(lambda rn=rn: launch_pack(rn))
            extras[f"resnet_{name}"] = {"GB/s": round(b_ / s_ / 1e9, 1), "frac": round(b_ / s_ / 1e9 / HBM_PEAK_GBS, 4),
                                        "ms_per_step": round(s_ * 1e3, 4), "bytes_per_step": b_,
                                        "pack_kernel_us": round(t_k * 1e6, 2),
                                        "pack_kernel_frac": round(pb_plain / t_k / 1e9 / HBM_PEAK_GBS, 4)}
        progress("graph replay of the step")
        # the same step replayed from a HIP graph (host dispatch removed)
        try:
            gs = torch.cuda.Stream()
            with torch.cuda.stream(gs):
                for _ in range(2):
                    step(NOISE)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph(keep_graph=True)
            with torch.cuda.graph(graph, stream=gs):
                step(NOISE)
            n_memset = graph_finalize(graph)
            s_g = time_steps(graph.replay, args.steps, 2)
            extras["resnet_noise_graph_replay"] = {"GB/s": round(rt_bytes / s_g / 1e9, 1),
                                                   "frac": round(rt_bytes / s_g / 1e9 / HBM_PEAK_GBS, 4),
                                                   "ms_per_step": round(s_g * 1e3, 4),
                                                   "memset_nodes_rewritten": n_memset}
            del graph
        except Exception as e:  # graph capture is an extra, never the headline
            extras["resnet_noise_graph_replay"] = {"error": str(e)[:200]}
        del packed, scale, xmin, y
        torch.cuda.empty_cache()
        progress("ViT MLP sweep")
        # config 3: ViT-B/16 MLP activation, GELU(N(0,1)) bf16 [256,197,3072], group 128, 1/2/4/8 bits,
        # stochastic rounding from the Philox stream
        vg = torch.Generator(device=dev).manual_seed(2)
        v = torch.nn.functional.gelu(torch.randn((256, 197, 3072), generator=vg, device=dev)).to(torch.bfloat16)
        vgrp = v.view(256, -1, 128)
        ve, vng = v.numel(), v.numel() // 128
        sweep = {}
        for b in (1, 2, 4, 8):
            def vstep(b=b):
                p, s, m = ops.quant_pack(vgrp, b, 128, False, 0.0, False, PHILOX, None, 1, 0, torch.float32)
                return ops.dequant_unpack(p, s, m, b, 128, torch.bfloat16)
            st = time_steps(vstep, args.steps, 2)
            vb = pack_bytes(ve, vng, 2, b) + unpack_bytes(ve, vng, 2, b)
            sweep[f"{b}bit"] = {"GB/s": round(vb / st / 1e9, 1), "frac": round(vb / st / 1e9 / HBM_PEAK_GBS, 4),
                                "packed_bytes": ve * b // 8 + vng * 8, "compression_vs_bf16": round(ve * 2 / (ve * b / 8 + vng * 8), 2),
                                "ms_per_step": round(st * 1e3, 4)}
        extras["vit_mlp_sweep_philox_g128"] = sweep
        # the reference's one measured figure (AC/test2.ipynb cell 0): its Triton dequant-unpack alone,
        # 2-bit, bf16 [8192, 768], g = 256, 0.024 ms per call on unstated hardware; the same operator
        # (act_lib::dequant_unpack_triton) on the same shape, 14,254,080 algorithmic bytes per call
        ng_r = 8192 * 768 // 256
        xr = torch.randn((1, ng_r, 256), generator=torch.Generator(device=dev).manual_seed(5), device=dev)
        pr, sr, mr = ops.quant_pack_triton(xr.to(torch.bfloat16), 2, 256, False, 0, True, 3.0)
        t_r = event_avg(lambda: ops.dequant_unpack_triton(pr, sr, mr, 2, 256, False, 0))
        rb = unpack_bytes(8192 * 768, ng_r, 2, 2) - ng_r * 4  # bf16 scale / min: 4 bytes per group, not 8
        extras["reference_notebook_dequant_8192x768_2bit"] = {
            "us": round(t_r * 1e6, 2), "GB/s": round(rb / t_r / 1e9, 1), "bytes": rb,
            "reference_us": 24.0, "vs_reference": round(24.0e-6 / t_r, 2),
            "note": "AC/test2.ipynb cell 0's figure, hardware unstated: a small, launch-bound call"}
        del xr, pr, sr, mr
        progress("fused activation layers")
        # fused activation layers: GELU / SiLU (y + 2-bit quantized derivative, g = 128, bf16
        # scale/min) on the ViT MLP activation, ReLU (y + 1-bit mask) on the ResNet activation;
        # bytes per element: forward in + y + codes (+ 4 B per group), backward codes (+ 4 B per
        # group) + dy + dx
        fused = {}
        vin = torch.randn((256, 197, 3072), generator=vg, device=dev).to(torch.bfloat16)
        dyv = torch.randn_like(vin)
        for name, fwd, bwd in (
                ("gelu", lambda: ops.gelu_fwd_fused_quan_pack(vin, 2, 128),
                 lambda o: ops.gelu_bwd_fused_dequan_unpack(o[1], dyv, o[2], o[3], 2, o[4], o[5], 128)),
                ("silu", lambda: ops.silu_fwd_quan_pack(vin, 2, 128, False, 0, False),
                 lambda o: ops.silu_bwd_fused_dequan_unpack(o[1], dyv, o[2], o[3], 2, o[4], o[5], 128, False, o[6],
                                                            o[7], o[8], o[9], False, 0))):
            o = fwd()
            tf = event_avg(fwd)
            tb = event_avg(lambda: bwd(o))
            fb = ve * (2 + 2) + ve * 2 // 8 + vng * 4
            bb = ve * 2 // 8 + vng * 4 + ve * (2 + 2)
            fused[f"{name}_vit_2bit_g128"] = {"fwd_us": round(tf * 1e6, 2), "fwd_frac": round(fb / tf / 1e9 / HBM_PEAK_GBS, 4),
                                              "bwd_us": round(tb * 1e6, 2), "bwd_frac": round(bb / tb / 1e9 / HBM_PEAK_GBS, 4)}
            del o
        del vin, dyv, v, vgrp
        torch.cuda.empty_cache()
        dyr = torch.randn_like(x)
        o = ops.relu_fwd_fused_pack(x, True, False, 1, G_SIZE)
        tf = event_avg(lambda: ops.relu_fwd_fused_pack(x, True, False, 1, G_SIZE))
        tb = event_avg(lambda: ops.relu_bwd_fused_unpack(o[1], dyr, 1, o[2], o[3], G_SIZE))
        fb = n_elem * (2 + 2) + n_elem // 8
        bb = n_elem // 8 + n_elem * (2 + 2)
        fused["relu_resnet_1bit"] = {"fwd_us": round(tf * 1e6, 2), "fwd_frac": round(fb / tf / 1e9 / HBM_PEAK_GBS, 4),
                                     "bwd_us": round(tb * 1e6, 2), "bwd_frac": round(bb / tb / 1e9 / HBM_PEAK_GBS, 4)}
        del o, dyr
        extras["fused_activation_layers"] = fused
        torch.cuda.empty_cache()
        progress("FP8 GEMM")
        # config 4: FP8 e4m3 scaled GEMM, beside hipBLASLt (torch._scaled_mm) on the same operands
        gemm = {}
        for (M, Nn, K) in ((8192, 8192, 8192), (4096, 11008, 4096)):
            gg = torch.Generator(device=dev).manual_seed(3)
            a = torch.randn((M, K), generator=gg, device=dev)
            bm = torch.randn((Nn, K), generator=gg, device=dev)
            sa, sb = 448.0 / a.abs().max(), 448.0 / bm.abs().max()
            a8, b8 = (a * sa).to(torch.float8_e4m3fn), (bm * sb).to(torch.float8_e4m3fn)
            del a, bm
            cm = torch.empty((M, Nn), dtype=torch.bfloat16, device=dev)
            osc = float(1.0 / (sa * sb))

            def gl():
                _lib.check(L.dopt_fp8_gemm_nt(a8.data_ptr(), b8.data_ptr(), M, Nn, K, K, K, osc, cm.data_ptr(), Nn,
                                              stream.cuda_stream), "fp8_gemm")
            # the part is power-limited on this data and its clock drifts with temperature, so the
            # two GEMMs are timed alternately (5 rounds of 10 launches each) and the medians compared
            ia, ib = (1.0 / sa).float().reshape(()), (1.0 / sb).float().reshape(())
            tgs, tbs, blas_err = [], [], None
            for _ in range(5):
                tgs.append(event_avg(gl, reps=10))
                if blas_err is None:
                    try:
                        tbs.append(event_avg(lambda: torch._scaled_mm(a8, b8.t(), scale_a=ia, scale_b=ib,
                                                                      out_dtype=torch.bfloat16), reps=10))
                    except Exception as e:
                        blas_err = str(e)[:200]
            tg = statistics.median(tgs)
            tf = 2.0 * M * Nn * K / tg / 1e12
            entry = {"TFLOP/s": round(tf, 1), "frac_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4), "us": round(tg * 1e6, 1),
                     "us_range": [round(min(tgs) * 1e6, 1), round(max(tgs) * 1e6, 1)]}
            if tbs:
                tb = statistics.median(tbs)
                entry["hipblaslt_TFLOP/s"] = round(2.0 * M * Nn * K / tb / 1e12, 1)
                entry["vs_hipblaslt"] = round(tb / tg, 3)
            if blas_err:
                entry["hipblaslt_error"] = blas_err
            gemm[f"{M}x{Nn}x{K}"] = entry
            del a8, b8, cm
        extras["fp8_gemm_nt"] = gemm
        progress("weight-gradient GEMM")
        # the compressed Linear layers' weight gradient dW = dy^T x_hat (+ db = sum dy) at the ViT-B/16
        # bs-128 shapes (K = 25216 tokens), 2-bit activations: the reference chain (dequantize, then
        # torch's GEMM and bias sum), hipBLASLt alone on x_hat, act_lib::dw_gemm on x_hat (with and
        # without the fused bias gradient) and on the packed codes (decoded inside the GEMM)
        dwx = {}
        Kt = 128 * 197
        for lname, cin, cout, gsz in (("qkv", 768, 2304, 256), ("proj", 768, 768, 256), ("fc1", 768, 3072, 256),
                                      ("fc2", 3072, 768, 512)):
            gd = torch.Generator(device=dev).manual_seed(7)
            xa = torch.randn((128, 197, cin), generator=gd, device=dev).to(torch.bfloat16)
            dyd = torch.randn((Kt, cout), generator=gd, device=dev).to(torch.bfloat16)
            pk, sc, mn = ops.quant_pack_triton(xa.view(128, -1, gsz), 2, gsz, False, 0, True, 3.0)
            xh = ops.dequant_unpack_triton(pk, sc, mn, 2, gsz, False, 0).view(Kt, cin)
            fl = 2.0 * Kt * cin * cout
            t = {"reference_chain": event_avg(lambda: (dyd.t().mm(ops.dequant_unpack_triton(pk, sc, mn, 2, gsz, False, 0)
                                                                   .view(Kt, cin)), dyd.sum(0)), reps=10),
                 "hipblaslt_mm": event_avg(lambda: dyd.t().mm(xh), reps=10),
                 "dw_gemm": event_avg(lambda: ops.dw_gemm(dyd, xh, None, None, None, cin, 0, 0, False, torch.bfloat16),
                                      reps=10),
                 "dw_gemm_db": event_avg(lambda: ops.dw_gemm(dyd, xh, None, None, None, cin, 0, 0, True, torch.bfloat16),
                                         reps=10),
                 "layer_dequant_dw_gemm_db": event_avg(
                     lambda: ops.dw_gemm(dyd, ops.dequant_unpack_triton(pk, sc, mn, 2, gsz, False, 0).view(Kt, cin), None,
                                         None, None, cin, 0, 0, True, torch.bfloat16), reps=10),
                 "packed_dw_gemm_db": event_avg(lambda: ops.dw_gemm(dyd, None, pk, sc, mn, cin, 2, gsz, True,
                                                                    torch.bfloat16), reps=10)}
            dwx[f"{lname}_{cout}x{cin}x{Kt}"] = {
                **{f"{k}_us": round(v * 1e6, 1) for k, v in t.items()},
                "dw_gemm_TFLOP/s": round(fl / t["dw_gemm"] / 1e12, 1),
                "dw_gemm_frac_bf16_peak": round(fl / t["dw_gemm"] / 1e12 / BF16_PEAK_TFLOPS, 4),
                "hipblaslt_TFLOP/s": round(fl / t["hipblaslt_mm"] / 1e12, 1),
                "layer_vs_reference_chain": round(t["reference_chain"] / t["layer_dequant_dw_gemm_db"], 3)}
            del xa, dyd, pk, sc, mn, xh
        extras["dw_gemm_vit_b16_bs128_2bit"] = dwx
        torch.cuda.empty_cache()
        torch.cuda.empty_cache()
        # the model-scale legs: a failure in one is recorded in its entry, and the JSON line (the
        # headline above) is still printed
        for key, label, leg in (("batchnorm_resnet_2bit", "BatchNorm layer", lambda: batchnorm_layer(torch, dev, event_avg)),
                                ("vit_b16_train_step_bs128", "ViT-B/16 train step", lambda: vit_train_step(torch, dev)),
                                ("resnet50_train_step_bs64", "ResNet-50 train step", lambda: resnet_train_step(torch, dev)),
                                ("vit_b16_qdrop_step_bs128_graph", "ViT-B/16 captured qdrop step",
                                 lambda: vit_qdrop_graph_step(torch, dev))):
            progress(label)
            try:
                extras[key] = leg()
            except Exception as e:  # noqa: BLE001  (reported in the JSON, not fatal to the headline)
                extras[key] = {"error": f"{type(e).__name__}: {str(e)[:300]}"}
                progress(f"{label} failed: {type(e).__name__}: {e}")
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
        out["extras"] = extras

    if not args.no_cpu:
        progress("CPU baseline")
        import numpy as np

        import oracle

        # the CPU restatement of the reference quantizer on the same workload (all 256 samples,
        # noise-tensor rounding, pack + unpack), every host thread, 2 warm-ups, median of 10
        def cpu_median(fn, reps=10, warm=2):
            ts = []
            for rep in range(reps + warm):
                t0 = time.perf_counter()
                fn()
                if rep >= warm:
                    ts.append(time.perf_counter() - t0)
            return statistics.median(ts), statistics.mean(ts)

        xs = x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1, G_SIZE)
        us = noise.cpu().numpy().reshape(-1, G_SIZE)

        def c2_round_trip():
            rp, rs, rm = oracle.quant_pack(xs, G_SIZE, BITS, rounding=oracle.STOCH_NOISE, noise=us)
            oracle.dequant_unpack(rp, rs, rm, G_SIZE, BITS, y_dtype=oracle.BF16)
        ct, cmean = cpu_median(c2_round_trip)
        del xs, us
        cpu_model = "unknown"
        try:
            with open("/proc/cpuinfo") as f:
                cpu_model = next(ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name"))
        except (OSError, StopIteration):
            pass
        configs = {"C2": {"GB/s": round(rt_bytes / ct / 1e9, 3), "s_per_round_trip": round(ct, 4)}}
        # config 1 (the reference's CPU case): fp32 [8,64,32,32] ~ N(0,1) seed 0, g = 256 as 16 x 16
        # spatial tiles, 2-bit nearest, fp32 scale/min, round trip to fp32
        g1 = torch.Generator().manual_seed(0)
        x1 = torch.randn(8, 64, 32, 32, generator=g1, dtype=torch.float32).numpy()

        def c1_round_trip():
            rp, rs, rm = oracle.quant_pack(x1, 256, 2, tile_nchw=(8, 64, 32, 32))
            oracle.dequant_unpack(rp, rs, rm, 256, 2, tile_nchw=(8, 64, 32, 32), y_dtype=oracle.F32)
        n1 = x1.size
        c1t, _ = cpu_median(c1_round_trip, reps=50, warm=5)
        c1_bytes = 2 * (n1 * 4 + n1 * 2 // 8 + (n1 // 256) * 8)
        configs["C1"] = {"GB/s": round(c1_bytes / c1t / 1e9, 3), "s_per_round_trip": round(c1t, 6)}
        # config 3: ViT-B/16 MLP activation GELU(N(0,1)) bf16 [256,197,3072], g = 128, Philox rounding
        # (the GPU sweep's stream), pack + unpack to bf16, each bit width
        vg3 = torch.Generator(device=dev).manual_seed(2)
        v3 = torch.nn.functional.gelu(torch.randn((256, 197, 3072), generator=vg3, device=dev)).to(torch.bfloat16)
        v3s = v3.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1, 128)
        del v3
        n3 = v3s.size
        for b in (1, 2, 4, 8):
            def c3_round_trip(b=b):
                rp, rs, rm = oracle.quant_pack(v3s, 128, b, rounding=oracle.STOCH_PHILOX, seed=1, offset=0)
                oracle.dequant_unpack(rp, rs, rm, 128, b, y_dtype=oracle.BF16)
            c3t, _ = cpu_median(c3_round_trip, reps=5, warm=1)
            c3_bytes = pack_bytes(n3, n3 // 128, 2, b) + unpack_bytes(n3, n3 // 128, 2, b)
            configs[f"C3_{b}bit"] = {"GB/s": round(c3_bytes / c3t / 1e9, 3), "s_per_round_trip": round(c3t, 4)}
        del v3s
        out["cpu_baseline"] = {"value": configs["C2"]["GB/s"], "unit": "GB/s", "cores": oracle.num_threads(),
                               "kind": "port", "cpu_model": cpu_model,
                               "sample": f"the full workload ({n_elem} elements, noise-tensor 2-bit, g={G_SIZE}), "
                                         "pack + unpack with the C oracle (OpenMP), median of 10 runs after 2 warm-ups "
                                         f"({cmean:.2f} s each); configs C1 (median of 50) and C3 (the full "
                                         "[256,197,3072] activation per bit width, median of 5) beside it",
                               "configs": configs}
        out["cpu_baseline"]["gpu_over_cpu"] = round(value / out["cpu_baseline"]["value"], 1)

    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
