"""Probe modes of bench.py: short runs of one kernel each, made to be profiled
(``rocprofv3 --pmc`` / ``--kernel-trace``) or timed on their own. ``bench.py --pmc-probe``,
``--fp8-probe``, ``--counter-probe``, ``--valu-probe``, ``--host-probe`` and ``--dw-probe`` call
these functions; the commands in ``profiles/`` name those flags."""
from __future__ import annotations

import json
import statistics
import time

from . import check, lib

N, C, H, W = 256, 256, 56, 56
G_SIZE, BITS = 256, 2
NEAREST, NOISE, PHILOX = 0, 1, 2


def resnet_inputs(torch, dev):
    gen = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((N, C, H, W), generator=gen, device=dev, dtype=torch.float32).abs_().to(torch.bfloat16)
    noise = torch.rand((N, C * H * W // G_SIZE, G_SIZE), generator=torch.Generator(device=dev).manual_seed(1),
                       device=dev)
    return x, noise


def pmc_probe() -> int:
    """A plain copy of known size (the counter calibration), then the dominant kernel three times and
    the unpack-dequant kernel three times."""
    import torch

    import deep_optimization_amd  # noqa: F401
    from deep_optimization_amd import _lib

    dev = torch.device("cuda:0")
    x, noise = resnet_inputs(torch, dev)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    y.copy_(x)  # 411,041,792 bytes read + the same written
    torch.cuda.synchronize()
    xg = x.view(N, -1, G_SIZE)
    n_groups = xg.shape[0] * xg.shape[1]
    packed = torch.empty((n_groups, G_SIZE * BITS // 32), dtype=torch.int32, device=dev)
    scale = torch.empty(n_groups, dtype=torch.float32, device=dev)
    xmin = torch.empty(n_groups, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    for _ in range(3):
        _lib.check(_lib.lib().dopt_quant_pack(xg.data_ptr(), _lib.BF16, n_groups, G_SIZE, BITS, None, NOISE,
                                              noise.data_ptr(), 0, 0, 0, 0.0, packed.data_ptr(), scale.data_ptr(),
                                              xmin.data_ptr(), _lib.F32, stream), "quant_pack")
    for _ in range(3):
        _lib.check(_lib.lib().dopt_dequant_unpack(packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), _lib.F32,
                                                  n_groups, G_SIZE, BITS, None, y.data_ptr(), _lib.BF16, stream),
                   "dequant_unpack")
    torch.cuda.synchronize()
    print(f"pmc probe: copy {x.numel() * 2} B, then 3 x quant_pack (noise, bf16, g={G_SIZE}, {BITS}-bit), "
          "3 x dequant_unpack (bf16 out)")
    return 0


def fp8_probe(mode: str) -> int:
    """The 8192^3 FP8 GEMM, 3 + 10 launches, on the bench's N(0,1) -> e4m3 operands ("random") or on
    constant operands ("constant": every A byte 0x38 = 1.0, every B byte 0x30 = 0.5), for
    rocprofv3 --pmc runs that compare clock (GRBM_GUI_ACTIVE) and MFMA occupancy between the two;
    "hipblaslt" runs torch._scaled_mm (hipBLASLt) on the "random" operands instead of this library."""
    import torch

    import deep_optimization_amd  # noqa: F401
    from deep_optimization_amd import _lib

    dev = torch.device("cuda:0")
    M = Nn = K = 8192
    if mode == "constant":
        a8 = torch.full((M, K), 0x38, dtype=torch.uint8, device=dev)
        b8 = torch.full((Nn, K), 0x30, dtype=torch.uint8, device=dev)
        osc = 1.0
    else:
        gg = torch.Generator(device=dev).manual_seed(3)
        a = torch.randn((M, K), generator=gg, device=dev)
        bm = torch.randn((Nn, K), generator=gg, device=dev)
        sa, sb = 448.0 / a.abs().max(), 448.0 / bm.abs().max()
        a8 = (a * sa).to(torch.float8_e4m3fn).view(torch.uint8)
        b8 = (bm * sb).to(torch.float8_e4m3fn).view(torch.uint8)
        osc = float(1.0 / (sa * sb))
        del a, bm
    cm = torch.empty((M, Nn), dtype=torch.bfloat16, device=dev)
    L = _lib.lib()
    stream = torch.cuda.current_stream(dev)

    def launch():
        _lib.check(L.dopt_fp8_gemm_nt(a8.data_ptr(), b8.data_ptr(), M, Nn, K, K, K, osc, cm.data_ptr(), Nn,
                                      stream.cuda_stream), "fp8_gemm")
    if mode == "hipblaslt":
        a8f, b8f = a8.view(torch.float8_e4m3fn), b8.view(torch.float8_e4m3fn)
        one = torch.ones((), dtype=torch.float32, device=dev)

        def launch():  # noqa: F811  (the hipBLASLt comparison)
            torch._scaled_mm(a8f, b8f.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
    for _ in range(3):
        launch()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(10):
        launch()
    e1.record(stream)
    e1.synchronize()
    us = e0.elapsed_time(e1) / 10 * 1e3
    print(f"fp8 probe ({mode}): {us:.1f} us per launch, {2.0 * M * Nn * K / us / 1e6:.0f} TFLOP/s")
    return 0


def counter_probe(name: str) -> int:
    """One kernel below 70% of HBM peak, 3 + 10 launches, for rocprofv3 --pmc runs (instruction mix,
    VALU activity, HBM bytes): "philox" / "nearest" = the ResNet-activation quant-pack (bf16 [256,256,56,56]
    |N(0,1)|, g = 256, 2-bit); "vit_philox" / "vit_unpack" = the ViT-MLP-activation 2-bit Philox quant-pack
    and its unpack-dequant (GELU(N(0,1)) bf16 [256,197,3072], g = 128), "vit_step" both in turn
    (that step); "gelu" / "silu" = the
    fused activation forward on the ViT MLP
    activation (bf16 [256,197,3072] N(0,1), g = 128, 2-bit); "bn_squash" / "bn_relu" = the
    BatchNorm normalize + quant-pack forward on the ResNet stage-1 activation (bf16
    [256,256,56,56], g = 512, 2-bit)."""
    import torch

    import deep_optimization_amd  # noqa: F401

    dev = torch.device("cuda:0")
    ops = torch.ops.act_lib
    gen = torch.Generator(device=dev).manual_seed(0)
    if name in ("philox", "nearest"):
        x = torch.randn((256, 256, 56, 56), generator=gen, device=dev).abs_().to(torch.bfloat16).view(256, -1, G_SIZE)
        rn = PHILOX if name == "philox" else NEAREST
        fn = lambda: ops.quant_pack(x, BITS, G_SIZE, False, 0.0, False, rn, None, 1, 0, torch.float32)  # noqa: E731
    elif name in ("vit_philox", "vit_unpack", "vit_step"):
        v = torch.nn.functional.gelu(torch.randn((256, 197, 3072), generator=gen, device=dev)).to(torch.bfloat16)
        vgrp = v.view(256, -1, 128)
        pk = lambda: ops.quant_pack(vgrp, 2, 128, False, 0.0, False, PHILOX, None, 1, 0, torch.float32)  # noqa: E731
        if name == "vit_philox":
            fn = pk
        elif name == "vit_step":
            fn = lambda: ops.dequant_unpack(*pk(), 2, 128, torch.bfloat16)  # noqa: E731
        else:
            p_, s_, m_ = pk()
            fn = lambda: ops.dequant_unpack(p_, s_, m_, 2, 128, torch.bfloat16)  # noqa: E731
    elif name in ("gelu", "silu"):
        v = torch.randn((256, 197, 3072), generator=gen, device=dev).to(torch.bfloat16)
        if name == "gelu":
            fn = lambda: ops.gelu_fwd_fused_quan_pack(v, 2, 128)  # noqa: E731
        else:
            fn = lambda: ops.silu_fwd_quan_pack(v, 2, 128, False, 0, False)  # noqa: E731
    elif name in ("bn_squash", "bn_relu"):
        N, C, HW = 256, 256, 56 * 56
        g = dict(M=N * HW, HW=HW, stride_n=C * HW, stride_c=HW)
        x = torch.randn((N, C, HW), generator=gen, device=dev).to(torch.bfloat16)
        w = torch.rand(C, generator=gen, device=dev) + 0.5
        b = torch.randn(C, generator=gen, device=dev)
        s_, q_ = ops.bn_fwd_reduce(x, **g, BLOCK_M=1024, num_warps=8, num_stages=5)
        if name == "bn_squash":
            fn = lambda: ops.bn_fwd_norm_quant_pack_fused(x, s_, q_, w, b, None, None, **g, BLOCK_M=1024, bits=2,  # noqa: E731
                                                          sync=False, avg_alam=False, alam_bits=0, num_warps=8,
                                                          num_stages=5)
        else:
            fn = lambda: ops.bn_relu_fwd_norm_fused_quant_pack(x, s_, q_, w, b, None, None, **g, relu=True,  # noqa: E731
                                                               relu6=False, BLOCK_SIZE=1024, BITS=2, sync=False)
    else:
        raise SystemExit(f"unknown counter probe {name!r}")
    for _ in range(13):
        fn()
    torch.cuda.synchronize()
    print(f"counter probe {name}: 13 launches")
    return 0


def valu_probe() -> int:
    """Issue cost of one VALU instruction kind (dopt_valu_probe): ns per wave-instruction per SIMD
    for v_fma_f32, v_exp_f32, v_rcp_f32 and v_mad_u64_u32 + v_xor_b32, median of 5 event-timed
    windows of 10 launches of 2048 workgroups (8192 waves, 4096 steps per lane); then the
    sustained bf16 MFMA rate of the weight-gradient GEMM's inner-loop shape with random and with
    constant operands."""
    import torch

    import deep_optimization_amd  # noqa: F401

    L = lib()
    dev = torch.device("cuda:0")
    blocks = 2048
    out = torch.empty(blocks * 256, device=dev)
    st = torch.cuda.current_stream(dev)
    simds = torch.cuda.get_device_properties(dev).multi_processor_count * 4
    per_simd = blocks * 4 * 8 * 512 / simds  # wave-instructions per SIMD per launch
    res = {}
    for kind, name in enumerate(("v_fma_f32", "v_exp_f32", "v_rcp_f32", "v_mad_u64_u32+v_xor_b32", "mfma_bf16_random",
                                 "mfma_bf16_constant", "mfma_fp8_random", "mfma_fp8_constant")):
        fn = lambda kind=kind: check(L.dopt_valu_probe(kind, out.data_ptr(), blocks, st.cuda_stream),  # noqa: E731
                                     "valu_probe")
        for _ in range(3):
            fn()
        ts = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            for _ in range(10):
                fn()
            e1.record(st)
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) / 10 * 1e3)
        us = statistics.median(ts)
        if kind < 4:
            res[name] = {"us_per_launch": round(us, 2), "ns_per_wave_instruction": round(us * 1e3 / per_simd, 4)}
        elif kind < 6:
            tf = blocks * 4 * 64 * 16 * 32768 / us / 1e6
            res[name] = {"us_per_launch": round(us, 2), "TFLOP/s": round(tf, 1), "frac_bf16_peak": round(tf / 2500.0, 4)}
        else:
            tf = blocks * 4 * 64 * 16 * 131072 / us / 1e6
            res[name] = {"us_per_launch": round(us, 2), "TFLOP/s": round(tf, 1), "frac_fp8_peak": round(tf / 5000.0, 4)}
    print(json.dumps({"valu_probe": res, "simds": simds}))
    return 0


def host_probe() -> int:
    """Host cost of one eager operator call, and of its parts, on inputs small enough that the GPU
    work is negligible (one 256-element bf16 group, 2-bit nearest): per-call wall time of 2000
    back-to-back calls (one synchronize at the end), medians of 5 windows, for
      - torch.ops.act_lib.quant_pack / dequant_unpack (dispatcher + Python wrapper + ctypes + launch),
      - the same Python implementations called directly (no dispatcher),
      - the raw ctypes calls into libdopt with preallocated outputs (marshalling + launch),
      - the wrapper's pieces: _aligned (contiguous + alignment test), torch.empty x 3, the stream
        lookup."""
    import torch

    import deep_optimization_amd  # noqa: F401
    from deep_optimization_amd import _lib, act_lib

    dev = torch.device("cuda:0")
    L = _lib.lib()
    ops = torch.ops.act_lib
    x = torch.randn((1, 1, G_SIZE), device=dev).to(torch.bfloat16)
    packed = torch.empty((1, G_SIZE * BITS // 32), dtype=torch.int32, device=dev)
    scale = torch.empty(1, dtype=torch.float32, device=dev)
    xmin = torch.empty(1, dtype=torch.float32, device=dev)
    y = torch.empty((1, 1, G_SIZE), dtype=torch.bfloat16, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    p0, s0, m0 = ops.quant_pack(x, BITS, G_SIZE, False, 0.0, False, NEAREST, None, 1, 0, torch.float32)

    def raw_pack():
        L.dopt_quant_pack(x.data_ptr(), _lib.BF16, 1, G_SIZE, BITS, None, NEAREST, None, 1, 0, 0, 0.0,
                          packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), _lib.F32, st)

    def raw_unpack():
        L.dopt_dequant_unpack(packed.data_ptr(), scale.data_ptr(), xmin.data_ptr(), _lib.F32, 1, G_SIZE, BITS, None,
                              y.data_ptr(), _lib.BF16, st)

    cases = {
        "op_quant_pack": lambda: ops.quant_pack(x, BITS, G_SIZE, False, 0.0, False, NEAREST, None, 1, 0, torch.float32),
        "op_dequant_unpack": lambda: ops.dequant_unpack(p0, s0, m0, BITS, G_SIZE, torch.bfloat16),
        "python_impl_quant_pack": lambda: act_lib._quant_pack(x, BITS, G_SIZE, False, 0.0, False, NEAREST, None, 1, 0,
                                                              torch.float32),
        "ctypes_quant_pack": raw_pack,
        "ctypes_dequant_unpack": raw_unpack,
        "aligned": lambda: act_lib._aligned(x),
        "torch_empty_x3": lambda: (torch.empty((1, 16), dtype=torch.int32, device=dev),
                                   torch.empty(1, dtype=torch.float32, device=dev),
                                   torch.empty(1, dtype=torch.float32, device=dev)),
        "stream_lookup": lambda: act_lib._stream(x),
    }
    res = {}
    for name, fn in cases.items():
        for _ in range(200):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            for _ in range(2000):
                fn()
            torch.cuda.synchronize()
            ts.append((time.perf_counter() - t0) / 2000 * 1e6)
        res[name] = round(statistics.median(ts), 2)
    print(json.dumps({"host_probe_us_per_call": res}))
    return 0


def dw_probe(tokens: str | None = None) -> int:
    """Weight-gradient GEMMs at the ViT-B/16 bs-128 fc1 shape (dy bf16 [K, 3072], x_hat bf16
    [K, 768], no bias gradient): three at K = 25216 tokens for rocprofv3 --pmc runs, or with
    `tokens` (comma-separated K values) five at each K, for a kernel-trace K sweep that separates
    the cost per token from the fixed cost of a call (pipeline fill, split partials, reduce)."""
    import torch

    import deep_optimization_amd  # noqa: F401

    dev = torch.device("cuda:0")
    cin, cout = 768, 3072
    ks, reps = ([int(k) for k in tokens.split(",")], 5) if tokens else ([128 * 197], 3)
    for K in ks:
        g = torch.Generator(device=dev).manual_seed(7)
        dy = torch.randn((K, cout), generator=g, device=dev).to(torch.bfloat16)
        xh = torch.randn((K, cin), generator=g, device=dev).to(torch.bfloat16)
        for _ in range(reps):
            torch.ops.act_lib.dw_gemm(dy, xh, None, None, None, cin, 0, 0, False, torch.bfloat16)
        torch.cuda.synchronize()
        print(f"dw probe: {reps} x dw_gemm M={cout} N={cin} K={K}", flush=True)
        del dy, xh
    return 0
