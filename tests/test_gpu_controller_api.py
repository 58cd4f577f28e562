"""The reference's Controller call sequence on the GPU, and its graph mode.

* ``test8.ipynb`` cell 2 (also Train/Trainer.py:179-183), statement for statement, on ViT-B/16
  (10 classes, batch 128) with test8's configuration, including its DIVISION low-pass
  ({'pool_kernel_size': 3}), and a list of two synthetic batches as the loader: the constructor
  analyses and traces, ``iterate`` sets the bits, ``warp_model(graph_mode=True, quantizer=True)``
  swaps 61 layers, and one step through ``traced_model`` gives a finite loss and gradients. One
  weight gradient of a layer the analysis gave DIVISION is checked against fp32
  dy^T . (dequant(quant(x)) + upsample(avgpool(x))), the reference's restore
  (module_utils.py:86-102 with ops.py:457-474), the operators themselves being bit-exact against
  the CPU oracle elsewhere.
* ``Controller.warmup`` / ``enable_graph_mode`` (controller.py:316-351): the rewritten model's
  forward and backward replay HIP graphs and give the losses and gradients of an eager copy of the
  same rewrite on three batches, before and after an in-place change of every parameter.
"""
import copy

import pytest
import torch
import torch.nn.functional as F
from torch import nn

import deep_optimization_amd  # noqa: F401
from deep_optimization_amd.controller import Controller
from deep_optimization_amd.vit import VisionTransformer, vit_base_patch16_224

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture
def restore_matmul_flags():
    flags = (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32,
             torch.get_float32_matmul_precision())
    yield
    torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32 = flags[:2]
    torch.set_float32_matmul_precision(flags[2])


def rel_err(got, want):
    got, want = got.double(), want.double()
    return ((got - want).norm() / want.norm().clamp_min(1e-30)).item()


def disable_act_inplace(m):
    for module in m.modules():
        if isinstance(module, (nn.ReLU, nn.SiLU, nn.GELU)) and hasattr(module, "inplace"):
            module.inplace = False


def test_test8_cell2_sequence(restore_matmul_flags):
    batch_size = 128
    g = torch.Generator().manual_seed(8)
    train_loader = [(torch.randn(batch_size, 3, 224, 224, generator=g), torch.randint(0, 10, (batch_size,), generator=g))
                    for _ in range(2)]
    print("[test8 cell 2] Controller(test=False) on ViT-B/16", flush=True)
    # --- test8.ipynb cell 2, verbatim apart from the model constructor (timm is not a dependency)
    DIVISION = {
        'pool_kernel_size': 3
    }
    config = {
        "default_bits": 2,
        'auto_precision': None,
        'DIVISION': DIVISION,
        "group_size": 256,
        'batch_size': batch_size,
        'fp8': False,
        'depth_point_conv': False,
        'rms_norm': False
    }
    torch.manual_seed(0)
    model = vit_base_patch16_224(num_classes=10)
    disable_act_inplace(model)
    criterion = nn.CrossEntropyLoss()
    controller = Controller(model, config, train_loader, criterion, test=False)
    controller.iterate(criterion)
    controller.warp_model(graph_mode=True, quantizer=True)
    # ---
    layers = [k for k, v in controller.meta.items() if isinstance(v, dict)]
    assert len(layers) == 61, layers
    assert set(controller.quantizer.bits) == set(layers) and set(controller.quantizer.bits.values()) == {2}
    division = sorted(k for k in layers if controller.meta[k]["DIVISION"] is not None)
    lf = controller.low_frequency_energy_ratio_grad
    assert division == sorted(k for k in layers if k in lf and lf[k] != 1
                              and lf[k] > controller.base_division_threshold_grad)
    print(f"[test8 cell 2] DIVISION layers: {division}", flush=True)
    assert division, "the analysis gave no layer DIVISION"

    model = controller.traced_model
    lin = next(k for k in division if isinstance(model.get_submodule(k), nn.Linear))
    mod = model.get_submodule(lin)
    cap = {}
    h1 = mod.register_forward_pre_hook(lambda m, args: cap.__setitem__("x", args[0].detach()))
    h2 = mod.register_full_backward_hook(lambda m, gin, gout: cap.__setitem__("dy", gout[0].detach()))
    x, y = (t.to(DEV) for t in train_loader[0])
    print("[test8 cell 2] one traced_model step", flush=True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss = criterion(model(x), y)
    loss.backward()
    h1.remove()
    h2.remove()
    assert torch.isfinite(loss), loss
    for n_, p in model.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n_

    m = controller.meta[lin]
    g_ = m["group_size"]
    xb = cap["x"].to(torch.bfloat16)
    packed, scale, xmin = torch.ops.act_lib.quant_pack_triton(xb.reshape(batch_size, -1, g_), 2, g_, False, 0,
                                                              True, 3.0)
    x_hat = torch.ops.act_lib.dequant_unpack_triton(packed, scale, xmin, 2, g_, False, 0).reshape(xb.shape)
    k = min(xb.shape[2], DIVISION["pool_kernel_size"])
    low = F.interpolate(F.avg_pool1d(xb, k, stride=k, padding=0), size=xb.shape[2], mode="nearest")
    restored = (x_hat + low.to(torch.bfloat16)).float()
    dy = cap["dy"].float().reshape(-1, mod.weight.shape[0])
    want = dy.t() @ restored.reshape(-1, mod.weight.shape[1])
    err = rel_err(mod.weight.grad, want)
    print(f"[test8 cell 2] {lin} dW rel err {err:.2e} against the DIVISION restore", flush=True)
    assert err <= 1e-2


def test_warmup_graph_mode_matches_eager(restore_matmul_flags):
    B = 32
    torch.manual_seed(3)
    base = VisionTransformer(depth=2, num_classes=10).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(4)
    batches = [(torch.randn(B, 3, 224, 224, generator=g, device=DEV), torch.randint(0, 10, (B,), generator=g, device=DEV))
               for _ in range(3)]
    crit = nn.CrossEntropyLoss()
    cfg = {"default_bits": 2, "batch_size": B, "auto_precision": None}
    eager = Controller(copy.deepcopy(base), dict(cfg), input_shape=(3, 224, 224)).warp_model(quantizer=True)
    ctl = Controller(copy.deepcopy(base), dict(cfg), batches, crit)
    print("[graph mode] Controller.warmup (rewrite, enable_graph_mode, capturing step)", flush=True)
    ctl.warmup(batches, crit, torch.cuda.Stream())
    graphed = ctl.traced_model
    assert len(graphed._dopt_graph_captures) == 1
    # the capturing step's gradients are the first batch's: compare, then start both from zero
    with torch.autocast("cuda", dtype=torch.bfloat16):
        crit(eager(batches[0][0]), batches[0][1]).backward()
    for (n_, pe), pg in zip(eager.named_parameters(), graphed.parameters()):
        assert rel_err(pg.grad, pe.grad) <= 1e-3, n_
    # three batches, then the same in-place change of every parameter in both models (the graphs
    # read the parameters where they live), then the three batches again; each compared with the
    # eager copy. (Comparing over optimizer steps instead would amplify the ~1e-5 differences of
    # the patch convolution's weight gradient, whose solver is MIOpen's choice, through the
    # training dynamics.)
    for rnd in range(2):
        if rnd == 1:
            with torch.no_grad():
                for pe, pg in zip(eager.parameters(), graphed.parameters()):
                    delta = torch.randn_like(pe) * 0.01 * pe.abs().mean().clamp_min(1e-3)
                    pe.mul_(0.9).add_(delta)
                    pg.mul_(0.9).add_(delta)
        for step, (x, y) in enumerate(batches):
            losses = []
            for m in (eager, graphed):
                m.zero_grad(set_to_none=True)
                with torch.autocast("cuda", dtype=torch.bfloat16):
                    loss = crit(m(x), y)
                loss.backward()
                losses.append(loss.item())
            worst = max(rel_err(pg.grad, pe.grad) for pe, pg in zip(eager.parameters(), graphed.parameters()))
            print(f"[graph mode] round {rnd} batch {step}: loss eager {losses[0]:.6f} graph {losses[1]:.6f}, "
                  f"worst grad rel err {worst:.2e}", flush=True)
            assert abs(losses[1] - losses[0]) <= 1e-4 * abs(losses[0])
            assert worst <= 1e-3
    assert len(graphed._dopt_graph_captures) == 1  # every step replayed the one capture
    # eval and no-grad calls run the eager forward
    graphed.eval()
    eager.eval()
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        torch.testing.assert_close(graphed(batches[0][0]), eager(batches[0][0]), rtol=0, atol=0)
