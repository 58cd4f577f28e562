"""The end-to-end workload: ViT-B/16 (12 blocks, 1000 classes) on a batch of 128
synthetic 224x224x3 N(0, 1) images, bf16 autocast, rewritten by the Controller with every selected
saved activation 2-bit (reference: Activation_Compression/controller.py:63-351 applied to timm's
vit_base_patch16_224 in test8.ipynb cells 2 and 9).

What is pinned:
  * the rewrite: 61 layers (the patch convolution and, per block, qkv, proj, fc1, GELU, fc2);
  * the forward: the compressed layers change only what is saved. With the plain model's GELU
    evaluated by the same fused formula (act_lib::gelu_triton, whose bf16 output equals the one
    the compressed GELU writes), the first step's loss is bit-identical to the plain model's, and
    so is the gradient of the head (an uncompressed Linear whose gradient depends only on the
    forward). Against torch's own tanh GELU, which may round each bf16 output differently, the
    loss agrees within 1e-2;
  * one mlp.fc1 weight gradient equals fp32 dy^T . x_hat within 1e-2 (relative Frobenius), with
    x_hat from the reference operator chain quant_pack_triton(clamp=True, alpha=3) ->
    dequant_unpack_triton, itself bit-exact against the CPU oracle;
  * two train steps: finite loss and a finite gradient for every parameter;
  * the bytes the autograd graph saves drop below 0.6x the plain model's.
"""
import copy

import pytest
import torch
import torch.nn.functional as F

import deep_optimization_amd  # noqa: F401
from deep_optimization_amd.controller import Controller
from deep_optimization_amd.vit import vit_base_patch16_224

pytestmark = pytest.mark.gpu
DEV = "cuda"
BATCH = 128


def rel_err(got, want):
    got, want = got.double(), want.double()
    return ((got - want).norm() / want.norm().clamp_min(1e-30)).item()


class _FusedFormulaGelu(torch.autograd.Function):
    """torch's GELU replaced by the fused kernels' formula (value and exact derivative in bf16)."""

    @staticmethod
    def forward(ctx, x):
        y, d = torch.ops.act_lib.gelu_triton(x)
        ctx.save_for_backward(d)
        return y

    @staticmethod
    def backward(ctx, dy):
        (d,) = ctx.saved_tensors
        return dy * d


class FusedFormulaGelu(torch.nn.Module):
    def forward(self, x):
        return _FusedFormulaGelu.apply(x)


def saved_bytes(model, x):
    seen, total = set(), [0]

    def pack(t):
        key = (t.untyped_storage().data_ptr(), t.dtype)
        if key not in seen and not isinstance(t, torch.nn.Parameter):
            seen.add(key)
            total[0] += t.untyped_storage().nbytes()
        return t

    with torch.autograd.graph.saved_tensors_hooks(pack, lambda t: t):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            model(x)
    return total[0]


def test_vit_b16_batch128_two_compressed_steps():
    print("[config 5] building ViT-B/16 and its Controller rewrite", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn((BATCH, 3, 224, 224), generator=gen, device=DEV)
    y = torch.randint(0, 1000, (BATCH,), generator=gen, device=DEV)
    torch.manual_seed(0)
    plain = vit_base_patch16_224().to(DEV).train()
    ctl = Controller(copy.deepcopy(plain), {"batch_size": BATCH, "default_bits": 2}, input_shape=(3, 224, 224))
    model = ctl.warp_model(quantizer=True)
    layers = [k for k, v in ctl.meta.items() if isinstance(v, dict)]
    assert len(layers) == 61, layers
    for blk in range(12):
        for part in ("attn.qkv", "attn.proj", "mlp.fc1", "mlp.act", "mlp.fc2"):
            assert f"blocks.{blk}.{part}" in ctl.meta

    # plain reference steps (same weights, same batch): torch's GELU, and the fused formula
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss_torch_gelu = F.cross_entropy(plain(x), y).item()
    same_formula = copy.deepcopy(plain)
    for blk in same_formula.blocks:
        blk.mlp.act = FusedFormulaGelu()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss_plain = F.cross_entropy(same_formula(x), y)
    loss_plain.backward()
    head_grad_plain = same_formula.head.weight.grad.detach().clone()
    del same_formula

    # capture mlp.fc1's input and output gradient in block 5
    fc1 = dict(model.named_modules())["blocks.5.mlp.fc1"]
    cap = {}
    h1 = fc1.register_forward_pre_hook(lambda m, args: cap.__setitem__("x", args[0].detach()))
    h2 = fc1.register_full_backward_hook(lambda m, gin, gout: cap.__setitem__("dy", gout[0].detach()))
    opt = torch.optim.AdamW(model.parameters(), lr=1e-3, fused=True)
    losses = []
    for step in range(2):
        print(f"[config 5] compressed step {step}", flush=True)
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = F.cross_entropy(model(x), y)
        loss.backward()
        assert torch.isfinite(loss), loss
        for n_, p in model.named_parameters():
            assert p.grad is not None and torch.isfinite(p.grad).all(), n_
        if step == 0:
            h1.remove()
            h2.remove()
            assert torch.equal(loss.detach(), loss_plain.detach()), (loss.item(), loss_plain.item())
            assert torch.equal(dict(model.named_parameters())["head.weight"].grad, head_grad_plain)
            assert abs(loss.item() - loss_torch_gelu) <= 1e-2 * abs(loss_torch_gelu)
            m = ctl.meta["blocks.5.mlp.fc1"]
            g = m["group_size"]
            assert m["bits"] == 2 and not m["act_padding"]
            xb = cap["x"].to(torch.bfloat16)
            groups = xb.reshape(BATCH, -1, g)
            packed, scale, xmin = torch.ops.act_lib.quant_pack_triton(groups, 2, g, False, 0, True, 3.0)
            x_hat = torch.ops.act_lib.dequant_unpack_triton(packed, scale, xmin, 2, g, False, 0).float()
            dyf = cap["dy"].float().reshape(-1, fc1.weight.shape[0])
            want = dyf.t() @ x_hat.reshape(-1, fc1.weight.shape[1])
            err = rel_err(fc1.weight.grad, want)
            print(f"[config 5] fc1 dW rel err {err:.2e}", flush=True)
            assert err <= 1e-2
        opt.step()
        losses.append(loss.item())

    print("[config 5] saved-activation bytes", flush=True)
    opt.zero_grad(set_to_none=True)
    plain.zero_grad(set_to_none=True)
    pb = saved_bytes(plain, x)
    cb = saved_bytes(model, x)
    print(f"[config 5] saved bytes plain {pb}, compressed {cb} ({cb / pb:.3f}x); losses {losses}", flush=True)
    assert cb < 0.6 * pb
