"""Controller model rewrite on the CPU: fx trace, FakeTensor shape propagation, the > 10 MiB
selection rule, per-layer meta and the module swap (reference Activation_Compression/controller.py:
63-351). No compressed forward runs here (the act_lib operators need the GPU); eval-mode forwards,
which are the plain torch layers, do.

Expected layer lists and meta values are worked out by hand from the ViT-B/16 shapes at batch 128:
patch conv output [128, 768, 14, 14] bf16 = 36.75 MiB, qkv output [128, 197, 2304] = 110.8 MiB,
proj / fc2 outputs [128, 197, 768] = 36.9 MiB, fc1 / GELU outputs [128, 197, 3072] = 147.8 MiB,
head output [128, 1000] = 0.24 MiB (not selected).
"""
import pytest
import torch
from torch import nn

from deep_optimization_amd.controller import Controller
from deep_optimization_amd.layers import DOConv1d, DOConv2d, DOConv3d, DOLinear
from deep_optimization_amd.modules.activations import DOGELU, DOReLU_Variance, DOSiLU
from deep_optimization_amd.modules.normalization import DOBatchNorm2d
from deep_optimization_amd.vit import vit_base_patch16_224


@pytest.fixture(scope="module")
def vit_controller():
    torch.manual_seed(0)
    model = vit_base_patch16_224()
    ref_state = {k: v.clone() for k, v in model.state_dict().items()}
    c = Controller(model, {"batch_size": 128, "default_bits": 2}, input_shape=(3, 224, 224), device="cpu")
    c.warp_model(quantizer=True)
    return c, ref_state


def _targets(c):
    return sorted(k for k, v in c.meta.items() if isinstance(v, dict))


def test_vit_selection(vit_controller):
    c, _ = vit_controller
    want = ["patch_embed.proj"] + [f"blocks.{i}.{n}" for i in range(12)
                                   for n in ("attn.qkv", "attn.proj", "mlp.fc1", "mlp.act", "mlp.fc2")]
    assert _targets(c) == sorted(want)
    assert "head" not in c.meta
    assert c.meta["batch_size"] == 128 and c.meta["group_size"] == 256


def test_vit_meta_values(vit_controller):
    c, _ = vit_controller
    # patch conv input [128, 3, 224, 224]: S = 150528 = 294 * 512
    m = c.meta["patch_embed.proj"]
    assert (m["group_size"], m["act_padding"], m["N"], m["NG"]) == (512, False, 128, 128 * 294)
    for i in (0, 11):
        for name in ("attn.qkv", "attn.proj", "mlp.fc1"):  # input [128, 197, 768]: S = 151296 = 591 * 256
            m = c.meta[f"blocks.{i}.{name}"]
            assert (m["group_size"], m["act_padding"], m["N"], m["NG"]) == (256, False, 128, 128 * 591)
            assert tuple(m["tensor_meta"].shape) == (128, 197, 768)
        for name in ("mlp.act", "mlp.fc2"):  # input [128, 197, 3072]: S = 605184 = 1182 * 512
            m = c.meta[f"blocks.{i}.{name}"]
            assert (m["group_size"], m["NG"]) == (512, 128 * 1182)
    for k in _targets(c):
        m = c.meta[k]
        assert m["bits"] == 2 and not m["pack_only"] and m["AVG_ALAM"] is False and m["ALAM_BITS"] == 0
        assert m["DIVISION"] is None


def test_vit_swap_and_weights(vit_controller):
    c, ref_state = vit_controller
    tm = c.traced_model
    mods = dict(tm.named_modules())
    assert type(mods["patch_embed.proj"]) is DOConv2d and mods["patch_embed.proj"].bias is not None
    assert type(mods["blocks.3.attn.qkv"]) is DOLinear and type(mods["blocks.3.mlp.act"]) is DOGELU
    assert type(mods["head"]) is nn.Linear
    assert mods["blocks.5.mlp.fc1"].target_name == "blocks.5.mlp.fc1"
    assert mods["blocks.5.mlp.fc1"].meta is c.meta and mods["blocks.5.mlp.fc1"].clamp_alpha == 3.0
    state = tm.state_dict()
    for k, v in ref_state.items():
        assert torch.equal(state[k], v), k
    assert tm.training


class _Cnn(nn.Module):
    def __init__(self):
        super().__init__()
        self.conv1 = nn.Conv2d(3, 32, 3, padding=1, bias=False)
        self.bn1 = nn.BatchNorm2d(32)
        self.act1 = nn.ReLU()
        self.conv2 = nn.Conv2d(32, 32, 3, padding=1, padding_mode="reflect")
        self.act2 = nn.SiLU()
        self.conv1d = nn.Conv1d(32, 16, 3, padding="same")
        self.fc = nn.Linear(16 * 64 * 64, 10)

    def forward(self, x):
        x = self.act2(self.conv2(self.act1(self.bn1(self.conv1(x)))))
        x = self.conv1d(x.flatten(2)[:, :, :4096])
        return self.fc(x.flatten(1))


def test_cnn_relu_mask_only_and_bits_override():
    torch.manual_seed(1)
    model = _Cnn()
    c = Controller(model, {"batch_size": 32, "default_bits": 2, "bits": {"conv2": 4}}, input_shape=(3, 64, 64),
                   device="cpu")
    c.warp_model(quantizer=True)
    # outputs: conv1 / bn1 / relu / conv2 / silu [32, 32, 64, 64] bf16 = 8 MiB -> none selected
    assert _targets(c) == []
    c = Controller(_Cnn(), {"batch_size": 64, "default_bits": 2, "bits": {"conv2": 4}}, input_shape=(3, 64, 64),
                   device="cpu")
    c.warp_model(quantizer=True)
    assert _targets(c) == ["act1", "act2", "bn1", "conv1", "conv2"]
    assert c.meta["act1"]["pack_only"] and c.meta["act1"]["bits"] == 1
    # BatchNorm groups per channel: S = N*H*W = 64*64*64 = 256 * 1024, N = C = 32
    m = c.meta["bn1"]
    assert (m["group_size"], m["act_padding"], m["N"], m["NG"]) == (1024, False, 32, 32 * 256)
    assert c.meta["conv2"]["bits"] == 4 and c.meta["act2"]["bits"] == 2
    mods = dict(c.traced_model.named_modules())
    assert type(mods["act1"]) is DOReLU_Variance and type(mods["act2"]) is DOSiLU
    assert type(mods["conv2"]) is DOConv2d and mods["conv2"].padding_mode == "reflect"
    assert mods["conv1"].bias is None and mods["conv2"].bias is not None
    assert type(mods["bn1"]) is DOBatchNorm2d and mods["bn1"].target_name == "bn1"


def test_eval_forward_equals_original():
    """DO* layers (other than DOGELU, which is the tanh GELU) are the plain layers in eval mode."""
    torch.manual_seed(2)
    model = _Cnn().eval()
    x = torch.randn(2, 3, 64, 64)
    with torch.no_grad():
        want = model(x)
    c = Controller(model, {"batch_size": 64, "default_bits": 2}, input_shape=(3, 64, 64), device="cpu")
    tm = c.warp_model(quantizer=True).eval()
    with torch.no_grad():
        got = tm(x)
    torch.testing.assert_close(got, want, rtol=0, atol=0)


def test_quantizer_false_traces_without_swapping():
    c = Controller(_Cnn(), {"batch_size": 64, "default_bits": 2}, input_shape=(3, 64, 64), device="cpu")
    tm = c.warp_model(quantizer=False)
    assert not any(isinstance(m, (DOLinear, DOConv2d, DOReLU_Variance)) for m in tm.modules())
    assert set(c.target_dict) == {"act1", "act2", "bn1", "conv1", "conv2"}


def test_conv_layers_construct_like_torch():
    for cls, base, shape in ((DOConv1d, nn.Conv1d, (2, 4, 9)), (DOConv2d, nn.Conv2d, (2, 4, 9, 9)),
                             (DOConv3d, nn.Conv3d, (2, 4, 5, 5, 5))):
        torch.manual_seed(3)
        m = cls(4, 6, 3, stride=1, padding=1, bias=True)
        ref = base(4, 6, 3, stride=1, padding=1, bias=True)
        ref.load_state_dict(m.state_dict())
        x = torch.randn(*shape) * 0.5  # inside the eval clamp of DOConv1d / DOConv3d
        m.eval()
        with torch.no_grad():
            torch.testing.assert_close(m(x), ref(x), rtol=0, atol=0)
    lin = DOLinear(8, 4, target_name="fc")
    assert lin.bias is not None and lin.clamp_alpha == 3.0 and lin.ema_grad_meta is None


def test_controller_needs_an_input_shape():
    with pytest.raises(ValueError):
        Controller(_Cnn(), {"batch_size": 4, "default_bits": 2}, device="cpu")
    loader = [(torch.zeros(4, 3, 64, 64), torch.zeros(4, dtype=torch.long))]
    c = Controller(_Cnn(), {"batch_size": 4, "default_bits": 2}, train_loader=loader, device="cpu")
    assert c.input_shape == (3, 64, 64)


def test_batchnorm_swap_keeps_state_and_fuse_bn_act():
    from deep_optimization_amd.fusion import DOBatchNormReLU2d, fuse_bn_act

    torch.manual_seed(4)
    model = _Cnn()
    with torch.no_grad():
        model.bn1.weight.uniform_(0.5, 1.5)
        model.bn1.bias.uniform_(-0.5, 0.5)
        model.bn1.running_mean.uniform_(-1, 1)
        model.bn1.running_var.uniform_(0.5, 2)
    ref = {k: v.clone() for k, v in model.bn1.state_dict().items()}
    x = torch.randn(2, 3, 64, 64)
    model.eval()
    with torch.no_grad():
        want = model(x)
    c = Controller(model, {"batch_size": 64, "default_bits": 2}, input_shape=(3, 64, 64), device="cpu")
    tm = c.warp_model(quantizer=True)
    for k, v in ref.items():
        assert torch.equal(tm.bn1.state_dict()[k], v), k
    fused = fuse_bn_act(tm)
    mods = dict(fused.named_modules())
    assert type(mods["bn1_bnact"]) is DOBatchNormReLU2d and "bn1" not in mods and "act1" not in mods
    assert "bn1_bnact" in c.meta and "bn1" not in c.meta
    assert mods["bn1_bnact"].target_name == "bn1_bnact" and c.meta["bn1_bnact"]["group_size"] == 1024
    for k, v in ref.items():
        assert torch.equal(mods["bn1_bnact"].state_dict()[k], v), k
    fused.eval()
    with torch.no_grad():
        torch.testing.assert_close(fused(x), want, rtol=0, atol=0)


def test_resnet50_selection_and_swap():
    """ResNet-50 at batch 64: every Conv / BatchNorm / ReLU whose output exceeds 10 MiB
    (controller.py's threshold) becomes its DO* counterpart: 37 convolutions, 37 BatchNorms and
    33 ReLUs; ReLUs keep 1-bit masks only, the others 2-bit codes of their saved input; small
    late-stage layers stay torch's."""
    from deep_optimization_amd.resnet import resnet50

    torch.manual_seed(0)
    c = Controller(resnet50(), {"batch_size": 64, "default_bits": 2}, input_shape=(3, 224, 224), device="cpu")
    model = c.warp_model(quantizer=True)
    kinds = {}
    for name, mod in model.named_modules():
        if name in c.meta:
            kinds[type(mod).__name__] = kinds.get(type(mod).__name__, 0) + 1
    assert kinds == {"DOConv2d": 37, "DOBatchNorm2d": 37, "DOReLU_Variance": 33}
    for k in _targets(c):
        m = c.meta[k]
        assert m["tensor_meta"].shape[0] == 64
        if k.split(".")[-1].startswith("relu"):
            assert m["pack_only"] and m["bits"] == 1
        else:
            assert not m["pack_only"] and m["bits"] == 2
    # output sizes decide: layer3.0.conv3 writes [64, 1024, 14, 14] (25.7 MB, selected), its 3x3
    # conv2 [64, 256, 14, 14] (6.4 MB, not), and so on down to layer4's [64, 512, 7, 7]
    assert "conv1" in c.meta and "bn1" in c.meta and "layer1.0.conv1" in c.meta
    assert "layer3.0.conv3" in c.meta and tuple(c.meta["layer3.0.conv3"]["tensor_meta"].shape) == (64, 256, 14, 14)
    assert "layer3.0.conv2" not in c.meta and "layer4.2.conv2" not in c.meta
    assert isinstance(model.get_submodule("layer1.0.bn1"), DOBatchNorm2d)
    assert isinstance(model.get_submodule("layer4.2.conv2"), nn.Conv2d)
