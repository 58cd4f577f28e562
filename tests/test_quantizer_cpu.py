"""The reference's Quantizer / Controller call API on the CPU (Activation_Compression/quantizer.py:
13-80, :170-288; controller.py:19-61, :63-351): construction with test=False, iterate, warp_model
with its reference default (quantizer=False), the DIVISION layer analysis, and the configuration
errors. The LFER statistics are pinned by values worked out by hand on tiny tensors.
"""
import pytest
import torch
import torch.nn.functional as F
from torch import nn

from deep_optimization_amd.controller import Controller
from deep_optimization_amd.layers import DOConv2d, RMSNorm
from deep_optimization_amd.modules.activations import DOReLU_Variance
from deep_optimization_amd.quantizer import Quantizer, lfer_of_act, lfer_of_grad


@pytest.fixture
def restore_matmul_flags():
    flags = (torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32,
             torch.get_float32_matmul_precision())
    yield
    torch.backends.cuda.matmul.allow_tf32, torch.backends.cudnn.allow_tf32 = flags[:2]
    torch.set_float32_matmul_precision(flags[2])


def test_quantizer_table():
    q = Quantizer({"default_bits": 2, "auto_precision": None}, {"a": None, "b": 8})
    assert q.default_bit == 2 and q.graph_mode is False and q.dims == {}
    q.iterate()
    assert q.bits == {"a": 2, "b": 2}
    q.clean_iterate()
    assert q.bits == {} and q.dims == {}
    with pytest.raises(NotImplementedError, match="auto_precision"):
        Quantizer({"default_bits": 2, "auto_precision": "hessian"}, {"a": 1}).iterate()


def test_quantizer_check_quantize():
    lin = nn.Linear(4, 4)
    q = Quantizer({"default_bits": 2}, {})
    q.filter_tensors(lin.named_parameters())
    assert len(q.unrelated_tensors) == 2
    assert not q.check_quantize(lin.weight)
    x = torch.randn(2, 4, requires_grad=True)
    assert q.check_quantize(x)
    assert not q.check_quantize(x.detach())
    assert not q.check_quantize(torch.randn(2, 2, 2, 2, 2, requires_grad=True))
    assert not q.check_quantize(torch.randn(4, requires_grad=True))
    assert not q.check_quantize(torch.zeros(2, 4, dtype=torch.uint8))
    assert q.check_quantize(torch.randn(2, 3, 4, dtype=torch.bfloat16, requires_grad=True))


def test_lfer_known_answers():
    # gradients: 2-D row mean; 3-D length-4 pool with stride 3 over the last axis; 4-D 3x3 kernel
    assert lfer_of_grad(torch.tensor([[1.0, 3.0], [2.0, 2.0]])) == pytest.approx(16 / 18, rel=1e-6)
    g3 = torch.arange(1.0, 11.0).reshape(1, 1, 10)
    # windows [1..4], [4..7], [7..10] -> 2.5, 5.5, 8.5, nearest-expanded to 4 + 3 + 3 positions
    assert lfer_of_grad(g3) == pytest.approx((4 * 6.25 + 3 * 30.25 + 3 * 72.25) / 385, rel=1e-6)
    g4 = torch.arange(1.0, 10.0).reshape(1, 1, 3, 3)
    assert lfer_of_grad(g4) == pytest.approx(9 * 25 / 285, rel=1e-6)
    assert lfer_of_grad(torch.randn(8, 4, 1, 1)) == 1
    assert lfer_of_grad(torch.randn(8, 1)) == 1
    # activations: 4-D 4x4 pool; 3-D length-4 pool with stride 4; 2-D feature mean
    assert lfer_of_act(torch.arange(16.0).reshape(1, 1, 4, 4)) == pytest.approx(900 / 1240, rel=1e-6)
    assert lfer_of_act(torch.arange(8.0).reshape(1, 1, 8)) == pytest.approx(130 / 140, rel=1e-6)
    assert lfer_of_act(torch.tensor([[1.0, 3.0]])) == pytest.approx(8 / 10, rel=1e-6)
    # a checkerboard has no energy below the pooling frequency
    cb = (torch.arange(4).reshape(4, 1) + torch.arange(4)) % 2 * 2.0 - 1
    assert lfer_of_act(cb.reshape(1, 1, 4, 4)) == pytest.approx(0.0, abs=1e-9)


class _Cnn(nn.Module):
    def __init__(self):
        super().__init__()
        self.conv1 = nn.Conv2d(3, 32, 3, padding=1, bias=False)
        self.bn1 = nn.BatchNorm2d(32)
        self.act1 = nn.ReLU()
        self.conv2 = nn.Conv2d(32, 32, 3, padding=1)
        self.act2 = nn.SiLU()
        self.pool = nn.AdaptiveAvgPool2d(4)
        self.fc = nn.Linear(32 * 16, 10)

    def forward(self, x):
        x = self.act2(self.conv2(self.act1(self.bn1(self.conv1(x)))))
        return self.fc(self.pool(x).flatten(1))


def _loader(batch=64, n_batches=2, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [(torch.randn(batch, 3, 64, 64, generator=g), torch.randint(0, 10, (batch,), generator=g))
            for _ in range(n_batches)]


def test_reference_call_sequence(restore_matmul_flags):
    """Trainer.py:179-183 / test8.ipynb cell 2 with test8's configuration keys."""
    torch.manual_seed(0)
    model = _Cnn()
    config = {"default_bits": 2, "auto_precision": None, "DIVISION": {"pool_kernel_size": 3}, "group_size": 256,
              "batch_size": 64, "fp8": False, "depth_point_conv": False, "rms_norm": False}
    loader = _loader()
    criterion = nn.CrossEntropyLoss()
    grads_before = [p.grad for p in model.parameters()]
    c = Controller(model, config, loader, criterion, test=False, device="cpu")
    # the constructor analyses and traces, swaps nothing, and seeds the quantizer's table
    assert all(g is None for g in grads_before) and all(p.grad is None for p in model.parameters())
    assert not any(isinstance(m, (DOConv2d, DOReLU_Variance)) for m in c.traced_model.modules())
    targets = {"act1", "act2", "bn1", "conv1", "conv2"}
    assert set(c.quantizer.bits) == targets
    assert set(c.low_frequency_energy_ratio_grad) == {"conv1", "conv2", "fc"}
    c.iterate(criterion)
    assert c.quantizer.bits == {t: 2 for t in targets}
    c.warp_model(graph_mode=True, quantizer=True)
    model = c.traced_model
    mods = dict(model.named_modules())
    assert type(mods["conv1"]) is DOConv2d and type(mods["act1"]) is DOReLU_Variance
    assert c.quantizer.graph_mode and torch.backends.cuda.matmul.allow_tf32
    # DIVISION goes to the selected Conv/Linear layers whose gradient LFER exceeds the 75th
    # percentile of the (non-1) gradient LFERs
    lf = c.low_frequency_energy_ratio_grad
    vals = sorted(v for v in lf.values() if v != 1)
    assert len(vals) == 3
    # torch.quantile(q=0.75) of 3 sorted values interpolates halfway between the 2nd and 3rd
    assert c.base_division_threshold_grad == pytest.approx(vals[1] + 0.5 * (vals[2] - vals[1]), rel=1e-6)
    for t in targets:
        want = config["DIVISION"] if t in lf and lf[t] > c.base_division_threshold_grad and lf[t] != 1 else None
        assert c.meta[t]["DIVISION"] == want, t
    assert sum(c.meta[t]["DIVISION"] is not None for t in targets) <= 1
    # a second rewrite leaves the compressed layers as they are
    before = {n: m for n, m in c.traced_model.named_modules()}
    c.warp_model(quantizer=True)
    after = dict(c.traced_model.named_modules())
    assert after["conv1"] is before["conv1"] and after["act1"] is before["act1"]


def test_division_statistics_match_a_direct_computation():
    """The analysis's gradient LFERs equal those of a plain bf16-autocast backward on the same
    64 samples, and its activation LFERs those of the layer inputs."""
    torch.manual_seed(1)
    model = _Cnn()
    loader = _loader(seed=3)
    q = Quantizer({"default_bits": 2}, {})
    lf_g, lf_a, lars, snr, var = q.select_division_layer_helper(model, nn.CrossEntropyLoss(), loader, device="cpu")
    x, y = loader[0]
    inputs = {}
    hooks = [getattr(model, n).register_forward_hook(lambda m, i, o, n=n: inputs.__setitem__(n, i[0]))
             for n in ("conv1", "conv2", "fc")]
    with torch.autocast("cpu", dtype=torch.bfloat16):
        loss = F.cross_entropy(model(x), y)
    loss.backward()
    for h in hooks:
        h.remove()
    for n in ("conv1", "conv2", "fc"):
        w = getattr(model, n).weight
        assert lf_g[n] == pytest.approx(lfer_of_grad(w.grad), rel=1e-5), n
        assert lf_a[n] == pytest.approx(lfer_of_act(inputs[n]), rel=1e-5), n
        assert lars[n] == pytest.approx(w.norm().item() / (w.grad.norm().item() + 1e-7), rel=1e-5)
        assert var[n] == pytest.approx(inputs[n].var().item(), rel=1e-3)
        assert snr[n] >= 0
    # the analysis leaves no hook behind
    assert all(not getattr(model, n)._forward_hooks for n in ("conv1", "conv2", "fc"))


def test_config_errors():
    base = {"default_bits": 2, "batch_size": 64}
    with pytest.raises(NotImplementedError, match="depth_point_conv"):
        Controller(_Cnn(), dict(base, depth_point_conv=True), input_shape=(3, 64, 64), device="cpu").warp_model()
    with pytest.raises(NotImplementedError, match="rms_norm"):
        Controller(_Cnn(), dict(base, rms_norm=True), input_shape=(3, 64, 64), device="cpu").warp_model()
    with pytest.raises(ValueError, match="train_loader and criterion"):
        Controller(_Cnn(), base, input_shape=(3, 64, 64), test=False, device="cpu")
    c = Controller(_Cnn(), dict(base, auto_precision="hessian"), input_shape=(3, 64, 64), device="cpu")
    with pytest.raises(NotImplementedError, match="auto_precision"):
        c.warp_model(quantizer=True)


def test_warp_model_default_swaps_nothing():
    c = Controller(_Cnn(), {"default_bits": 2, "batch_size": 64}, input_shape=(3, 64, 64), device="cpu")
    c.warp_model()
    assert not any(isinstance(m, (DOConv2d, DOReLU_Variance)) for m in c.traced_model.modules())
    assert not any(isinstance(v, dict) for v in c.meta.values())


def test_rmsnorm_layer():
    torch.manual_seed(2)
    m = RMSNorm(8)
    with torch.no_grad():
        m.weight.uniform_(0.5, 1.5)
    x = torch.randn(3, 5, 8, dtype=torch.float64)
    want = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-8) * m.weight.double()
    torch.testing.assert_close(m.double()(x), want, rtol=1e-12, atol=0)
