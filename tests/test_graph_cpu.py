"""Weight-noise helpers of the captured training step (deep_optimization_amd.graph), on the CPU.

Mirrors Activation_Compression/cuda_graph_utils.py:123-170. Pinned by invariants of the
reference's formula p += alpha * (|p| / |theta|) * theta with theta ~ U(-alpha, alpha):
  * the added noise has L2 norm alpha * |p| (per parameter);
  * it is parallel to a draw that lies in [-alpha, alpha] (the noise divided by its own scale);
  * denoise restores p up to the rounding of one fp32 add and subtract;
  * every trainable parameter gets a buffer, BatchNorm ones included (the reference's BatchNorm2d
    test never excludes anything), frozen ones do not.
"""
import pytest
import torch
import torch.nn as nn

from deep_optimization_amd.graph import NODE_TYPES, denoise, inject_noise, prepare_theta


def small_model():
    torch.manual_seed(0)
    m = nn.Sequential(nn.Conv2d(3, 8, 3), nn.BatchNorm2d(8), nn.ReLU(), nn.Flatten(), nn.Linear(8 * 6 * 6, 10))
    m[0].bias.requires_grad_(False)
    return m


def test_prepare_theta_covers_trainable_parameters():
    m = small_model()
    prepare_theta(m)
    for name, p in m.named_parameters():
        assert hasattr(p, "_theta") == p.requires_grad, name
        if p.requires_grad:
            assert p._theta.shape == p.shape and p._theta.dtype == p.dtype
    bufs = {id(p._theta) for p in m.parameters() if hasattr(p, "_theta")}
    prepare_theta(m)  # buffers are kept: a captured graph holds their addresses
    assert bufs == {id(p._theta) for p in m.parameters() if hasattr(p, "_theta")}


@pytest.mark.parametrize("alpha", [0.0375, 0.2])
def test_inject_and_denoise(alpha):
    m = small_model()
    prepare_theta(m)
    before = {n: p.detach().clone() for n, p in m.named_parameters()}
    torch.manual_seed(123)
    inject_noise(m, alpha=alpha)
    # the same generator stream, drawn independently: the theta of each trainable parameter in order
    torch.manual_seed(123)
    thetas = {n: torch.empty_like(p).uniform_(-alpha, alpha) for n, p in m.named_parameters() if p.requires_grad}
    for n, p in m.named_parameters():
        if not p.requires_grad:
            assert torch.equal(p, before[n]) and not hasattr(p, "_noise"), n
            continue
        assert p._denoise is True
        noise = p._noise.double()
        # what was added is the noise, up to one fp32 rounding per element
        added = p.detach().double() - before[n].double()
        ulp = torch.finfo(torch.float32).eps * (p.detach().double().abs() + noise.abs())
        assert bool(((added - noise).abs() <= ulp).all()), n
        # |noise| = alpha |p|, and noise = c * theta for one constant c > 0
        pn = before[n].double().norm().item()
        assert abs(noise.norm().item() - alpha * pn) <= 1e-5 * alpha * pn, n
        if pn == 0:  # a zero parameter (BatchNorm bias at init) gets zero noise
            assert not noise.any(), n
            continue
        th = thetas[n].double()
        c = (noise * th).sum() / (th * th).sum()
        assert c > 0 and bool(((noise - c * th).abs() <= 1e-6 * noise.abs().max()).all()), n
    draws = [p._noise.clone() for p in m.parameters() if p.requires_grad]
    denoise(m)
    for n, p in m.named_parameters():
        assert not hasattr(p, "_noise") and not hasattr(p, "_denoise")
        ulp = 2 * torch.finfo(torch.float32).eps * (before[n].abs() + 1)
        assert bool(((p.detach() - before[n]).abs() <= ulp).all()), n
    # a second injection draws new noise
    inject_noise(m, alpha=alpha)
    again = [p._noise for p in m.parameters() if p.requires_grad]
    assert all(not torch.equal(a, b) for a, b in zip(draws, again) if a.any())
    denoise(m)


def test_node_type_names_follow_hip_enum():
    # hipGraphNodeType: Kernel 0, Memcpy 1, Memset 2, ..., BatchMemOp 14
    assert NODE_TYPES[0] == "kernel" and NODE_TYPES[2] == "memset" and NODE_TYPES[4] == "graph"
    assert len(NODE_TYPES) == 15
