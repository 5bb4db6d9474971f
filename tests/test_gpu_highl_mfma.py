"""GPU parity of the high-degree bf16 path (csrc/edgewise_hl.hip) at BASELINE
config 5's representation: in = out = Repr(range(7), C) with C = 64 and 128
(config 5's own), bf16 features and bases.

The float64 oracle runs on the same bf16-rounded inputs; outputs and every
gradient (edge features, channel patterns, radial MLP, distances) must agree
to the north-star bf16 bar, 2e-2 (max|diff| / max|ref|).  The library's
launch log confirms that the high-degree kernels, not the shape-generic ones,
produced the results.
"""
import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from helpers import rel_err
from oracle import layer as OL
from oracle import wigner as OW

pytestmark = pytest.mark.gpu
L6 = list(range(7))
BF16_TOL = 2e-2


@pytest.mark.parametrize("C,E,seed,log", [(64, 300, 1, False), (128, 97, 2, False), (64, 500, 3, True)])
def test_high_degree_bf16_matches_oracle(dev, C, E, seed, log):
    """log: logarithmic bins (min_dist 0.5), distances from 0.05 to 12.05."""
    torch.manual_seed(seed)
    rp = fe.Repr(L6, C)
    kw = dict(log_bins=True, min_dist=0.5) if log else {}
    layer = fe.EquivariantEdgewiseLinear(rp, rp, num_bins=100, **kw).to(dev)
    g = torch.Generator().manual_seed(seed + 50)
    x = torch.randn(E, C, 49, generator=g).bfloat16()
    d = torch.randn(E, 3, generator=g)
    r = torch.rand(E, generator=g) * (12.0 if log else 9.5) + 0.05
    P = OW.basis(L6, d).float().bfloat16()
    xg = x.to(dev).requires_grad_(True)
    rg = r.to(dev).requires_grad_(True)
    NAT.profile_summary()
    NAT.profile_enable(True)
    y = layer(P.to(dev), P.to(dev), xg, rg)
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev).bfloat16())
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert "k_hl_mix" in launched and "k_hl_dfe" in launched and "k_hl_mix_t" in launched, launched
    assert y.dtype == torch.bfloat16 and xg.grad.dtype == torch.bfloat16

    params, cfg = OL.module_cfg(layer)
    xd = x.double().requires_grad_(True)
    rd = r.double().requires_grad_(True)
    Pd = P.double()
    yref = OL.edgewise_linear(xd, Pd, Pd, rd, params, cfg)
    yref.backward(gy.bfloat16().double())
    assert rel_err(y, yref) < BF16_TOL
    assert rel_err(xg.grad, xd.grad) < BF16_TOL
    assert rel_err(rg.grad, rd.grad) < BF16_TOL
    for name, p in layer.radial_weights.named_parameters():
        assert rel_err(p.grad, params[name].grad) < BF16_TOL, name


def test_high_degree_edges_past_a_tile_and_empty(dev):
    """E not a multiple of the 16-edge tile, and E = 0 (zero parameter gradients)."""
    torch.manual_seed(7)
    rp = fe.Repr(L6, 64)
    layer = fe.EquivariantEdgewiseLinear(rp, rp, num_bins=100).to(dev)
    for E in (1, 17):
        g = torch.Generator().manual_seed(E)
        x = torch.randn(E, 64, 49, generator=g).bfloat16()
        d = torch.randn(E, 3, generator=g)
        r = torch.rand(E, generator=g) * 9
        P = OW.basis(L6, d).float().bfloat16()
        xg = x.to(dev).requires_grad_(True)
        y = layer(P.to(dev), P.to(dev), xg, r.to(dev))
        y.float().pow(2).sum().backward()
        params, cfg = OL.module_cfg(layer)
        xd = x.double().requires_grad_(True)
        yref = OL.edgewise_linear(xd, P.double(), P.double(), r.double(), params, cfg)
        yref.pow(2).sum().backward()
        assert rel_err(y, yref) < BF16_TOL
        assert rel_err(xg.grad, xd.grad) < BF16_TOL
        layer.zero_grad()
    x0 = torch.zeros(0, 64, 49, dtype=torch.bfloat16, device=dev, requires_grad=True)
    P0 = torch.zeros(0, 49, 49, dtype=torch.bfloat16, device=dev)
    y0 = layer(P0, P0, x0, torch.zeros(0, device=dev))
    assert y0.shape == (0, 64, 49)
    y0.float().sum().backward()
    for p in layer.radial_weights.parameters():
        assert p.grad is None or torch.all(p.grad == 0)


def test_high_degree_dense_bases(dev):
    """Bases with entries off the degree blocks (any P, Q is accepted): the
    rotations then sum over every entry, read from global memory."""
    torch.manual_seed(9)
    rp = fe.Repr(L6, 64)
    layer = fe.EquivariantEdgewiseLinear(rp, rp, num_bins=100).to(dev)
    g = torch.Generator().manual_seed(90)
    E = 37
    x = torch.randn(E, 64, 49, generator=g).bfloat16()
    P = (torch.randn(E, 49, 49, generator=g) / 7).bfloat16()
    Q = (torch.randn(E, 49, 49, generator=g) / 7).bfloat16()
    r = torch.rand(E, generator=g) * 9 + 0.1
    xg = x.to(dev).requires_grad_(True)
    y = layer(P.to(dev), Q.to(dev), xg, r.to(dev))
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev).bfloat16())
    params, cfg = OL.module_cfg(layer)
    xd = x.double().requires_grad_(True)
    yref = OL.edgewise_linear(xd, P.double(), Q.double(), r.double(), params, cfg)
    yref.backward(gy.bfloat16().double())
    assert rel_err(y, yref) < BF16_TOL
    assert rel_err(xg.grad, xd.grad) < BF16_TOL
