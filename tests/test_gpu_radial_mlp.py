"""The radial network of SeparableRadialNet at the bin edges as one-workgroup
kernels (RadialMLPFn: feq_radial_fwd / feq_radial_bwd) against the same network
in float64 PyTorch (radial.py:200-275): the table F and the six parameter
gradients within float32 rounding of sums of at most a few hundred terms
(1e-6 / 1e-5 of the largest value), the same bits on every call, and the layer
falling back to PyTorch where the kernels do not take the shape."""
import pytest
import torch

import flash_eq as fe
from flash_eq import ops
from helpers import rel_err

pytestmark = pytest.mark.gpu


def _ref(net, basis, gF):
    t = net.trunk
    ps = [p.detach().double().requires_grad_(True)
          for p in (t[0].weight, t[0].bias, t[2].weight, t[2].bias, net.head.weight, net.head.bias)]
    b = basis.detach().double()
    h = torch.nn.functional.silu(b @ ps[0].t() + ps[1])
    h = torch.nn.functional.silu(h @ ps[2].t() + ps[3])
    F = h @ ps[4].t() + ps[5]
    F.backward(gF.double())
    return F.detach(), [p.grad for p in ps]


@pytest.mark.parametrize("num_bins,rank,wdim,hidden", [(100, 4, 19, 64), (100, 4, 10, 64), (16, 4, 3, 64),
                                                      (50, 2, 7, 32), (100, 4, 231, 64), (7, 3, 5, 300)])
def test_fused_radial_network(dev, num_bins, rank, wdim, hidden):
    torch.manual_seed(num_bins + wdim)
    net = fe.layers.radial.SeparableRadialNet(num_bins=num_bins, out_mult=8, in_mult=8, weight_dim=wdim,
                                              rank=rank, hidden_dim=hidden).to(dev)
    basis = net._edge_basis()
    assert net._fused_mlp_ok(basis)
    gF = torch.randn(num_bins + 1, rank * wdim, device=dev)
    t = net.trunk
    params = [t[0].weight, t[0].bias, t[2].weight, t[2].bias, net.head.weight, net.head.bias]
    outs = []
    for _ in range(2):
        for p in params:
            p.grad = None
        F = net.radial_functions()
        F.view(num_bins + 1, -1).backward(gF)
        outs.append((F.detach().clone(), [p.grad.clone() for p in params]))
    Fr, gr = _ref(net, basis, gF)
    assert rel_err(outs[0][0].view(num_bins + 1, -1), Fr) < 1e-6
    for a, b in zip(outs[0][1], gr):
        assert rel_err(a, b) < 1e-5
    assert torch.equal(outs[0][0], outs[1][0])
    for a, b in zip(outs[0][1], outs[1][1]):
        assert torch.equal(a, b)


def test_radial_network_fallback_and_basis_cache(dev):
    """Over 4096 outputs the kernels decline and PyTorch's layers run, as they do
    for float64 parameters; the cached basis follows a change of the bin edges."""
    torch.manual_seed(3)
    net = fe.layers.radial.SeparableRadialNet(num_bins=100, out_mult=8, in_mult=8, weight_dim=1100,
                                              rank=4).to(dev)
    basis = net._edge_basis()
    assert not net._fused_mlp_ok(basis)
    F = net.radial_functions()
    assert F.shape == (101, 4, 1100)
    assert not net.to(torch.float64)._fused_mlp_ok(net._edge_basis())
    net = net.to(torch.float32)          # new buffers: the basis is formed again, then kept
    basis = net._edge_basis()
    assert net._edge_basis() is basis
    with torch.no_grad():
        net.bin_edges.mul_(0.5)
    b2 = net._edge_basis()
    assert b2 is not basis
    assert rel_err(b2, net._sinusoidal_basis(net.bin_edges)) == 0.0
