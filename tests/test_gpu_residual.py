"""The transformer block's residual connection with LayerScale in one pass
(feq_scale_add / feq_scale_add_bwd, ops.ResidualScaleFn).

The reference writes it as x + drop_path(layer_scale(y)) (transformer.py:245,
:252; LayerScale :23-38) and autograd forms grad_x = g, grad_y = gamma g and
grad_gamma = sum g y.  Checked against those float64 formulas: out, grad_x and
grad_y at float32 rounding (1e-6 relative), grad_gamma at 1e-6 relative (its
products and sum in float64), ragged lengths (vectorised body and scalar
tail), gamma without gradient, and the block's launch log (the fused
kernels, no elementwise multiply for the layer scale).
"""
import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from flash_eq.ops import ResidualScaleFn
from helpers import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [4096 * 9, 1001, 3, 0])
def test_matches_float64(dev, n):
    g = torch.Generator().manual_seed(n + 1)
    x, y, go = (torch.randn(n, generator=g) for _ in range(3))
    gamma = torch.tensor(0.37)
    xd, yd = x.to(dev).requires_grad_(True), y.to(dev).requires_grad_(True)
    gd = gamma.to(dev).requires_grad_(True)
    out = ResidualScaleFn.apply(xd, yd, gd)
    out.backward(go.to(dev))
    if n == 0:
        assert out.shape == (0,) and xd.grad.shape == (0,) and yd.grad.shape == (0,)
        assert gd.grad.item() == 0.0
        return
    ref = x.double() + gamma.double() * y.double()
    assert rel_err(out, ref) < 1e-6
    assert torch.equal(xd.grad.cpu(), go)
    assert rel_err(yd.grad, gamma.double() * go.double()) < 1e-6
    gg = (go.double() * y.double()).sum()
    assert abs(gd.grad.item() - gg.item()) <= 1e-6 * (go.double() * y.double()).abs().sum().item()


def test_gamma_without_gradient(dev):
    x = torch.randn(5000, device=dev, requires_grad=True)
    y = torch.randn(5000, device=dev, requires_grad=True)
    gamma = torch.tensor(2.0, device=dev)
    ResidualScaleFn.apply(x, y, gamma).sum().backward()
    assert torch.allclose(y.grad, torch.full_like(y, 2.0))
    assert torch.equal(x.grad, torch.ones_like(x))


def test_block_uses_the_fused_residuals(dev):
    torch.manual_seed(0)
    blk = fe.EquivariantTransformerBlock(fe.Repr([0, 1, 2], 64), fe.Repr([0, 1, 2], 64), num_heads=8).to(dev)
    N, k = 200, 8
    gen = torch.Generator().manual_seed(2)
    coords = torch.randn(N, 3, generator=gen) * 4
    d = torch.cdist(coords, coords)
    d.fill_diagonal_(float("inf"))
    src = d.topk(k, largest=False).indices.reshape(-1)
    dst = torch.arange(N).repeat_interleave(k)
    vec = (coords[src] - coords[dst]).to(dev)
    P, Q = fe.WignerDBasis([fe.Repr([0, 1, 2], 1), fe.Repr([0, 1, 2], 1)]).to(dev)(vec)
    x = torch.randn(N, 64, 9, generator=gen).to(dev).requires_grad_(True)
    graph = fe.Graph(src.to(dev), dst.to(dev), N)
    NAT.profile_summary()
    NAT.profile_enable(True)
    out = blk(P, Q, x, vec.norm(dim=-1), graph)
    out.square().sum().backward()
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert launched.get("k_scale_add", (0,))[0] == 2, launched
    assert blk.layer_scale_attn.gamma.grad is not None and blk.layer_scale_mlp.gamma.grad is not None
