"""The transformer block's residual connection with LayerScale in one pass
(feq_scale_add / feq_scale_add_bwd, ops.ResidualScaleFn).

The reference writes it as x + drop_path(layer_scale(y)) (transformer.py:245,
:252; LayerScale :23-38) and autograd forms grad_x = g, grad_y = gamma g and
grad_gamma = sum g y.  Checked against those float64 formulas: out, grad_x and
grad_y at float32 rounding (1e-6 relative), grad_gamma at 1e-6 relative (its
products and sum in float64), ragged lengths (vectorised body and scalar
tail), gamma without gradient, the MLP's component-major branch
(feq_scale_add_cm, against the same formulas), the separable norm's
component-major output (bit for bit the node-major kernels' values), and the
block's launch log (the fused kernels, and no transposes: the attention
reads the QK projection's component-major table).
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
    # the attention residual in one pass; the MLP's component-major branch
    # joins through the transposing sum, and the MLP runs without transposes
    assert launched.get("k_scale_add", (0,))[0] == 1, launched
    assert launched.get("k_scale_add_cm", (0,))[0] == 1, launched
    assert launched.get("k_scale_add_cm_bwd", (0,))[0] == 1, launched
    ntr = sum(v[0] for k, v in launched.items() if k.startswith("k_transpose"))
    assert ntr == 0, launched      # the attention reads the projection's component-major table
    assert blk.layer_scale_attn.gamma.grad is not None and blk.layer_scale_mlp.gamma.grad is not None


@pytest.mark.parametrize("N,mult", [(1001, 64), (333, 6)])
def test_component_major_branch_matches_float64(dev, N, mult):
    """x (N, mult, dim) + gamma y with y component-major (dim, N, mult); 64
    channels move in 16-byte pieces, 6 in 4-byte ones."""
    dim = 9
    g = torch.Generator().manual_seed(5)
    x, go = torch.randn(N, mult, dim, generator=g), torch.randn(N, mult, dim, generator=g)
    y = torch.randn(dim, N, mult, generator=g)
    gamma = torch.tensor(-0.61)
    xd, yd = x.to(dev).requires_grad_(True), y.to(dev).requires_grad_(True)
    gd = gamma.to(dev).requires_grad_(True)
    from flash_eq.ops import ResidualScaleCmFn
    out = ResidualScaleCmFn.apply(xd, yd, gd)
    out.backward(go.to(dev))
    yt = y.double().permute(1, 2, 0)
    assert rel_err(out, x.double() + gamma.double() * yt) < 1e-6
    assert torch.equal(xd.grad.cpu(), go)
    assert rel_err(yd.grad, (gamma.double() * go.double()).permute(2, 0, 1)) < 1e-6
    gg = (go.double() * yt).sum()
    assert abs(gd.grad.item() - gg.item()) <= 1e-6 * (go.double() * yt).abs().sum().item()


@pytest.mark.parametrize("mult", [64, 6])
@pytest.mark.parametrize("kind", ["separable", "equivariant"])
def test_component_major_norm_output_is_the_transpose(dev, kind, mult):
    """The separable and the equivariant layer norm with their output (and
    gradient) component-major: the node-major kernels' values, bit for bit
    (16-byte row accesses at 64 channels, 4-byte ones at 6)."""
    torch.manual_seed(1)
    cls = fe.SeparableEquivariantLayerNorm if kind == "separable" else fe.EquivariantLayerNorm
    norm = cls(fe.Repr([0, 1, 2], mult)).to(dev)
    with torch.no_grad():
        for p in norm.parameters():
            p.normal_()
    x = torch.randn(777, mult, 9, device=dev)
    gy = torch.randn(777, mult, 9, device=dev)
    x1 = x.clone().requires_grad_(True)
    y1 = norm(x1)
    y1.backward(gy)
    g1 = [p.grad.clone() for p in norm.parameters()]
    for p in norm.parameters():
        p.grad = None
    x2 = x.clone().requires_grad_(True)
    assert norm.cm_ok(x2)
    y2 = norm.forward_cm(x2)
    y2.backward(gy.permute(2, 0, 1).contiguous())
    assert torch.equal(y2, y1.detach().permute(2, 0, 1))
    assert torch.equal(x2.grad, x1.grad)
    for a, b in zip(g1, norm.parameters()):
        assert torch.equal(a, b.grad)


@pytest.mark.parametrize("cm", [False, True])
@pytest.mark.parametrize("lvals,mult", [([0, 1, 2], 64), ([0, 1, 2], 6), ([0, 0, 1, 2], 8), ([0, 1, 2], 128)])
@pytest.mark.parametrize("kind", ["separable", "equivariant"])
def test_norm_pair_adds_the_second_branch_gradient(dev, kind, lvals, mult, cm):
    """forward_pair returns (norm(x), x); the second output's gradient is added
    inside the norm's backward kernel (feq_*norm_bwd_add): x.grad is bitwise
    the norm's input gradient plus that gradient, as autograd's separate sum
    gives it; the parameter gradients are unchanged.  Layouts: 16-byte rows
    (64), 4-byte rows (6), two scalar irreps (the separable norm's general
    instance), two channels per lane (128)."""
    torch.manual_seed(2)
    cls = fe.SeparableEquivariantLayerNorm if kind == "separable" else fe.EquivariantLayerNorm
    rp = fe.Repr(lvals, mult)
    norm = cls(rp).to(dev)
    with torch.no_grad():
        for p in norm.parameters():
            p.normal_()
    dim = rp.dim()
    x = torch.randn(501, mult, dim, device=dev)
    gy = torch.randn(501, mult, dim, device=dev)
    ga = torch.randn(501, mult, dim, device=dev)
    gyl = gy.permute(2, 0, 1).contiguous() if cm else gy
    x1 = x.clone().requires_grad_(True)
    y1 = norm.forward_cm(x1) if cm else norm(x1)
    (y1 * gyl).sum().backward()
    g1 = [p.grad.clone() for p in norm.parameters()]
    ref = x1.grad + ga
    for p in norm.parameters():
        p.grad = None
    x2 = x.clone().requires_grad_(True)
    assert norm.cm_ok(x2)
    y2, a2 = norm.forward_pair(x2, cm)
    assert torch.equal(a2, x2) and torch.equal(y2, y1)
    NAT.profile_summary()
    NAT.profile_enable(True)
    ((y2 * gyl).sum() + (a2 * ga).sum()).backward()
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert launched.get("k_sepnorm_bwd" if kind == "separable" else "k_eqnorm_bwd", (0,))[0] == 1, launched
    assert torch.equal(x2.grad, ref)
    for a, b in zip(g1, norm.parameters()):
        assert torch.equal(a, b.grad)
    # only the second branch used: its gradient passes through
    x3 = x.clone().requires_grad_(True)
    _, a3 = norm.forward_pair(x3, cm)
    (a3 * ga).sum().backward()
    assert torch.equal(x3.grad, ga)
