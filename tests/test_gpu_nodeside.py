"""GPU parity of the node-side kernels (csrc/nodeside.hip): the separable
equivariant layer norm, the equivariant layer norm and the norm gating, forward
and every gradient, against the float64 oracle (whose index-form restatements
are pinned to the reference's own vectors in test_node_side_cpu.py).

Layouts cover scalars in the middle, repeated and missing scalars, a single
irrep, one channel (no LayerNorm), and 1, 2 and 4 channels per lane (up to 256
channels, with a partial last lane group).  The library's launch log confirms
that the kernels, not the PyTorch formulation, produced the results.
"""
import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from helpers import rel_err
from oracle import layer as OL

pytestmark = pytest.mark.gpu
TOL = 1e-5
CASES = [([0, 1, 2], 64), ([1, 0, 2], 5), ([0, 0, 1, 2], 7), ([2, 1], 33), ([0], 8),
         ([1, 2, 0, 1], 100), ([0, 1, 2], 128), ([0, 1], 200), ([0, 1, 2], 256), ([0, 1, 2], 1)]


def _randomise(m, g):
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.5 + 1.0)
    return m


def _run(module, x, gy, dev):
    """Forward and backward on the GPU with the launch log on; returns
    (y, grad_x, {param name: grad}, launched kernel names)."""
    m = module.to(dev)
    xg = x.to(dev).requires_grad_(True)
    NAT.profile_summary()
    NAT.profile_enable(True)
    y = m(xg)
    y.backward(gy.to(dev))
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    return y, xg.grad, {n: p.grad for n, p in m.named_parameters()}, launched


def _leaf(t):
    return t.detach().double().cpu().requires_grad_(True)


@pytest.mark.parametrize("lvals,mult", CASES)
def test_separable_norm_matches_oracle(dev, lvals, mult):
    g = torch.Generator().manual_seed(mult + len(lvals))
    rp = fe.Repr(lvals, mult)
    m = _randomise(fe.SeparableEquivariantLayerNorm(rp), g)
    # scalars with a large common offset: the channel statistics are two-pass
    x = torch.randn(37, mult, rp.dim(), generator=g) + 3.0
    gy = torch.randn(x.shape, generator=g)
    ws = _leaf(m.scalar_norm.weight) if m.nscalar else None
    bs = _leaf(m.scalar_norm.bias) if m.nscalar else None
    wh = _leaf(m.higher_norm.weight) if m.nhigher else None
    y, gx, grads, launched = _run(m, x, gy, dev)
    assert "k_sepnorm_fwd" in launched and "k_sepnorm_bwd" in launched, launched
    xd = _leaf(x)
    yref = OL.separable_layer_norm(xd, lvals, ws, bs, wh)
    yref.backward(gy.double())
    assert rel_err(y, yref) < TOL
    assert rel_err(gx, xd.grad) < TOL
    if ws is not None:
        assert rel_err(grads["scalar_norm.weight"], ws.grad) < TOL
        assert rel_err(grads["scalar_norm.bias"], bs.grad) < TOL
    if wh is not None:
        assert rel_err(grads["higher_norm.weight"], wh.grad) < TOL


@pytest.mark.parametrize("lvals,mult", CASES)
def test_equivariant_norm_matches_oracle(dev, lvals, mult):
    g = torch.Generator().manual_seed(100 + mult + len(lvals))
    rp = fe.Repr(lvals, mult)
    m = _randomise(fe.EquivariantLayerNorm(rp), g)
    x = torch.randn(29, mult, rp.dim(), generator=g)
    gy = torch.randn(x.shape, generator=g)
    y, gx, grads, launched = _run(m, x, gy, dev)
    assert "k_eqnorm_fwd" in launched and "k_eqnorm_bwd" in launched, launched
    xd = _leaf(x)
    if m.lnorm is not None:
        w, b = _leaf(m.lnorm.weight), _leaf(m.lnorm.bias)
        yref = OL.equivariant_layer_norm(xd, lvals, w, b)
    else:   # one channel: x / (norm + eps) (norm.py:160-165)
        idx = torch.tensor([k for k, l in enumerate(lvals) for _ in range(2 * l + 1)])
        yref = xd / (OL.rep_norms(xd, lvals, 1e-8) + 1e-8)[..., idx]
    yref.backward(gy.double())
    assert rel_err(y, yref) < TOL
    assert rel_err(gx, xd.grad) < TOL
    if m.lnorm is not None:
        assert rel_err(grads["lnorm.weight"], w.grad) < TOL
        assert rel_err(grads["lnorm.bias"], b.grad) < TOL


@pytest.mark.parametrize("lvals,mult", CASES[:8])
def test_gating_matches_oracle(dev, lvals, mult):
    g = torch.Generator().manual_seed(200 + mult + len(lvals))
    rp = fe.Repr(lvals, mult)
    m = fe.EquivariantGating(rp)
    with torch.no_grad():
        m.linear.weight.copy_(torch.randn(m.linear.weight.shape, generator=g) * 0.2)
        m.linear.bias.copy_(torch.randn(m.linear.bias.shape, generator=g))
    x = torch.randn(300, mult, rp.dim(), generator=g)
    gy = torch.randn(x.shape, generator=g)
    W, b = _leaf(m.linear.weight), _leaf(m.linear.bias)
    y, gx, grads, launched = _run(m, x, gy, dev)
    assert "k_gate_apply" in launched and "k_gate_bwd_x" in launched, launched
    xd = _leaf(x)
    yref = OL.gating(xd, lvals, W, b)
    yref.backward(gy.double())
    assert rel_err(y, yref) < TOL
    assert rel_err(gx, xd.grad) < TOL
    assert rel_err(grads["linear.weight"], W.grad) < TOL
    assert rel_err(grads["linear.bias"], b.grad) < TOL


def test_node_kernels_batched_and_empty(dev):
    """Leading batch dimensions flatten to nodes; zero nodes give zero parameter
    gradients."""
    rp = fe.Repr([0, 1, 2], 16)
    torch.manual_seed(3)
    sln = fe.SeparableEquivariantLayerNorm(rp).to(dev)
    x = torch.randn(3, 5, 16, 9, device=dev)
    y = sln(x)
    y2 = sln(x.reshape(15, 16, 9)).reshape(3, 5, 16, 9)
    assert torch.equal(y, y2)
    for m in (sln, fe.EquivariantLayerNorm(rp).to(dev), fe.EquivariantGating(rp).to(dev)):
        x0 = torch.zeros(0, 16, 9, device=dev, requires_grad=True)
        y0 = m(x0)
        assert y0.shape == (0, 16, 9)
        y0.sum().backward()
        for n, p in m.named_parameters():
            assert p.grad is not None and torch.all(p.grad == 0), n


@pytest.mark.parametrize("lvals,cin,cout", [([0, 1, 2], 64, 128), ([1, 0, 2], 5, 3),
                                            ([0, 0, 1, 2], 7, 9), ([2, 1], 33, 16)])
def test_equivariant_linear_matches_oracle(dev, lvals, cin, cout):
    """EqLinearFn (one GEMM per irrep into a component-major table, bias as the
    GEMM's bias column) against the oracle's per-irrep einsum plus bias."""
    g = torch.Generator().manual_seed(300 + cin + cout)
    lin = fe.EquivariantLinear(fe.Repr(lvals, cin), fe.Repr(lvals, cout), bias=True)
    if lin.bias is not None:
        with torch.no_grad():
            lin.bias.copy_(torch.randn(lin.bias.shape, generator=g))
    x = torch.randn(41, cin, fe.Repr(lvals, cin).dim(), generator=g)
    gy = torch.randn(41, cout, x.shape[-1], generator=g)
    W = _leaf(lin.weight)
    bias = _leaf(lin.bias) if lin.bias is not None else None
    y, gx, grads, _ = _run(lin, x, gy, dev)
    xd = _leaf(x)
    yref = OL.equivariant_linear(xd, W, lvals)
    if bias is not None:
        offs = fe.Repr(lvals, cin).cumdims().tolist()
        locs = [offs[k] for k, l in enumerate(lvals) if l == 0]
        yref = yref.clone()
        yref[..., locs] = yref[..., locs] + bias
    yref.backward(gy.double())
    assert rel_err(y, yref) < TOL
    assert rel_err(gx, xd.grad) < TOL
    assert rel_err(grads["weight"], W.grad) < TOL
    if bias is not None:
        assert rel_err(grads["bias"], bias.grad) < TOL


@pytest.mark.parametrize("lvals,mult,n", [([0, 1, 2], 128, 500), ([1, 2, 0, 1], 100, 333), ([0, 1, 2], 7, 301)])
def test_component_major_gating_equals_node_major(dev, lvals, mult, n):
    """The (dim, N, mult) gating kernels give the node-major kernels' results
    (channel counts a multiple of 4 take the 16-byte form, 7 the 4-byte one)."""
    g = torch.Generator().manual_seed(17)
    rp = fe.Repr(lvals, mult)
    m = fe.EquivariantGating(rp).to(dev)
    x = torch.randn(n, mult, rp.dim(), generator=g).to(dev)
    gy = torch.randn(n, mult, rp.dim(), generator=g).to(dev)
    x1 = x.clone().requires_grad_(True)
    y1 = m(x1)
    y1.backward(gy)
    gw1 = m.linear.weight.grad.clone()
    m.zero_grad()
    x2 = x.permute(2, 0, 1).contiguous().requires_grad_(True)
    y2 = m.forward_cm(x2)
    y2.backward(gy.permute(2, 0, 1).contiguous())
    assert rel_err(y2.permute(1, 2, 0), y1) < 1e-6
    assert rel_err(x2.grad.permute(1, 2, 0), x1.grad) < 1e-6
    assert rel_err(m.linear.weight.grad, gw1) < 1e-6


def test_block_kernels_equal_pytorch_formulation(dev, monkeypatch):
    """A whole transformer block with the node-side kernels (fused norms,
    component-major MLP) against the same block with its node side in the
    PyTorch formulation (pinned to the oracle in test_node_side_cpu.py), both
    float32 on the GPU: output and every gradient."""
    import flash_eq.ops as fops
    from flash_eq.layers import linear as flin

    torch.manual_seed(21)
    rp = fe.Repr([0, 1, 2], 16)
    blk = fe.EquivariantTransformerBlock(rp, rp, num_heads=2, layer_scale_init=0.5).to(dev)
    g = torch.Generator().manual_seed(22)
    Nn, E = 60, 600
    src = torch.randint(0, Nn, (E,), generator=g).to(dev)
    dst = torch.randint(0, Nn, (E,), generator=g).to(dev)
    vec = (torch.randn(E, 3, generator=g) * 2).to(dev)
    x = torch.randn(Nn, 16, 9, generator=g).to(dev)
    gy = torch.randn(Nn, 16, 9, generator=g).to(dev)
    P = fe.WignerDBasis([rp]).to(dev)(vec)[0]
    graph = fe.Graph(src, dst, Nn)

    def run():
        blk.zero_grad()
        xg = x.clone().requires_grad_(True)
        y = blk(P, P, xg, vec.norm(dim=-1), graph)
        y.backward(gy)
        return y.detach(), xg.grad, {n: p.grad.clone() for n, p in blk.named_parameters()
                                     if p.grad is not None}

    NAT.profile_summary()
    NAT.profile_enable(True)
    y1, gx1, g1 = run()
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert "k_sepnorm_bwd" in launched and "k_gate_bwd_x" in launched, launched
    monkeypatch.setattr(fops, "node_kernels_ok", lambda *a, **k: False)
    monkeypatch.setattr(flin.EquivariantLinear, "fused_ok", lambda self, f: False)
    y2, gx2, g2 = run()
    assert rel_err(y1, y2) < TOL
    assert rel_err(gx1, gx2) < TOL
    assert set(g1) == set(g2)
    for n in g1:
        assert rel_err(g1[n], g2[n]) < TOL, n
