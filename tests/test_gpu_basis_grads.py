"""Gradients for the bases P and Q on the split kernels (feq_edgewise_fwd_ym / _bwd_pq).

The reference forms grad_P and grad_Q by torch.bmm autograd around its
block-diagonal op (flash_eq/layers/linear.py:135, :160).  Here the split
forward keeps m (the rows before the Q rotation) and the split input-gradient
kernel forms grad_Q = gy^T m from its producers' rows and grad_P = x^T dL/df
from the tile's accumulators, so a layer whose bases require grad (coordinate
gradients through WignerDBasis) stays on the split kernels.  Checked against
the float64 oracle at 1e-5 relative for every gradient, in the edge-rows form,
the message-passing form (gather and per-node input-gradient sums inside the
kernels), the pooled form of the attention's V projection, the zero-embedded
small layouts, the scalar-output layouts on their own wave-per-edge kernels,
with only one of P and Q requiring grad, and for ragged tiles; the launch log
shows the fast kernels and no shape-generic ones.
"""
import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from helpers import rel_err
from oracle import layer as OL
from oracle import wigner as OW

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _check(dev, lin, lout, cin, cout, E, seed, graph_nodes=None, grad_p=True, grad_q=True, rmax=9.5,
           kernels=("k_ews_fwd", "k_ews_bwd_x")):
    torch.manual_seed(seed)
    layer = fe.EquivariantEdgewiseLinear(fe.Repr(lin, cin), fe.Repr(lout, cout), num_bins=50).to(dev)
    g = torch.Generator().manual_seed(seed + 1)
    din = sum(2 * l + 1 for l in lin)
    d = torch.randn(E, 3, generator=g)
    r = torch.rand(E, generator=g) * rmax + 0.05
    P, Q = OW.basis(lin, d).float(), OW.basis(lout, d).float()
    if graph_nodes:
        xn = torch.randn(graph_nodes, cin, din, generator=g)
        src = torch.randint(0, graph_nodes, (E,), generator=g)
        dst = torch.randint(0, graph_nodes, (E,), generator=g)
        x = xn[src]
    else:
        x = torch.randn(E, cin, din, generator=g)
    Pg = P.to(dev).requires_grad_(grad_p)
    Qg = Q.to(dev).requires_grad_(grad_q)
    rg = r.to(dev).requires_grad_(True)
    NAT.profile_summary()
    NAT.profile_enable(True)
    if graph_nodes:
        xg = xn.to(dev).requires_grad_(True)
        graph = fe.Graph(src.to(dev), dst.to(dev), graph_nodes)
        y = layer(Pg, Qg, xg, rg, graph=graph)
    else:
        xg = x.to(dev).requires_grad_(True)
        y = layer(Pg, Qg, xg, rg)
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev))
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert all(k in launched for k in kernels), launched
    assert "k_ew_bwd" not in launched and "k_ew_fwd" not in launched, launched

    params, cfg = OL.module_cfg(layer)
    xd, rd = x.double().requires_grad_(True), r.double().requires_grad_(True)
    Pd, Qd = P.double().requires_grad_(grad_p), Q.double().requires_grad_(grad_q)
    yref = OL.edgewise_linear(xd, Pd, Qd, rd, params, cfg)
    yref.backward(gy.double())
    gx_ref = xd.grad
    if graph_nodes:
        gx_ref = torch.zeros(graph_nodes, cin, din, dtype=torch.float64).index_add_(0, src, xd.grad)
    errs = {"y": rel_err(y, yref), "gx": rel_err(xg.grad, gx_ref), "gr": rel_err(rg.grad, rd.grad)}
    if grad_p:
        errs["gP"] = rel_err(Pg.grad, Pd.grad)
    else:
        assert Pg.grad is None
    if grad_q:
        errs["gQ"] = rel_err(Qg.grad, Qd.grad)
    else:
        assert Qg.grad is None
    for name, p in layer.radial_weights.named_parameters():
        errs[name] = rel_err(p.grad, params[name].grad)
    print({k: f"{v:.1e}" for k, v in errs.items()})
    bars = {"gr": 1e-4}
    for k, v in errs.items():
        assert v < bars.get(k, TOL), (k, errs)


@pytest.mark.parametrize("lin,cin,E", [([0, 1, 2], 64, 1003), ([0, 1], 64, 777)])
def test_edge_rows(dev, lin, cin, E):
    _check(dev, lin, [0, 1, 2], cin, 64, E, seed=E)


@pytest.mark.parametrize("grad_p,grad_q", [(True, False), (False, True)])
def test_one_basis_requires_grad(dev, grad_p, grad_q):
    _check(dev, [0, 1, 2], [0, 1, 2], 64, 64, 500, seed=7, grad_p=grad_p, grad_q=grad_q)


def test_message_passing_form(dev):
    """Node table read at src inside the kernels, input gradient summed per
    source node over the CSR by source; edges past a tile and repeated sources."""
    _check(dev, [0, 1, 2], [0, 1, 2], 64, 64, 1201, seed=11, graph_nodes=150)


def test_embedded_layout(dev):
    """[0,1]x32 -> [0,1,2]x64 above the embedding threshold runs zero-embedded
    in the [0,1,2]x64 kernels; the embedded bases' gradients flow back through
    the embedding."""
    _check(dev, [0, 1], [0, 1, 2], 32, 64, 4500, seed=13, graph_nodes=900)


@pytest.mark.parametrize("graph_nodes,grad_p,grad_q", [(700, True, True), (None, True, True),
                                                       (700, True, False), (None, False, True)])
def test_scalar_output_layout(dev, graph_nodes, grad_p, grad_q):
    """[0,1,2]x64 -> [0]x8 (the last layer of config 4's model) on its own
    scalar-output kernels: the forward keeps m = y / Q, the wave-per-edge
    backward forms grad_Q = gy . m and grad_P in the m = 0 columns (zero in
    the others, which y does not read)."""
    _check(dev, [0, 1, 2], [0], 64, 8, 4200, seed=17, graph_nodes=graph_nodes, grad_p=grad_p,
           grad_q=grad_q, kernels=("k_ew0_fwd", "k_ew0_bwd"))


def test_scalar_output_one_channel(dev):
    """[0,1,2]x64 -> [0]x1, ragged tiles."""
    _check(dev, [0, 1, 2], [0], 64, 1, 1001, seed=19, graph_nodes=300,
           kernels=("k_ew0_fwd", "k_ew0_bwd"))


@pytest.mark.parametrize("lin,cin", [([0, 1, 2], 64), ([0, 1], 32)])
def test_pooled_form(dev, lin, cin):
    """The V projection fused with the head weighting and the sum by
    destination (feq_edgewise_fwd_src_pool_ym / _bwd_src_pool_pq), bases with
    gradients: out[n] = sum over e into n of attn[e, head(c)] layer(x[src])[e]
    against the float64 oracle, with the gradients of x, P, Q, attn, r and the
    radial network; edges without a destination (dst outside the node range)
    add nothing and get zero basis gradients.  [0,1]x32 runs zero-embedded."""
    torch.manual_seed(21)
    heads, Nn, E = 8, 500, 4700
    lout = [0, 1, 2]
    layer = fe.EquivariantEdgewiseLinear(fe.Repr(lin, cin), fe.Repr(lout, 64), num_bins=40).to(dev)
    g = torch.Generator().manual_seed(22)
    din = sum(2 * l + 1 for l in lin)
    xn = torch.randn(Nn, cin, din, generator=g)
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn, (E,), generator=g)
    d = torch.randn(E, 3, generator=g)
    r = torch.rand(E, generator=g) * 9.5 + 0.05
    attn = torch.rand(E, heads, generator=g)
    P, Q = OW.basis(lin, d).float(), OW.basis(lout, d).float()
    graph = fe.Graph(src.to(dev), dst.to(dev), Nn)
    xg, rg, ag = (t.to(dev).requires_grad_(True) for t in (xn, r, attn))
    Pg, Qg = P.to(dev).requires_grad_(True), Q.to(dev).requires_grad_(True)
    NAT.profile_summary()
    NAT.profile_enable(True)
    out = layer.attention_pool(Pg, Qg, xg, rg, graph, ag, heads)
    assert out is not None
    w = torch.randn(out.shape, generator=g)
    (out * w.to(dev)).sum().backward()
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert "k_pool_order" in launched and "k_ews_bwd_x" in launched, launched
    assert "k_pool_fwd" not in launched and "k_ew_bwd" not in launched, launched

    params, cfg = OL.module_cfg(layer)
    xd, rd, ad = xn.double().requires_grad_(True), r.double().requires_grad_(True), \
        attn.double().requires_grad_(True)
    Pd, Qd = P.double().requires_grad_(True), Q.double().requires_grad_(True)
    v = OL.edgewise_linear(xd[src], Pd, Qd, rd, params, cfg)              # (E, 64, 9)
    head_of = torch.arange(64) // (64 // heads)
    ref = torch.zeros(Nn, 64, 9, dtype=torch.float64).index_add_(0, dst, v * ad[:, head_of, None])
    (ref * w.double()).sum().backward()
    errs = {"out": rel_err(out, ref), "gx": rel_err(xg.grad, xd.grad), "gP": rel_err(Pg.grad, Pd.grad),
            "gQ": rel_err(Qg.grad, Qd.grad), "gattn": rel_err(ag.grad, ad.grad), "gr": rel_err(rg.grad, rd.grad)}
    for name, p in layer.radial_weights.named_parameters():
        errs[name] = rel_err(p.grad, params[name].grad)
    print({k: f"{v:.1e}" for k, v in errs.items()})
    bars = {"gr": 1e-4}
    for k, v in errs.items():
        assert v < bars.get(k, TOL), (k, errs)


def test_pq_entry_points_reject_unsupported(dev):
    """Layouts without split kernels say so (the layer then uses the
    shape-generic pair, which forms the gradients itself)."""
    layer = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1], 8), fe.Repr([0, 1], 8)).to(dev)
    from flash_eq.ops import edgewise_pq_supported
    assert not edgewise_pq_supported(layer.layout(), layer.binning(), 4)
    big = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1, 2], 64), fe.Repr([0, 1, 2], 64)).to(dev)
    assert edgewise_pq_supported(big.layout(), big.binning(), 4)
