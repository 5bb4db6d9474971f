"""float64 modules (``.double()``): EquivariantEdgewiseLinear and WignerDBasis.

The reference runs its layer in float64 through the block-diagonal op's float64
dispatch (block_diagonal.cu:1332) and its bases through a float64 matrix_exp
(tests/test_edge_cases.py:254-270).  Here the layer's float64 route is the
reference's own composition (bmm, the float64 block-diagonal kernels, bmm) and
the bases come from the float64 forms of the closed-form kernels.  Both are
checked against the float64 oracle: the layer on the same bases at 1e-10
relative (measured ~1e-15); the bases and their direction gradients at 1e-6.
The closed form uses the exact algebra of the generators ([G0, G1] = G2, with
V = exp(pi/2 G1) formed from the float32-rounded G1), while the reference's
float64 matrix_exp exponentiates the float32-rounded generators themselves:
the two differ by ~3e-7, the size of that rounding (measured 2.9e-7).
"""
import pytest
import torch

import flash_eq as fe
from helpers import rel_err
from oracle import layer as OL
from oracle import wigner as OW

pytestmark = pytest.mark.gpu


def test_fp64_layer(dev):
    """The reference's own case (tests/test_edge_cases.py:254-270)."""
    in_repr = fe.Repr(lvals=[0, 1], mult=2)
    out_repr = fe.Repr(lvals=[0, 1], mult=2)
    layer = fe.EquivariantEdgewiseLinear(in_repr, out_repr).to(dev).double()
    basis = fe.WignerDBasis([in_repr, out_repr]).to(dev).double()
    num_edges = 20
    edge_features = torch.randn(num_edges, 2, 4, device=dev, dtype=torch.float64)
    directions = torch.randn(num_edges, 3, device=dev, dtype=torch.float64)
    distances = torch.rand(num_edges, device=dev, dtype=torch.float64) * 5.0
    P, Q = basis(directions)
    output = layer(P, Q, edge_features, distances)
    assert P.dtype == torch.float64 and Q.dtype == torch.float64
    assert output.dtype == torch.float64
    assert torch.isfinite(output).all()


@pytest.mark.parametrize("lin,lout,cin,cout,E,log", [([0, 1], [0, 1, 2], 4, 6, 200, False),
                                                     ([0, 1, 2], [0, 1, 2], 8, 8, 333, True),
                                                     ([1, 2], [0, 2], 3, 5, 17, False)])
def test_fp64_layer_matches_oracle(dev, lin, lout, cin, cout, E, log):
    torch.manual_seed(E)
    rin, rout = fe.Repr(lin, cin), fe.Repr(lout, cout)
    kw = dict(log_bins=True, min_dist=0.5) if log else {}
    layer = fe.EquivariantEdgewiseLinear(rin, rout, num_bins=20, max_dist=8.0, **kw).to(dev).double()
    g = torch.Generator().manual_seed(E + 1)
    x = torch.randn(E, cin, rin.dim(), generator=g, dtype=torch.float64)
    d = torch.randn(E, 3, generator=g, dtype=torch.float64)
    r = torch.rand(E, generator=g, dtype=torch.float64) * 9.5 + 0.05
    P, Q = OW.basis(lin, d), OW.basis(lout, d)
    xg, rg = x.to(dev).requires_grad_(True), r.to(dev).requires_grad_(True)
    Pg, Qg = P.to(dev).requires_grad_(True), Q.to(dev).requires_grad_(True)
    y = layer(Pg, Qg, xg, rg)
    gy = torch.randn(y.shape, generator=g, dtype=torch.float64)
    y.backward(gy.to(dev))
    params, cfg = OL.module_cfg(layer)
    xd, rd = x.clone().requires_grad_(True), r.clone().requires_grad_(True)
    Pd, Qd = P.clone().requires_grad_(True), Q.clone().requires_grad_(True)
    yref = OL.edgewise_linear(xd, Pd, Qd, rd, params, cfg)
    yref.backward(gy)
    assert y.dtype == torch.float64
    errs = {"y": rel_err(y, yref), "gx": rel_err(xg.grad, xd.grad), "gP": rel_err(Pg.grad, Pd.grad),
            "gQ": rel_err(Qg.grad, Qd.grad), "gr": rel_err(rg.grad, rd.grad)}
    for name, p in layer.radial_weights.named_parameters():
        errs[name] = rel_err(p.grad, params[name].grad)
    print({k: f"{v:.1e}" for k, v in errs.items()})
    assert max(errs.values()) < 1e-10, errs


@pytest.mark.parametrize("lvals", [[0, 1, 2], [0, 1], list(range(7)), [2, 0, 1, 1]])
def test_fp64_basis_and_gradient(dev, lvals):
    E = 301
    g = torch.Generator().manual_seed(len(lvals))
    v = torch.randn(E, 3, generator=g, dtype=torch.float64) * 2.0
    v[:3] = torch.tensor([[0.0, 0.0, 1.5], [0.0, 0.0, -0.7], [0.0, 0.0, 0.0]], dtype=torch.float64)
    vd = v.to(dev).requires_grad_(True)
    (M,) = fe.WignerDBasis([fe.Repr(lvals, 2)]).to(dev).double()(vd)
    assert M.dtype == torch.float64
    W = torch.randn(M.shape, generator=g, dtype=torch.float64)
    (M * W.to(dev)).sum().backward()
    vo = v.clone().requires_grad_(True)
    Mo = OW.basis(lvals, vo)
    (Mo * W).sum().backward()
    em = rel_err(M, Mo)
    # the poles (rows 0-2) carry gradients of order 1/eps: compared relative to
    # their own size, the other rows relative to the largest of theirs
    eg = rel_err(vd.grad[3:], vo.grad[3:])
    ep = ((vd.grad[:3].cpu() - vo.grad[:3]).abs() / vo.grad[:3].abs().clamp(min=1.0)).max().item()
    print(f"lvals {lvals}: basis {em:.1e}, direction gradient {eg:.1e}, poles {ep:.1e}")
    assert torch.isfinite(vd.grad).all()
    assert em < 1e-6 and eg < 1e-6 and ep < 1e-6
