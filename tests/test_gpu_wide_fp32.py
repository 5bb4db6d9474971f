"""float32 layers wider than the fused kernels' LDS.

The reference accepts any layout with lmax <= 16 (block_diagonal.cu:1298).
The fused float32 kernels keep an edge's rows and the workgroup's
channel-pattern gradient in LDS, which lvals 0..6 at 64 channels (189 KB)
or 0..4 at 128 in and 64 out channels (220 KB) exceed:
``feq_edgewise_fused_supported`` says so and the layer takes the reference's
own composition (linear.py:131-160): bmm, the block-diagonal kernels of
blockdiag.hip on the formed radial table, bmm.  Checked against the float64
oracle on the module's parameters at 1e-5 relative, with every gradient
(features, both bases, distances, radial network), and the launch log shows
the block-diagonal kernels and no fused ones.
"""
import ctypes

import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from helpers import rel_err
from oracle import layer as OL
from oracle import wigner as OW

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("lin,lout,cin,cout,E", [(list(range(7)), list(range(7)), 64, 64, 150),
                                                 ([0, 1, 2, 3, 4], [0, 1, 2, 3, 4], 128, 64, 97)])
def test_wide_layer_takes_the_composition(dev, lin, lout, cin, cout, E):
    torch.manual_seed(E)
    rin, rout = fe.Repr(lin, cin), fe.Repr(lout, cout)
    layer = fe.EquivariantEdgewiseLinear(rin, rout, num_bins=12, max_dist=8.0).to(dev)
    assert not NAT.lib().feq_edgewise_fused_supported(ctypes.byref(layer.layout()),
                                                      ctypes.byref(layer.binning()), 4)
    g = torch.Generator().manual_seed(E + 1)
    x = torch.randn(E, cin, rin.dim(), generator=g)
    d = torch.randn(E, 3, generator=g)
    r = torch.rand(E, generator=g) * 8.5 + 0.05
    P, Q = OW.basis(lin, d.double()).float(), OW.basis(lout, d.double()).float()
    xg, rg = x.to(dev).requires_grad_(True), r.to(dev).requires_grad_(True)
    Pg, Qg = P.to(dev).requires_grad_(True), Q.to(dev).requires_grad_(True)
    NAT.profile_summary()
    NAT.profile_enable(True)
    y = layer(Pg, Qg, xg, rg)
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev))
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert any(k.startswith("k_bd_") for k in launched), launched
    assert not any(k.startswith(("k_ew_", "k_ews_")) for k in launched), launched
    assert y.dtype == torch.float32

    params, cfg = OL.module_cfg(layer)
    xd, rd = x.double().requires_grad_(True), r.double().requires_grad_(True)
    Pd, Qd = P.double().requires_grad_(True), Q.double().requires_grad_(True)
    yref = OL.edgewise_linear(xd, Pd, Qd, rd, params, cfg)
    yref.backward(gy.double())
    errs = {"y": rel_err(y, yref), "gx": rel_err(xg.grad, xd.grad), "gP": rel_err(Pg.grad, Pd.grad),
            "gQ": rel_err(Qg.grad, Qd.grad), "gr": rel_err(rg.grad, rd.grad)}
    for name, p in layer.radial_weights.named_parameters():
        errs[name] = rel_err(p.grad, params[name].grad)
    print({k: f"{v:.1e}" for k, v in errs.items()})
    assert max(errs.values()) < 1e-5, errs


def test_wide_layer_message_passing_form(dev):
    """With a graph the rows are gathered first (index_select) and the input
    gradient is summed per source node by its autograd."""
    torch.manual_seed(3)
    rp = fe.Repr(list(range(7)), 64)
    layer = fe.EquivariantEdgewiseLinear(rp, rp, num_bins=10).to(dev)
    Nn, E = 40, 120
    g = torch.Generator().manual_seed(4)
    x = torch.randn(Nn, 64, 49, generator=g)
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn, (E,), generator=g)
    d = torch.randn(E, 3, generator=g)
    r = torch.rand(E, generator=g) * 9.0 + 0.1
    P = OW.basis(list(range(7)), d.double()).float().to(dev)
    graph = fe.Graph(src.to(dev), dst.to(dev), Nn)
    xg = x.to(dev).requires_grad_(True)
    y = layer(P, P, xg, r.to(dev), graph=graph)
    y.square().sum().backward()
    xe = x[src].to(dev).requires_grad_(True)
    y2 = layer(P, P, xe, r.to(dev))
    y2.square().sum().backward()
    ref_gx = torch.zeros_like(xg).index_add_(0, src.to(dev), xe.grad)
    assert torch.equal(y, y2)
    assert rel_err(xg.grad, ref_gx) < 1e-6
