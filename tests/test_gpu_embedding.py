"""GPU parity of small layouts run zero-embedded in larger split-fp16 layouts
(ops._Embedding, the smallest of [0,1]x64 -> [0,1,2]x64 and [0,1,2]x64 ->
[0,1,2]x64 that holds them): BASELINE config 1's layer ([0,1]x32 -> [0,1,2]x64,
also the first layer of config 4, channels padded only) and a layout with odd
channel counts; and config 4's last layer ([0,1,2]x64 -> [0]x8), which has
kernels of its own (edgewise_scalar.hip).  Against the float64 oracle at the
fp32 bar (1e-5), outputs and every gradient, in the plain and the
message-passing form.  The launch log must show the fast kernels, not the
generic ones."""
import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from helpers import rel_err
from oracle import layer as OL
from oracle import wigner as OW

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.mark.parametrize("lin,cin,lout,cout,kernel", [
    ([0, 1], 32, [0, 1, 2], 64, "k_ews_bwd_x"),
    ([0, 1, 2], 64, [0], 8, "k_ew0_bwd"),
    ([0], 13, [0, 1], 40, "k_ews_bwd_x"),
])
@pytest.mark.parametrize("message_passing", [False, True])
def test_embedded_layout_matches_oracle(dev, lin, cin, lout, cout, kernel, message_passing):
    torch.manual_seed(3)
    rin, rout = fe.Repr(lin, cin), fe.Repr(lout, cout)
    layer = fe.EquivariantEdgewiseLinear(rin, rout, num_bins=100, max_dist=10.0).to(dev)
    g = torch.Generator().manual_seed(len(lin) * 10 + cout)
    Nn, E = 300, 5000
    din = sum(2 * l + 1 for l in lin)
    x = torch.randn(Nn, cin, din, generator=g)
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn, (E,), generator=g)
    d = torch.randn(E, 3, generator=g)
    r = torch.rand(E, generator=g) * 9.5 + 0.05
    P, Q = OW.basis(lin, d).float(), OW.basis(lout, d).float()
    xg = x.to(dev).requires_grad_(True)
    rg = r.to(dev).requires_grad_(True)
    graph = fe.Graph(src.to(dev), dst.to(dev), Nn)
    NAT.profile_summary()
    NAT.profile_enable(True)
    if message_passing:
        y = layer(P.to(dev), Q.to(dev), xg, rg, graph=graph)
    else:
        y = layer(P.to(dev), Q.to(dev), graph.gather_src(xg), rg)
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev))
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert kernel in launched and "k_ew_bwd" not in launched, launched
    params, cfg = OL.module_cfg(layer)
    xd = x.double().requires_grad_(True)
    rd = r.double().requires_grad_(True)
    yref = OL.edgewise_linear(xd[src], P.double(), Q.double(), rd, params, cfg)
    yref.backward(gy.double())
    assert y.shape == (E, cout, sum(2 * l + 1 for l in lout))
    assert rel_err(y, yref) < TOL
    assert rel_err(xg.grad, xd.grad) < TOL
    assert rel_err(rg.grad, rd.grad) < 1e-4
    for name, p in layer.radial_weights.named_parameters():
        assert rel_err(p.grad, params[name].grad) < TOL, name


def test_embedding_targets_have_split_kernels(dev):
    """Every embedding target is a layout the split kernels serve, and the c1
    layout takes the smallest one ([0,1]x64 -> [0,1,2]x64: channels padded,
    no slots added)."""
    from flash_eq import ops
    for tin, tout in ops._EMB_TARGETS:
        L = NAT.make_layout(list(range(tin + 1)), list(range(tout + 1)), 64, 64)
        B = NAT.make_binning(0.0, 0.1, 100, False, 1.0)
        assert ops.edgewise_src_supported(L, B, 4), (tin, tout)
    emb = ops.embedding_for([0, 1], [0, 1, 2], 32, 64, 4, dev)
    assert emb.Din == 4 and emb.Dout == 9 and emb.pcols is None and emb.qcols is None
