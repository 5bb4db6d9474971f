"""EquivariantLinear on the split-fp16 matrix-core kernels (feq_eqlinear_fwd / _bwd_x).

The reference's EquivariantLinear (flash_eq/layers/linear.py:242-268) mixes the
channels of every degree with its own weight and adds the bias to the scalar
degrees; autograd forms its gradients.  Here the forward, the input
gradient and the weight and bias gradients are one launch each over every
component (plus the fixed-order sum of the weight gradient's partials), with
the products on the fp16 matrix cores (hi + lo split operands, three
products, float32 sums).
Checked against the float64 oracle (oracle/model.py: linear) at 1e-5 relative
for the output and every gradient, at the layouts of the transformer block
(the fused QK projection, the MLP's up and down maps, config 4's first block)
and others, ragged row counts, rows whose magnitudes span 1e-30..1e30 (each
row is scaled on its own: every row within 1e-5 of its own size), and the
launch log (k_eql_mm per map and direction, k_eql_wgrad per map).
"""
import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from helpers import rel_err
from oracle import model as OM

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _run(dev, lvals, cin, cout, rows, seed, bias=True, row_scales=None):
    torch.manual_seed(seed)
    lin = fe.EquivariantLinear(fe.Repr(lvals, cin), fe.Repr(lvals, cout), bias=bias).to(dev)
    if lin.bias is not None:
        with torch.no_grad():
            lin.bias.normal_()
    g = torch.Generator().manual_seed(seed + 1)
    dim = sum(2 * l + 1 for l in lvals)
    x = torch.randn(rows, cin, dim, generator=g)
    if row_scales is not None:
        x = x * row_scales[:, None, None]
    xg = x.to(dev).requires_grad_(True)
    NAT.profile_summary()
    NAT.profile_enable(True)
    y = lin(xg)
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev))
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    xd = x.double().requires_grad_(True)
    wd = lin.weight.detach().double().cpu().requires_grad_(True)
    bd = lin.bias.detach().double().cpu().requires_grad_(True) if lin.bias is not None else None
    yref = OM.linear(xd, wd, bd, lvals)
    yref.backward(gy.double())
    return lin, xg, y, xd, wd, bd, yref, launched


@pytest.mark.parametrize("lvals,cin,cout,rows", [
    ([0, 1, 2], 64, 128, 2003),     # the attention's fused QK projection
    ([0, 1, 2], 128, 64, 1501),     # the MLP's down map
    ([0, 1], 32, 64, 777),          # config 4's first block, QK projection
    ([0, 1, 2, 3], 32, 32, 300),
    ([0, 0, 1, 2], 64, 64, 17),     # two scalar irreps: two bias columns
    ([1, 2], 128, 128, 1000),       # no scalar irrep: no bias
])
def test_matches_float64_oracle(dev, lvals, cin, cout, rows):
    lin, xg, y, xd, wd, bd, yref, launched = _run(dev, lvals, cin, cout, rows, seed=rows)
    assert launched.get("k_eql_mm", (0,))[0] == 2, launched
    assert launched.get("k_eql_wgrad", (0,))[0] == 1, launched
    errs = {"y": rel_err(y, yref), "gx": rel_err(xg.grad, xd.grad), "gw": rel_err(lin.weight.grad, wd.grad)}
    if bd is not None:
        errs["gb"] = rel_err(lin.bias.grad, bd.grad)
    print({k: f"{v:.1e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v < TOL, (k, errs)


def test_rows_of_any_magnitude(dev):
    """Each row's operands are scaled by their own power of two: rows from
    1e-30 to 1e30 keep float32 relative accuracy, row by row."""
    rows = 640
    g = torch.Generator().manual_seed(3)
    sc = torch.pow(10.0, torch.empty(rows).uniform_(-30, 30, generator=g))
    lin, xg, y, xd, wd, bd, yref, _ = _run(dev, [0, 1, 2], 64, 128, rows, seed=5, bias=False,
                                           row_scales=sc)
    yd = y.detach().double().cpu()
    per_row = ((yd - yref).abs().amax(dim=(1, 2)) / yref.abs().amax(dim=(1, 2))).max().item()
    print(f"worst per-row relative error {per_row:.1e}")
    assert per_row < TOL
    assert torch.isfinite(xg.grad).all()


def test_zero_rows_and_fallback_agree(dev, monkeypatch):
    """No rows: empty outputs.  The library path (FEQ_EQLINEAR=lib) and the
    kernels agree to float32 rounding."""
    lin = fe.EquivariantLinear(fe.Repr([0, 1, 2], 64), fe.Repr([0, 1, 2], 128)).to(dev)
    x0 = torch.zeros(0, 64, 9, device=dev, requires_grad=True)
    y0 = lin(x0)
    y0.sum().backward()
    assert y0.shape == (0, 128, 9) and x0.grad.shape == (0, 64, 9)
    x = torch.randn(500, 64, 9, device=dev)
    y1 = lin(x)
    monkeypatch.setenv("FEQ_EQLINEAR", "lib")
    y2 = lin(x)
    assert rel_err(y1, y2) < TOL


def test_block_uses_the_kernels(dev):
    """A transformer block's QK projection and MLP run k_eql_mm (forward and
    input gradient: six launches) and its output matches the library path."""
    torch.manual_seed(0)
    blk = fe.EquivariantTransformerBlock(fe.Repr([0, 1, 2], 64), fe.Repr([0, 1, 2], 64), num_heads=8).to(dev)
    N, k = 300, 12
    g = torch.Generator().manual_seed(1)
    coords = torch.randn(N, 3, generator=g) * 4
    d = torch.cdist(coords, coords)
    d.fill_diagonal_(float("inf"))
    src = d.topk(k, largest=False).indices.reshape(-1)
    dst = torch.arange(N).repeat_interleave(k)
    vec = (coords[src] - coords[dst]).to(dev)
    P, Q = fe.WignerDBasis([fe.Repr([0, 1, 2], 1), fe.Repr([0, 1, 2], 1)]).to(dev)(vec)
    x = torch.randn(N, 64, 9, generator=g).to(dev).requires_grad_(True)
    graph = fe.Graph(src.to(dev), dst.to(dev), N)
    NAT.profile_summary()
    NAT.profile_enable(True)
    out = blk(P, Q, x, vec.norm(dim=-1), graph)
    out.square().sum().backward()
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    launched = NAT.profile_summary()
    assert launched.get("k_eql_mm", (0,))[0] == 6, launched
    assert launched.get("k_eql_wgrad", (0,))[0] == 3, launched
