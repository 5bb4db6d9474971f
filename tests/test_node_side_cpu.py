"""Node-side modules (norms, gating, EquivariantLinear) on the CPU.

The oracle's index-form restatements are first pinned against the vectors the
reference's own modules wrote (lvals [0, 1, 2]); the modules, which work on
per-irrep slices of the component axis, are then checked against the oracle
on layouts the vectors do not cover (scalars in the middle, repeated and
missing scalars, a single irrep), forward and gradients, in float64.
"""
import os

import numpy as np
import pytest
import torch

import flash_eq as fe
from oracle import layer as OL

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))
LAYOUTS = [[0, 1, 2], [1, 0, 2], [0, 0, 1, 2], [2, 1], [0], [1, 2, 0, 1]]


def G(key):
    return torch.from_numpy(GOLD[key])


def test_oracle_separable_norm_and_gating_match_reference_vectors():
    x = G("node__x").double()
    torch.manual_seed(4)
    sln = fe.SeparableEquivariantLayerNorm(fe.Repr([0, 1, 2], 6))
    y = OL.separable_layer_norm(x, [0, 1, 2], sln.scalar_norm.weight.double(),
                                sln.scalar_norm.bias.double(), sln.higher_norm.weight.double())
    assert (y - G("sln__y").double()).abs().max() < 2e-6
    torch.manual_seed(4)
    gate = fe.EquivariantGating(fe.Repr([0, 1, 2], 6))
    y = OL.gating(x, [0, 1, 2], gate.linear.weight.double(), gate.linear.bias.double())
    assert (y - G("gate__y").double()).abs().max() < 2e-6


def _randomise(m, g):
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=g, dtype=p.dtype))
    return m


def _check_grads(y, yref, inputs, refs, g):
    assert (y - yref).abs().max() < 1e-10
    go = torch.randn(y.shape, generator=g, dtype=torch.float64)
    gs = torch.autograd.grad(y, inputs, go)
    grs = torch.autograd.grad(yref, refs, go)
    for a, b in zip(gs, grs):
        assert (a - b).abs().max() < 1e-10


@pytest.mark.parametrize("lvals", LAYOUTS)
def test_separable_layer_norm_layouts(lvals):
    g = torch.Generator().manual_seed(len(lvals))
    rp = fe.Repr(lvals, 5)
    m = _randomise(fe.SeparableEquivariantLayerNorm(rp).double(), g)
    x = torch.randn(7, 5, rp.dim(), generator=g, dtype=torch.float64, requires_grad=True)
    y = m(x)
    has_s = hasattr(m, "scalar_norm")
    has_h = hasattr(m, "higher_norm")
    sw = m.scalar_norm.weight if has_s else None
    sb = m.scalar_norm.bias if has_s else None
    hw = m.higher_norm.weight if has_h else None
    yref = OL.separable_layer_norm(x, lvals, sw, sb, hw)
    params = [p for p in (sw, sb, hw) if p is not None]
    _check_grads(y, yref, [x] + params, [x] + params, g)


@pytest.mark.parametrize("lvals", LAYOUTS)
def test_layer_norm_gating_linear_layouts(lvals):
    g = torch.Generator().manual_seed(10 + len(lvals))
    rp = fe.Repr(lvals, 4)
    x = torch.randn(6, 4, rp.dim(), generator=g, dtype=torch.float64, requires_grad=True)
    ln = _randomise(fe.EquivariantLayerNorm(rp).double(), g)
    y = ln(x)
    yref = OL.equivariant_layer_norm(x, lvals, ln.lnorm.weight, ln.lnorm.bias)
    _check_grads(y, yref, [x, ln.lnorm.weight], [x, ln.lnorm.weight], g)
    gate = _randomise(fe.EquivariantGating(rp).double(), g)
    y = gate(x)
    yref = OL.gating(x, lvals, gate.linear.weight, gate.linear.bias)
    _check_grads(y, yref, [x, gate.linear.weight], [x, gate.linear.weight], g)
    lin = _randomise(fe.EquivariantLinear(rp, fe.Repr(lvals, 3), bias=True).double(), g)
    y = lin(x)
    yref = OL.equivariant_linear(x, lin.weight, lvals)
    if lin.bias is not None:
        offs = rp.cumdims().tolist()
        locs = [offs[k] for k, l in enumerate(lvals) if l == 0]
        yref = yref.clone()
        yref[..., locs] = yref[..., locs] + lin.bias
    params = [lin.weight] + ([lin.bias] if lin.bias is not None else [])
    _check_grads(y, yref, [x] + params, [x] + params, g)
