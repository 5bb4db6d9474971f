"""Gradient of WignerDBasis with respect to the edge directions (``feq_wigner_basis_bwd``).

The reference differentiates its bases through ``torch.linalg.matrix_exp``
(``representations/wigner.py:183``) and the float32 frame of ``rot_to_ez``
(``:220-238``); EquivariantTransformer therefore carries coordinate gradients
(``transformer.py:406-410``).  The oracle's float64 ``matrix_exp`` path under
torch autograd is the check: every gradient within 1e-5 of it (relative to the
largest entry), for several irrep layouts, through the tuple of a multi-repr
basis (equal lvals share one output), and for the degenerate frames of the
reference: the zero vector and exactly -e_z, where the axis normalisation
divides by eps (the gradient is huge there, in the reference as here).
"""
import pytest
import torch

import flash_eq as fe
from oracle import wigner as OW

pytestmark = pytest.mark.gpu


def _dirs(E, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(E, 3, generator=g) * 2.0


@pytest.mark.parametrize("lvals", [[0, 1, 2], [0, 1], [1], [0, 1, 2, 3, 4, 5, 6], [2, 0, 1, 1]])
def test_basis_gradient_matches_matrix_exp_autograd(dev, lvals):
    E = 777
    v = _dirs(E, 5 + len(lvals))
    vd = v.to(dev).requires_grad_(True)
    (M,) = fe.WignerDBasis([fe.Repr(lvals, 3)]).to(dev)(vd)
    g = torch.Generator().manual_seed(99)
    W = torch.randn(M.shape, generator=g)
    (M * W.to(dev)).sum().backward()
    vo = v.double().requires_grad_(True)
    (OW.basis(lvals, vo) * W.double()).sum().backward()
    err = ((vd.grad.double().cpu() - vo.grad).abs().max() / vo.grad.abs().max()).item()
    print(f"lvals {lvals}: direction-gradient rel err {err:.2e}")
    assert err < 1e-5


def test_multi_repr_gradient_sums_over_outputs(dev):
    reprs = [fe.Repr([0, 1], 2), fe.Repr([0, 1, 2], 4), fe.Repr([0], 8), fe.Repr([0, 1, 2], 1)]
    E = 300
    v = _dirs(E, 17)
    vd = v.to(dev).requires_grad_(True)
    outs = fe.WignerDBasis(reprs).to(dev)(vd)
    assert outs[1] is outs[3]
    g = torch.Generator().manual_seed(5)
    Ws = [torch.randn(o.shape, generator=g) for o in outs]
    sum((o * w.to(dev)).sum() for o, w in zip(outs, Ws)).backward()
    vo = v.double().requires_grad_(True)
    refs = OW.basis_tuple([[int(l) for l in r.lvals] for r in reprs], vo)
    sum((o * w.double()).sum() for o, w in zip(refs, Ws)).backward()
    err = ((vd.grad.double().cpu() - vo.grad).abs().max() / vo.grad.abs().max()).item()
    assert err < 1e-5


def test_degenerate_frames_follow_the_reference(dev):
    """Zero vector and -e_z: axis 0 -> D = I in the forward; the gradient is the
    matrix exponential's derivative at 0 scaled by 1/eps, as torch gives it."""
    v = torch.tensor([[0.0, 0.0, 0.0], [0.0, 0.0, -2.0], [0.3, -0.2, 1.1], [0.0, 0.0, -0.5]])
    lv = [0, 1, 2]
    vd = v.to(dev).requires_grad_(True)
    (M,) = fe.WignerDBasis([fe.Repr(lv, 1)]).to(dev)(vd)
    W = torch.randn(M.shape, generator=torch.Generator().manual_seed(3))
    (M * W.to(dev)).sum().backward()
    vo = v.double().requires_grad_(True)
    (OW.basis(lv, vo) * W.double()).sum().backward()
    got, ref = vd.grad.double().cpu(), vo.grad
    assert torch.isfinite(got).all()
    rel = ((got - ref).abs() / ref.abs().clamp(min=1.0)).max().item()
    assert rel < 1e-4, (got, ref)


def test_plus_z_directions_take_the_float64_frame(dev):
    """Directions exactly along +e_z (and -e_z): the gradient kernel evaluates
    the reference's frame formula (rot_to_ez, wigner.py:198-240) in float64,
    where its clamp of d_z to [-1 + eps, 1 - eps] binds (d_z = |v| / (|v| +
    eps) lies within eps of +-1): the angle is arccos(1 - eps) whatever |v|,
    and no gradient passes the clamp, so every entry is finite.  The
    reference's own float32 autograd rounds the clamp's bounds to +-1 and
    returns NaN there (0 * -inf).  This pins the chosen, finite value: the
    float64 evaluation of the formula."""
    v = torch.tensor([[0.0, 0.0, 1.0], [0.0, 0.0, 2.5], [0.0, 0.0, 0.25], [0.0, 0.0, -1.0]])
    lv = [0, 1, 2]
    vd = v.to(dev).requires_grad_(True)
    (M,) = fe.WignerDBasis([fe.Repr(lv, 1)]).to(dev)(vd)
    W = torch.randn(M.shape, generator=torch.Generator().manual_seed(11))
    (M * W.to(dev)).sum().backward()
    got = vd.grad.double().cpu()
    vo = v.double().requires_grad_(True)
    (OW.basis(lv, vo) * W.double()).sum().backward()
    assert torch.isfinite(got).all()
    assert torch.all(got[:, 2] == 0.0)            # d_z itself carries no gradient on the axis
    rel = ((got - vo.grad).abs() / vo.grad.abs().clamp(min=1.0)).max().item()
    assert rel < 1e-4, (got, vo.grad)
    v32 = v.clone().requires_grad_(True)          # the float32 evaluation: NaN, as in the reference
    (OW.basis(lv, v32) * W).sum().backward()
    assert torch.isnan(v32.grad).any()


def test_zero_edges(dev):
    vd = torch.zeros(0, 3, device=dev, requires_grad=True)
    (M,) = fe.WignerDBasis([fe.Repr([0, 1, 2], 1)]).to(dev)(vd)
    M.sum().backward()
    assert vd.grad.shape == (0, 3)
