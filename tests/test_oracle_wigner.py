"""Pins of the oracle's Wigner-D construction (oracle/wigner.py).

* scipy KAT: l=1 rot(cartesian=True) == Rotation.from_rotvec (tests/test_layers.py:645-699);
* so(3) algebra: cyclic commutators, antisymmetry, D(0)=I, orthogonality,
  homomorphism D(R1)D(R2) = D(R1 R2) with the composite read off the l=1 block;
* the m=0 column of the basis equals closed-form real spherical harmonics of
  the edge direction (l=1: (y, z, x); l=2: the five normalised quadratics);
* rot_to_ez special cases: zero vector and exactly -e_z give the identity.
"""
import math

import numpy as np
import pytest
import torch

from oracle import wigner as OW
from oracle.layout import m_first_perm


def test_scipy_kat_l1():
    from scipy.spatial.transform import Rotation
    g = torch.Generator().manual_seed(42)
    axis, angle = OW.random_rotation((32,), generator=g)
    mine = OW.rot([1], axis, angle, cartesian=True).numpy()
    ref = Rotation.from_rotvec((axis * angle[:, None]).double().numpy()).as_matrix()
    assert np.abs(mine - ref).max() < 1e-6


@pytest.mark.parametrize("l", [1, 2, 3, 4, 6])
def test_generator_algebra(l):
    g = torch.from_numpy(OW.irrep_generators(l)).double()
    for a in range(3):
        assert torch.allclose(g[a], -g[a].T, atol=0)
    comm = lambda x, y: x @ y - y @ x
    tol = 1e-5 * (l + 1) ** 2
    assert (comm(g[0], g[1]) - g[2]).abs().max() < tol
    assert (comm(g[1], g[2]) - g[0]).abs().max() < tol
    assert (comm(g[2], g[0]) - g[1]).abs().max() < tol
    # Casimir: sum G_a^2 = -l(l+1) I
    cas = g[0] @ g[0] + g[1] @ g[1] + g[2] @ g[2]
    assert (cas + l * (l + 1) * torch.eye(2 * l + 1, dtype=torch.float64)).abs().max() < tol


@pytest.mark.parametrize("lv", [[0, 1, 2], [1, 2, 2], [3]])
def test_orthogonal_identity_homomorphism(lv):
    g = torch.Generator().manual_seed(7)
    a1, t1 = OW.random_rotation((8,), generator=g, dtype=torch.float64)
    a2, t2 = OW.random_rotation((8,), generator=g, dtype=torch.float64)
    d1 = OW.rot(lv, a1, t1, cartesian=True)
    d2 = OW.rot(lv, a2, t2, cartesian=True)
    eye = torch.eye(d1.shape[-1], dtype=torch.float64)
    assert (d1 @ d1.mT - eye).abs().max() < 1e-5
    assert (OW.rot(lv, a1, torch.zeros(8, dtype=torch.float64)) - eye).abs().max() == 0
    # composite rotation from the l=1 (Cartesian) matrices, back to axis-angle
    from scipy.spatial.transform import Rotation
    r1 = OW.rot([1], a1, t1, cartesian=True).numpy()
    r2 = OW.rot([1], a2, t2, cartesian=True).numpy()
    rv = Rotation.from_matrix(r1 @ r2).as_rotvec()
    ang = np.linalg.norm(rv, axis=-1)
    ax = rv / ang[:, None]
    d12 = OW.rot(lv, torch.from_numpy(ax), torch.from_numpy(ang), cartesian=True)
    assert (d1 @ d2 - d12).abs().max() < 1e-5


def test_basis_m0_columns_are_real_harmonics():
    g = torch.Generator().manual_seed(3)
    d = torch.randn(200, 3, generator=g)
    d = d / d.norm(dim=-1, keepdim=True)
    p1 = OW.basis([1], d).numpy()
    p2 = OW.basis([2], d).numpy()
    dn = d.double().numpy()
    assert np.abs(p1[:, :, 0] - OW.real_sh_l1(dn)).max() < 1e-6
    assert np.abs(p2[:, :, 0] - OW.real_sh_l2(dn)).max() < 2e-6
    # combined repr: m=0 columns sit at the per-l m=0 slots
    p = OW.basis([0, 1, 2], d).numpy()
    assert np.abs(p[:, 0, 0] - 1).max() == 0
    assert np.abs(p[:, 1:4, 1] - OW.real_sh_l1(dn)).max() < 1e-6
    assert np.abs(p[:, 4:9, 2] - OW.real_sh_l2(dn)).max() < 2e-6


def test_rot_to_ez_special_directions():
    lv = [0, 1, 2]
    dirs = torch.tensor([[0.0, 0.0, 0.0], [0.0, 0.0, -1.0], [0.0, 0.0, 2.0]])
    m = OW.basis(lv, dirs)
    perm = m_first_perm(lv)
    ident_cols = torch.eye(9, dtype=torch.float64)[:, perm]
    assert torch.equal(m[0], ident_cols)       # zero vector: axis 0 -> identity
    assert torch.equal(m[1], ident_cols)       # exactly -e_z: axis 0 -> identity (reference quirk)
    assert (m[2] - ident_cols).abs().max() < 1e-6   # +e_z: angle 0


def test_basis_dedup_returns_same_object():
    d = torch.randn(5, 3)
    a, b, c = OW.basis_tuple([[0, 1], [0, 1], [0]], d)
    assert a is b and c.shape == (5, 1, 1)
