"""Wigner-D matrices and the WignerDBasis (oracle, float64 via matrix_exp).

Restates ``representations/types.py:74-135`` (generators) and
``representations/wigner.py:112-240, 313-370`` (``rot``, ``rot_to_ez``,
``WignerDBasis.forward``).  The matrix exponential is the library routine
``torch.linalg.matrix_exp`` evaluated in float64 on the float32-rounded
generators, exactly the operands the reference feeds its float32 call.

Pinned by ``tests/test_oracle_wigner.py``:
* l=1 ``rot(cartesian=True)`` equals ``scipy.spatial.transform.Rotation``
  (the reference KAT ``tests/test_layers.py:645-699``);
* so(3) commutators ``[G0,G1]=G2`` (cyclic), orthogonality, ``D(0)=I``,
  homomorphism ``D(R1) D(R2) = D(R1 R2)``;
* the m=0 column of the l=1, l=2 basis matrices equals the closed-form real
  spherical harmonics of the edge direction;
* the special cases of ``rot_to_ez`` (zero vector, exactly -e_z -> identity).
"""
from __future__ import annotations

import math
from typing import List, Sequence

import numpy as np
import torch

from .layout import m_first_perm


def _ladder(l: int):
    """Float32-valued J+ (with the reference's minus sign) and J- (``types.py:74-84``)."""
    n = 2 * l + 1
    jp = np.zeros((n, n), np.float64)
    jm = np.zeros((n, n), np.float64)
    for m in range(-l, l):
        jp[m + 1 + l, m + l] = -float(np.sqrt(np.float32(l * (l + 1) - m * (m + 1)), dtype=np.float32))
    for m in range(-l + 1, l + 1):
        jm[m - 1 + l, m + l] = float(np.sqrt(np.float32(l * (l + 1) - m * (m - 1)), dtype=np.float32))
    return jp, jm


def _real_map(l: int) -> np.ndarray:
    """Complex -> real SH change of basis with overall phase (-i)^l (``types.py:114-135``)."""
    n = 2 * l + 1
    s = 2.0 ** -0.5
    q = np.zeros((n, n), np.complex128)
    for m in range(-l, 0):
        q[l + m, l - m] = s
        q[l + m, l + m] = -1j * s
    for m in range(1, l + 1):
        q[l + m, l + m] = ((-1) ** m) * s
        q[l + m, l - m] = 1j * ((-1) ** m) * s
    q[l, l] = 1.0
    return ((-1j) ** l) * q


def irrep_generators(l: int) -> np.ndarray:
    """(3, 2l+1, 2l+1) float32 generators in slot order [Lz, Lx, Ly] (``types.py:86-112``)."""
    jp, jm = _ladder(l)
    jx = 0.5 * (jp + jm)
    jy = -0.5j * (jp - jm)
    jz = 1j * np.diag(np.arange(-l, l + 1).astype(np.complex128))
    q = _real_map(l)
    qh = q.conj().T
    conv = [(qh @ j @ q).real.astype(np.float32) for j in (jy, jx, jz)]
    return np.stack(conv, 0)


def repr_generators(lvals: Sequence[int]) -> np.ndarray:
    """Block-diagonal (3, dim, dim) float32 generators (``wigner.py:112-130``)."""
    lv = [int(l) for l in lvals]
    dim = sum(2 * l + 1 for l in lv)
    g = np.zeros((3, dim, dim), np.float32)
    o = 0
    for l in lv:
        n = 2 * l + 1
        g[:, o:o + n, o:o + n] = irrep_generators(l)
        o += n
    return g


def _scalar_slots(lvals: Sequence[int]) -> List[int]:
    out, o = [], 0
    for l in lvals:
        if int(l) == 0:
            out.append(o)
        o += 2 * int(l) + 1
    return out


def rot(lvals: Sequence[int], axis: torch.Tensor, angle: torch.Tensor,
        cartesian: bool = False) -> torch.Tensor:
    """``WignerD.rot`` in float64: ``matrix_exp(angle * axis . G)`` (``wigner.py:144-196``).

    ``cartesian=True`` reorders the axis (x, y, z) -> (z, x, y); NaNs become 0
    (``nan_to_num``) and every l=0 diagonal entry is forced to 1.
    """
    axis = axis.to(torch.float64)
    angle = angle.to(torch.float64)
    if cartesian:
        axis = axis[..., [2, 0, 1]]
    g = torch.from_numpy(repr_generators(lvals)).to(torch.float64)
    dim = g.shape[-1]
    k = torch.einsum("...a,aij->...ij", axis, g) * angle[..., None, None]
    d = torch.linalg.matrix_exp(k)
    d = torch.nan_to_num(d, 0.0)
    for s in _scalar_slots(lvals):
        d[..., s, s] = 1.0
    return d.reshape(*axis.shape[:-1], dim, dim)


def edge_frame(directions: torch.Tensor, eps: float = 1e-8):
    """Axis and angle of ``rot_to_ez``, computed in the input dtype (``wigner.py:220-238``).

    ``d = v/(|v|+eps)``, ``axis = (-d_y, d_x, 0)/(|.|+eps)``,
    ``angle = arccos(clamp(d_z, -1+eps, 1-eps))``.
    """
    d = directions / (torch.linalg.norm(directions, dim=-1, keepdim=True) + eps)
    axis = torch.stack([-d[..., 1], d[..., 0], torch.zeros_like(d[..., 0])], dim=-1)
    axis = axis / (torch.linalg.norm(axis, dim=-1, keepdim=True) + eps)
    angle = torch.arccos(d[..., 2].clamp(-1 + eps, 1 - eps))
    return axis, angle


def rot_to_ez(lvals: Sequence[int], directions: torch.Tensor) -> torch.Tensor:
    """``WignerD.rot_to_ez`` = ``rot(axis, angle).mT`` (``wigner.py:198-240``), float64 result."""
    eps = 1e-5 if directions.dtype in (torch.float16, torch.bfloat16) else 1e-8
    axis, angle = edge_frame(directions, eps)
    return rot(lvals, axis, angle).mT


def basis(lvals: Sequence[int], directions: torch.Tensor) -> torch.Tensor:
    """One ``WignerDBasis`` output: ``rot_to_ez(v).mT[..., perm]`` (``wigner.py:358-367``).

    Returns float64 (E, dim, dim); column j is column ``perm[j]`` of the
    Wigner-D matrix of the rotation taking e_z to the edge direction.
    """
    m = rot_to_ez(lvals, directions).mT
    perm = torch.tensor(m_first_perm(lvals), dtype=torch.long)
    return m[..., perm]


def basis_tuple(reprs_lvals: Sequence[Sequence[int]], directions: torch.Tensor):
    """Dedup-by-lvals ``WignerDBasis.forward``: equal lvals give the same tensor object."""
    cache = {}
    out = []
    for lv in reprs_lvals:
        key = tuple(int(l) for l in lv)
        if key not in cache:
            cache[key] = basis(key, directions)
        out.append(cache[key])
    return tuple(out)


def random_rotation(shape=(), generator=None, dtype=torch.float32):
    """Haar-random axis/angle via a unit quaternion (``wigner.py:27-93``)."""
    q = torch.randn((*shape, 4), generator=generator, dtype=dtype)
    q = q / q.norm(dim=-1, keepdim=True)
    sgn = torch.sign(q[..., 0:1])
    sgn = torch.where(sgn == 0, torch.ones_like(sgn), sgn)
    q = q * sgn
    half = torch.acos(q[..., 0].clamp(-1.0, 1.0))
    angle = 2 * half
    sh = torch.sin(half)
    small = sh < 1e-6
    axis = q[..., 1:] / torch.where(small, torch.ones_like(sh), sh)[..., None]
    default = torch.zeros_like(axis)
    default[..., 2] = 1.0
    axis = torch.where(small[..., None], default, axis)
    axis = axis / (axis.norm(dim=-1, keepdim=True) + 1e-8)
    return axis, angle


def real_sh_l1(d: np.ndarray) -> np.ndarray:
    """Closed-form l=1 real harmonics of unit vectors in this basis' (m=-1,0,1) order."""
    x, y, z = d[..., 0], d[..., 1], d[..., 2]
    return np.stack([y, z, x], -1)


def real_sh_l2(d: np.ndarray) -> np.ndarray:
    """Closed-form normalised l=2 real harmonics (m=-2..2) of unit vectors."""
    x, y, z = d[..., 0], d[..., 1], d[..., 2]
    r3 = math.sqrt(3.0)
    return np.stack([r3 * x * y, r3 * y * z, 0.5 * (3 * z * z - 1), r3 * x * z,
                     0.5 * r3 * (x * x - y * y)], -1)
