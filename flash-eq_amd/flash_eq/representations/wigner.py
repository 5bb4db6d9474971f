"""Wigner-D matrices and the per-edge WignerDBasis (drop-in for ``representations/wigner.py``).

* ``random_rotation`` and ``WignerD`` (``rot``/``rot_to_ez``) keep the
  reference's torch implementation (``wigner.py:27-240``): they are utilities
  for building rotations, not part of the per-edge hot path.
* ``WignerDBasis.forward`` -- the hot path -- runs the HIP kernel
  ``feq_wigner_basis``: the per-edge matrix exponential of the reference
  (``wigner.py:180-183``) is replaced by the closed form
  ``Z(phi) V Z(theta rho) V^T Z(-phi)`` (Z: the m-diagonal generator's 2x2
  rotations; V = exp(pi/2 G1), built here once per representation in float64).
  Module structure and buffer names (``_wigner_modules.i.generators``,
  ``_perm_i``) match the reference so state dicts interchange.
"""
from __future__ import annotations

import math
from typing import Sequence, cast

import torch
import torch.nn as nn

from .. import _native as N
from ..utils import get_epsilon
from .types import Irrep, Repr


def random_rotation(shape: tuple = (), device=None, dtype: torch.dtype = torch.float32):
    """Haar-random rotation(s) as (axis (..., 3), angle (...)) via a unit quaternion."""
    q = torch.randn((*shape, 4), device=device, dtype=dtype)
    q = q / q.norm(dim=-1, keepdim=True)
    sgn = torch.sign(q[..., 0:1])
    q = q * torch.where(sgn == 0, torch.ones_like(sgn), sgn)
    half = torch.acos(q[..., 0].clamp(-1.0, 1.0))
    angle = 2 * half
    sin_half = torch.sin(half)
    small = sin_half < 1e-6
    axis = q[..., 1:] / torch.where(small, torch.ones_like(sin_half), sin_half)[..., None]
    fallback = torch.zeros_like(axis)
    fallback[..., 2] = 1.0
    axis = torch.where(small[..., None], fallback, axis)
    axis = axis / (axis.norm(dim=-1, keepdim=True) + 1e-8)
    return axis, angle


class WignerD(nn.Module):
    """Wigner-D matrices of a representation from axis-angle rotations."""

    def __init__(self, repr: Repr) -> None:
        super().__init__()
        self.repr = repr
        dim = repr.dim()
        gens = torch.zeros(3, dim, dim)
        off = 0
        for ir in repr.irreps:
            n = ir.dim()
            gens[:, off:off + n, off:off + n] = ir._generators()
            off += n
        self.register_buffer("generators", gens.view(3, -1))

    def _apply(self, fn, *args, **kwargs):
        super()._apply(fn, *args, **kwargs)
        # matrix_exp is unreliable in float16: keep float16 generators in float32
        if self.generators.dtype == torch.float16:
            self.generators = self.generators.float()
        return self

    def rot(self, axis: torch.Tensor, angle: torch.Tensor, cartesian: bool = False) -> torch.Tensor:
        """``matrix_exp(angle * sum_k axis_k G_k)`` with slots [Lz, Lx, Ly] (``wigner.py:144-196``)."""
        if cartesian:
            axis = axis[..., [2, 0, 1]]
        dim = self.repr.dim()
        *batch, _ = axis.shape
        half = axis.dtype == torch.float16
        if half:
            axis, angle = axis.float(), angle.float()
        k = (axis @ self.generators).view(*batch, dim, dim) * angle[..., None, None]
        d = torch.nan_to_num(torch.linalg.matrix_exp(k), 0.0)
        if half:
            d = d.half()
        offs = self.repr.cumdims()
        for i, ir in enumerate(self.repr.irreps):
            if ir.l == 0:
                d[..., offs[i], offs[i]] = 1.0
        return d

    def rot_to_ez(self, directions: torch.Tensor, cartesian: bool = False) -> torch.Tensor:
        """Rotation relating e_z and ``directions`` (``wigner.py:198-240``), transposed."""
        eps = get_epsilon(directions.dtype)
        d = directions / (torch.linalg.norm(directions, dim=-1, keepdim=True) + eps)
        axis = torch.stack([-d[..., 1], d[..., 0], torch.zeros_like(d[..., 0])], dim=-1)
        axis = axis / (torch.linalg.norm(axis, dim=-1, keepdim=True) + eps)
        angle = torch.arccos(d[..., 2].clamp(-1 + eps, 1 - eps))
        return self.rot(axis, angle, cartesian).mT


def _build_m_order_permutation(lvals: torch.Tensor) -> torch.Tensor:
    """std (l, m) order -> m-first order: all m=0, then (+m, -m) per l (``wigner.py:243-272``)."""
    lv = [int(l) for l in lvals]
    starts = []
    off = 0
    for l in lv:
        starts.append(off)
        off += 2 * l + 1
    perm = [starts[k] + l for k, l in enumerate(lv)]
    for m in range(1, (max(lv) if lv else 0) + 1):
        for k, l in enumerate(lv):
            if l >= m:
                perm += [starts[k] + l + m, starts[k] + l - m]
    return torch.tensor(perm, dtype=torch.long)


def _z_matrix(z: torch.Tensor, partner: torch.Tensor, x: float) -> torch.Tensor:
    n = z.numel()
    out = torch.zeros(n, n, dtype=torch.float64)
    for r in range(n):
        out[r, r] += math.cos(float(z[r]) * x)
        p = int(partner[r])
        if p != r:
            out[r, p] += math.sin(float(z[r]) * x)
    return out


def _check_factorisation(g, v, z, partner) -> None:
    """exp(a (cos p G0 + sin p G1)) == Z(p) V Z(a) V^T Z(-p) at fixed sample angles."""
    for phi, ang in ((0.3, 1.1), (-2.0, 2.9), (1.7, 0.4)):
        k = ang * (math.cos(phi) * g[0] + math.sin(phi) * g[1])
        ref = torch.linalg.matrix_exp(k)
        fac = _z_matrix(z, partner, phi) @ v @ _z_matrix(z, partner, ang) @ v.T @ _z_matrix(z, partner, -phi)
        if (ref - fac).abs().max() > 1e-5:
            raise RuntimeError("closed-form Wigner-D factorisation does not hold for these generators")


def _wigner_plan(repr: Repr) -> torch.Tensor:
    """float64 constants of the closed-form kernel, per irrep: V | z | partner.

    V = exp(pi/2 G1) from the float32 generators (float64 arithmetic); z[r] is
    the signed m with which the m-diagonal generator G2 couples row r to its
    partner row.  The factorisation is checked against matrix_exp here.
    """
    chunks = []
    for ir in repr.irreps:
        n = ir.dim()
        g = ir._generators().to(torch.float64)
        v = torch.linalg.matrix_exp((math.pi / 2) * g[1])
        z = torch.zeros(n, dtype=torch.float64)
        partner = torch.arange(n, dtype=torch.float64)
        for r in range(n):
            nz = (g[2, r].abs() > 0.5).nonzero().flatten().tolist()
            if len(nz) > 1:
                raise RuntimeError("unexpected structure of the m-diagonal generator")
            if nz:
                m = float(g[2, r, nz[0]])
                if abs(m - round(m)) > 1e-5:
                    raise RuntimeError("non-integer coupling in the m-diagonal generator")
                z[r], partner[r] = round(m), nz[0]
        # the kernel relies on this structure: row r pairs with row 2l - r at m = l - r
        l = (n - 1) // 2
        if any(int(z[r]) != l - r or int(partner[r]) != n - 1 - r for r in range(n)):
            raise RuntimeError("m-diagonal generator does not pair row r with row 2l - r")
        _check_factorisation(g, v, z, partner)
        chunks += [v.reshape(-1), z, partner]
    return torch.cat(chunks) if chunks else torch.zeros(0, dtype=torch.float64)


class _WignerBasisFn(torch.autograd.Function):
    """One WignerDBasis output M (E, dim, dim) from the directions (E, 3); the
    backward (``feq_wigner_basis_bwd``) is the exact derivative of the
    reference's ``matrix_exp`` path (rot_to_ez, wigner.py:198-240) with respect
    to the directions."""

    @staticmethod
    def forward(ctx, directions, lvals_i32, plan, perm_i32):
        dev = directions.device
        # float64 directions run the float64 kernels (a float64 module); every
        # other dtype the float32 ones (the reference computes half-precision
        # bases in float32, wigner.py:132-142)
        wdt = torch.float64 if directions.dtype == torch.float64 else torch.float32
        dirs = directions.detach().to(wdt).contiguous()
        E = dirs.shape[0]
        dim = int(perm_i32.numel())
        out = torch.empty(E, dim, dim, dtype=wdt, device=dev)
        lv = (N.ctypes.c_int32 * len(lvals_i32))(*lvals_i32)
        fn = "feq_wigner_basis_f64" if wdt == torch.float64 else "feq_wigner_basis"
        with torch.cuda.device(dev):
            rc = getattr(N.lib(), fn)(lv, len(lvals_i32), N.ptr(plan), N.ptr(perm_i32), E,
                                      N.ptr(dirs) if E else None, N.ptr(out) if E else None,
                                      N.stream_ptr(dev))
        N.check(rc, fn)
        ctx.save_for_backward(dirs, plan, perm_i32)
        ctx.meta = (tuple(lvals_i32), directions.dtype)
        return out

    @staticmethod
    def backward(ctx, grad):
        dirs, plan, perm_i32 = ctx.saved_tensors
        lvals, ddt = ctx.meta
        dev = dirs.device
        E = dirs.shape[0]
        g = grad.detach().to(dirs.dtype).contiguous()
        gd = torch.empty_like(dirs)
        lv = (N.ctypes.c_int32 * len(lvals))(*lvals)
        fn = "feq_wigner_basis_bwd_f64" if dirs.dtype == torch.float64 else "feq_wigner_basis_bwd"
        with torch.cuda.device(dev):
            rc = getattr(N.lib(), fn)(lv, len(lvals), N.ptr(plan), N.ptr(perm_i32), E,
                                      N.ptr(dirs) if E else None, N.ptr(g) if E else None,
                                      N.ptr(gd) if E else None, N.stream_ptr(dev))
        N.check(rc, fn)
        return gd.to(ddt), None, None, None


class WignerDBasis(nn.Module):
    """Per-edge basis matrices for a list of representations (``wigner.py:275-370``).

    Returns one (E, dim, dim) matrix per representation (float64 for float64
    directions, else float32 cast to a half-precision input's dtype); column j is
    column ``perm[j]`` of the Wigner-D matrix of the rotation taking e_z to the
    edge direction.  Representations with equal lvals share one result tensor.
    """

    def __init__(self, reprs: Sequence[Repr]) -> None:
        super().__init__()
        if len(reprs) == 0:
            raise ValueError("reprs must contain at least one Repr")
        self.reprs = list(reprs)
        index: dict = {}
        self._input_to_unique: list = []
        uniq: list = []
        for r in reprs:
            key = tuple(r.lvals.tolist())
            if key not in index:
                index[key] = len(uniq)
                uniq.append(r)
            self._input_to_unique.append(index[key])
        self._num_unique = len(uniq)
        self._wigner_modules = nn.ModuleList([WignerD(r) for r in uniq])
        for i, r in enumerate(uniq):
            self.register_buffer(f"_perm_{i}", _build_m_order_permutation(r.lvals))
        self._lvals = [[int(l) for l in r.lvals] for r in uniq]
        # kernel constants: host copies plus a per-device cache (kept out of
        # the module's buffers so dtype casts of the module never touch them)
        self._plans = [_wigner_plan(r) for r in uniq]
        self._perms = [_build_m_order_permutation(r.lvals).to(torch.int32) for r in uniq]
        self._device_consts: dict = {}

    def _consts(self, device: torch.device):
        key = str(device)
        hit = self._device_consts.get(key)
        if hit is None:
            hit = [(p.to(device), q.to(device)) for p, q in zip(self._plans, self._perms)]
            self._device_consts[key] = hit
        return hit

    def forward(self, directions: torch.Tensor) -> tuple:
        N.require_cuda_tensor(directions, "directions")
        if directions.dim() != 2 or directions.shape[-1] != 3:
            raise ValueError(f"directions must have shape (E, 3), got {tuple(directions.shape)}")
        outs = []
        consts = self._consts(directions.device)
        for i in range(self._num_unique):
            plan, perm = consts[i]
            m = _WignerBasisFn.apply(directions, self._lvals[i], plan, perm)
            if directions.dtype in (torch.float16, torch.bfloat16):
                m = m.to(directions.dtype)
            outs.append(m)
        return tuple(outs[k] for k in self._input_to_unique)

    def extra_repr(self) -> str:
        return f"reprs=[{', '.join(str(r) for r in self.reprs)}], num_unique={self._num_unique}"
