"""Equivariant normalisations (drop-in for ``flash_eq/layers/norm.py``).

Node-side O(N C D) work next to the edge path.  Formulas follow
``norm.py:19-249``.  On float32 GPU tables, ``SeparableEquivariantLayerNorm``
and ``EquivariantLayerNorm`` run fused HIP kernels (one wave per node, forward
and backward: ``csrc/nodeside.hip``).  Other dtypes and devices run the
PyTorch formulation below, in which per-irrep reductions and broadcasts are
slices of the component axis (one run of 2l+1 components per irrep): their
backward passes are slices, sums and broadcasts again.  The reference's
``x[..., ix]`` expansion has an ``index_put_(accumulate=True)`` backward, which
PyTorch runs as a sort over every element (4.5 ms per call at 20k nodes x 128
channels on MI355X).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import ops
from ..representations import Repr
from ..utils import get_epsilon


def irrep_slices(repr: Repr) -> list[tuple[int, int]]:
    """[start, stop) of every irrep's components along the last axis."""
    offs = repr.cumdims().tolist()
    return [(offs[k], offs[k + 1]) for k in range(repr.nreps())]


def irrep_sums(x: torch.Tensor, slices: list[tuple[int, int]]) -> torch.Tensor:
    """(..., dim) -> (..., nreps): the sum of each irrep's components."""
    return torch.stack([x[..., a:b].sum(-1) for a, b in slices], dim=-1)


def irrep_expand(g: torch.Tensor, slices: list[tuple[int, int]]) -> torch.Tensor:
    """(..., nreps) -> (..., dim): value k repeated over irrep k's components
    (the reference's ``g[..., repr.indices()]``)."""
    lead = g.shape[:-1]
    return torch.cat([g[..., k:k + 1].expand(*lead, b - a) for k, (a, b) in enumerate(slices)],
                     dim=-1)


class RepNorm(nn.Module):
    """Per-irrep Euclidean norms sqrt(sum_{d in irrep} x_d^2 + eps): (..., dim) -> (..., nreps)."""

    def __init__(self, repr: Repr, epsilon: float | None = None) -> None:
        super().__init__()
        self.num_reps = repr.nreps()
        self._epsilon = epsilon
        self.register_buffer("indices", torch.tensor(repr.indices(), dtype=torch.long))
        self._slices = irrep_slices(repr)

    def forward(self, st: torch.Tensor) -> torch.Tensor:
        eps = self._epsilon if self._epsilon is not None else get_epsilon(st.dtype)
        return (irrep_sums(st * st, self._slices) + eps).sqrt()


class _ChannelLayerNorm(nn.Module):
    """LayerNorm of scalar components over the channel axis (dim -2)."""

    def __init__(self, mult: int, nscalar: int, epsilon: float | None = None) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(mult, nscalar))
        self.bias = nn.Parameter(torch.zeros(mult, nscalar))
        self._epsilon = epsilon

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        eps = self._epsilon if self._epsilon is not None else get_epsilon(x.dtype)
        mu = x.mean(dim=-2, keepdim=True)
        sd = x.std(dim=-2, keepdim=True, unbiased=False)
        return (x - mu) / (sd + eps) * self.weight + self.bias


class _EquivariantRMSNorm(nn.Module):
    """One RMS over all channels and l>0 components, per-channel learnable scale."""

    def __init__(self, mult: int, epsilon: float | None = None) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(mult))
        self._epsilon = epsilon

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return x * self.factor([x])

    def factor(self, parts: list[torch.Tensor]) -> torch.Tensor:
        """weight / RMS over the channels and components of ``parts`` (the l > 0
        runs of one feature tensor), shaped (..., mult, 1)."""
        eps = self._epsilon if self._epsilon is not None else get_epsilon(parts[0].dtype)
        count = sum(p.shape[-2] * p.shape[-1] for p in parts)
        ssq = sum(p.pow(2).sum(dim=(-2, -1), keepdim=True) for p in parts)
        rms = torch.sqrt(ssq / count + eps)
        return self.weight[..., None] / rms


class EquivariantLayerNorm(nn.Module):
    """LayerNorm over the channel axis of the per-irrep norms, applied as a rescale."""

    def __init__(self, repr: Repr, epsilon: float | None = None) -> None:
        super().__init__()
        self.mult = repr.mult
        self.norm = RepNorm(repr)
        self.lnorm = nn.LayerNorm(repr.mult) if repr.mult > 1 else None
        self._epsilon = epsilon
        self.register_buffer("ix", torch.tensor(repr.indices(), dtype=torch.long))
        self._slices = irrep_slices(repr)
        self._lv = tuple(int(l) for l in repr.lvals.tolist())

    def _kernels_ok(self, f: torch.Tensor) -> bool:
        w = self.lnorm.weight if self.lnorm is not None else None
        b = self.lnorm.bias if self.lnorm is not None else None
        return self._epsilon is None and ops.node_kernels_ok(f, self._lv, self.mult, w, b) and (
            self.lnorm is None or (w is not None and b is not None))

    def cm_ok(self, f: torch.Tensor) -> bool:
        """Whether ``forward_cm`` takes these features (the kernels, and a node
        row of at most 1152 floats)."""
        return self._kernels_ok(f) and self.mult * sum(2 * l + 1 for l in self._lv) <= 1152

    def forward_cm(self, f: torch.Tensor) -> torch.Tensor:
        """The norm of node-major features returned component-major (dim, N,
        mult), for a channel-mixing map that follows; ``cm_ok(f)``."""
        w = self.lnorm.weight if self.lnorm is not None else None
        b = self.lnorm.bias if self.lnorm is not None else None
        ln_eps = self.lnorm.eps if self.lnorm is not None else 0.0
        return ops.EqNormFn.apply(f, w, b, self._lv, self.mult, get_epsilon(f.dtype), ln_eps, True)

    def forward_pair(self, f: torch.Tensor, cm: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """(the norm of f, f again for a second branch): the second branch's
        gradient is added in the norm's backward kernel, not by autograd in a
        separate pass.  The norm is component-major with ``cm``; ``cm_ok(f)``."""
        w = self.lnorm.weight if self.lnorm is not None else None
        b = self.lnorm.bias if self.lnorm is not None else None
        ln_eps = self.lnorm.eps if self.lnorm is not None else 0.0
        return ops.EqNormFn.apply(f, w, b, self._lv, self.mult, get_epsilon(f.dtype), ln_eps, cm, True)

    def forward(self, f: torch.Tensor) -> torch.Tensor:
        eps = self._epsilon if self._epsilon is not None else get_epsilon(f.dtype)
        w = self.lnorm.weight if self.lnorm is not None else None
        b = self.lnorm.bias if self.lnorm is not None else None
        if self._kernels_ok(f):
            ln_eps = self.lnorm.eps if self.lnorm is not None else 0.0
            return ops.EqNormFn.apply(f, w, b, self._lv, self.mult, eps, ln_eps)
        norms = self.norm(f)                                  # (..., mult, nreps)
        if self.lnorm is None:
            return f * irrep_expand(1.0 / (norms + eps), self._slices)
        ln = self.lnorm(norms.transpose(-2, -1)).transpose(-2, -1)
        return f * irrep_expand(ln / (norms + eps), self._slices)


class SeparableEquivariantLayerNorm(nn.Module):
    """EquiformerV2 separable norm: LayerNorm on scalars, shared RMS on l > 0."""

    def __init__(self, repr: Repr, epsilon: float | None = None) -> None:
        super().__init__()
        self.repr = repr
        nscalar, locs = repr.find_scalar()
        self.scalar_locs = locs
        self.nscalar = nscalar
        mask = torch.ones(repr.dim(), dtype=torch.bool)
        mask[locs] = False
        self.register_buffer("higher_mask", mask)
        self.nhigher = repr.nreps() - nscalar
        if nscalar > 0:
            self.scalar_norm = _ChannelLayerNorm(repr.mult, nscalar, epsilon)
        if self.nhigher > 0:
            self.higher_norm = _EquivariantRMSNorm(repr.mult, epsilon)
        self._lv = tuple(int(l) for l in repr.lvals.tolist())
        # component runs in order: ("s", j) = scalar number j, ("h", a, b) = a run
        # of consecutive l > 0 components
        self._runs: list[tuple] = []
        for k, (a, b) in enumerate(irrep_slices(repr)):
            if a in locs:
                self._runs.append(("s", locs.index(a)))
            elif self._runs and self._runs[-1][0] == "h" and self._runs[-1][2] == a:
                self._runs[-1] = ("h", self._runs[-1][1], b)
            else:
                self._runs.append(("h", a, b))

    def _kernel_args(self, f: torch.Tensor):
        ws = self.scalar_norm.weight if self.nscalar > 0 else None
        bs = self.scalar_norm.bias if self.nscalar > 0 else None
        wh = self.higher_norm.weight if self.nhigher > 0 else None
        if not (self.nscalar <= ops.NODE_MAX_SCALARS
                and ops.node_kernels_ok(f, self._lv, self.repr.mult, ws, bs, wh)):
            return None
        mod = self.scalar_norm if self.nscalar > 0 else self.higher_norm
        eps = mod._epsilon if mod._epsilon is not None else get_epsilon(f.dtype)
        return ws, bs, wh, eps

    def cm_ok(self, f: torch.Tensor) -> bool:
        """Whether ``forward_cm`` takes these features (the kernels, and a node
        row of at most 1152 floats)."""
        return self._kernel_args(f) is not None and self.repr.mult * self.repr.dim() <= 1152

    def forward_cm(self, f: torch.Tensor) -> torch.Tensor:
        """The norm of node-major features returned component-major (dim, N,
        mult), for a channel-mixing map that follows; ``cm_ok(f)``."""
        ws, bs, wh, eps = self._kernel_args(f)
        return ops.SepNormFn.apply(f, ws, bs, wh, self._lv, self.repr.mult, eps, True)

    def forward_pair(self, f: torch.Tensor, cm: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
        """(the norm of f, f again for a second branch such as the residual
        connection): the second branch's gradient is added in the norm's
        backward kernel, not by autograd in a separate pass.  The norm is
        component-major with ``cm``; ``cm_ok(f)``."""
        ws, bs, wh, eps = self._kernel_args(f)
        return ops.SepNormFn.apply(f, ws, bs, wh, self._lv, self.repr.mult, eps, cm, True)

    def forward(self, f: torch.Tensor) -> torch.Tensor:
        args = self._kernel_args(f)
        if args is not None:
            ws, bs, wh, eps = args
            return ops.SepNormFn.apply(f, ws, bs, wh, self._lv, self.repr.mult, eps)
        ys = None
        if self.nscalar > 0:
            xs = torch.cat([f[..., a:a + 1] for a in self.scalar_locs], dim=-1)
            ys = self.scalar_norm(xs)
        hp = [f[..., r[1]:r[2]] for r in self._runs if r[0] == "h"]
        fac = self.higher_norm.factor(hp) if hp else None
        out, i = [], 0
        for r in self._runs:
            if r[0] == "s":
                out.append(ys[..., r[1]:r[1] + 1])
            else:
                out.append(hp[i] * fac)
                i += 1
        return torch.cat(out, dim=-1) if len(out) > 1 else out[0]

    def extra_repr(self) -> str:
        return f"nscalar={self.nscalar}, nhigher={self.nhigher}"
