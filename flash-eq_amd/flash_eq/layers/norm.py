"""Equivariant normalisations (drop-in for ``flash_eq/layers/norm.py``).

Node-side O(N C D) elementwise work, kept in PyTorch (not on the edge hot path).
Formulas follow ``norm.py:19-249``.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..representations import Repr
from ..utils import get_epsilon


class RepNorm(nn.Module):
    """Per-irrep Euclidean norms sqrt(sum_{d in irrep} x_d^2 + eps): (..., dim) -> (..., nreps)."""

    def __init__(self, repr: Repr, epsilon: float | None = None) -> None:
        super().__init__()
        self.num_reps = repr.nreps()
        self._epsilon = epsilon
        self.register_buffer("indices", torch.tensor(repr.indices(), dtype=torch.long))

    def forward(self, st: torch.Tensor) -> torch.Tensor:
        eps = self._epsilon if self._epsilon is not None else get_epsilon(st.dtype)
        sq = st * st
        acc = torch.zeros(*sq.shape[:-1], self.num_reps, device=sq.device, dtype=sq.dtype)
        acc = acc.index_add(-1, self.indices, sq)
        return (acc + eps).sqrt()


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
        eps = self._epsilon if self._epsilon is not None else get_epsilon(x.dtype)
        rms = torch.sqrt(x.pow(2).mean(dim=(-2, -1), keepdim=True) + eps)
        return x * (self.weight[..., None] / rms)


class EquivariantLayerNorm(nn.Module):
    """LayerNorm over the channel axis of the per-irrep norms, applied as a rescale."""

    def __init__(self, repr: Repr, epsilon: float | None = None) -> None:
        super().__init__()
        self.mult = repr.mult
        self.norm = RepNorm(repr)
        self.lnorm = nn.LayerNorm(repr.mult) if repr.mult > 1 else None
        self._epsilon = epsilon
        self.register_buffer("ix", torch.tensor(repr.indices(), dtype=torch.long))

    def forward(self, f: torch.Tensor) -> torch.Tensor:
        eps = self._epsilon if self._epsilon is not None else get_epsilon(f.dtype)
        norms = self.norm(f)                                  # (..., mult, nreps)
        if self.lnorm is None:
            return f * (1.0 / (norms + eps))[..., self.ix]
        ln = self.lnorm(norms.transpose(-2, -1)).transpose(-2, -1)
        return f * (ln / (norms + eps))[..., self.ix]


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

    def forward(self, f: torch.Tensor) -> torch.Tensor:
        out = f.clone()
        if self.nscalar > 0:
            out[..., self.scalar_locs] = self.scalar_norm(f[..., self.scalar_locs])
        if self.nhigher > 0:
            out[..., self.higher_mask] = self.higher_norm(f[..., self.higher_mask])
        return out

    def extra_repr(self) -> str:
        return f"nscalar={self.nscalar}, nhigher={self.nhigher}"
