"""Norm-based gating (drop-in for ``flash_eq/layers/gating.py:17-76``).

On float32 GPU tables the irrep norms and the sigmoid gate run as kernels
(``csrc/nodeside.hip``) around the Linear's GEMM; otherwise PyTorch."""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import ops
from ..representations import Repr
from ..utils import get_epsilon, init_linear_weights
from .linear import rows_linear
from .norm import RepNorm, irrep_expand, irrep_slices


class EquivariantGating(nn.Module):
    """x * sigmoid(Linear(per-irrep norms)) broadcast over each irrep's components."""

    def __init__(self, repr: Repr) -> None:
        super().__init__()
        self.repr = repr
        self.norm = RepNorm(repr)
        width = repr.nreps() * repr.mult
        self.linear = nn.Linear(width, width)
        self.register_buffer("ix", torch.tensor(repr.indices(), dtype=torch.long))
        self.outdims = (repr.mult, repr.nreps())
        self._slices = irrep_slices(repr)
        self.activation = nn.Sigmoid()
        self.apply(init_linear_weights)
        self._lv = tuple(int(l) for l in repr.lvals.tolist())

    def kernels_ok(self, st: torch.Tensor) -> bool:
        return self.norm._epsilon is None and ops.node_kernels_ok(
            st, self._lv, self.repr.mult, self.linear.weight, self.linear.bias)

    def forward_cm(self, st_cm: torch.Tensor) -> torch.Tensor:
        """The gating of component-major features (dim, N, mult); kernels_ok."""
        return ops.GatingFn.apply(st_cm, self.linear.weight, self.linear.bias, self._lv,
                                  self.repr.mult, get_epsilon(st_cm.dtype), True)

    def forward(self, st: torch.Tensor) -> torch.Tensor:
        if self.kernels_ok(st):
            return ops.GatingFn.apply(st, self.linear.weight, self.linear.bias, self._lv,
                                      self.repr.mult, get_epsilon(st.dtype))
        norms = self.norm(st)
        *batch, _, _ = norms.shape
        flat = norms.flatten(-2, -1)
        lin = rows_linear(flat.reshape(-1, flat.shape[-1]), self.linear.weight) + self.linear.bias
        gates = self.activation(lin.view(*batch, *self.outdims))
        return st * irrep_expand(gates, self._slices)
