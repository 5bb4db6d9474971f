"""Half-precision modules computed in float32.

A composed module (attention layer, transformer block, transformer) moved to
bfloat16/float16 keeps its parameters, inputs and outputs in that dtype but
runs in float32 inside: one cast of the parameters and inputs on the way in,
one of the output on the way out, autograd carrying the gradients back to the
half-precision leaves.  The kernels then run their float32 forms, every
intermediate (normalisation statistics, softmax sums, parameter-gradient
reductions) keeps float32 precision, and the result differs from a float64
evaluation on the same half-precision values by the output rounding alone.
The normalisations keep the epsilon of the module's dtype (1e-5), as the
reference's half-precision modules use.
(The edgewise layer at the high-degree layouts has genuine bf16 kernels and is
not wrapped.)
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..utils import epsilon_dtype

HALF = (torch.float16, torch.bfloat16)


def half_dtype(*tensors) -> torch.dtype | None:
    """The half-precision dtype of the first such CUDA tensor, else None."""
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.is_cuda and t.dtype in HALF:
            return t.dtype
    return None


def _up(v):
    if isinstance(v, torch.Tensor) and v.is_floating_point() and v.dtype != torch.float32:
        return v.float()
    return v


def _up_all(named) -> dict:
    """float32 copies of named tensors: those of one half-precision dtype and
    device are cast together (one concatenation and one cast, split back into
    views: two launches instead of one per tensor, and one for their
    gradients); the rest one by one."""
    named = list(named)
    out, groups = {}, {}
    for k, v in named:
        if (isinstance(v, torch.Tensor) and v.is_floating_point() and v.dtype in HALF
                and v.numel() > 0):
            groups.setdefault((v.dtype, v.device), []).append((k, v))
        else:
            out[k] = _up(v)
    for items in groups.values():
        if len(items) == 1:
            out[items[0][0]] = _up(items[0][1])
            continue
        flat = torch.cat([v.reshape(-1) for _, v in items]).float()
        for (k, v), piece in zip(items, torch.split(flat, [v.numel() for _, v in items])):
            out[k] = piece.view(v.shape)
    return out


def run_float32(module: nn.Module, dtype: torch.dtype, args: tuple, kwargs: dict):
    """``module(*args, **kwargs)`` with float32 copies of its floating
    parameters, buffers and tensor arguments; the output cast to ``dtype``."""
    state = _up_all(module.named_parameters())
    state.update(_up_all(module.named_buffers()))
    seen = {}

    def up(v):   # one float32 copy per distinct argument (P passed as P and Q: one cast)
        if not isinstance(v, torch.Tensor):
            return v
        if id(v) not in seen:
            seen[id(v)] = _up(v)
        return seen[id(v)]

    with epsilon_dtype(dtype):          # the norms keep get_epsilon(dtype) (utils.py:19-27)
        out = torch.func.functional_call(module, state, tuple(up(a) for a in args),
                                         {k: up(v) for k, v in kwargs.items()})
    return out.to(dtype)
