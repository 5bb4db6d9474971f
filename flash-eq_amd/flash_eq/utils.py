"""Small numeric helpers shared by the layers.

Mirrors the behaviour of the reference helpers in ``flash_eq/utils.py:8-27``
(Xavier init for ``nn.Linear`` with zero bias; dtype-aware epsilon).
"""
from __future__ import annotations

import contextlib
import threading

import torch
import torch.nn as nn

_LOW_PRECISION = (torch.float16, torch.bfloat16)


def init_linear_weights(module: nn.Module) -> None:
    """Xavier-uniform weight and zero bias for every ``nn.Linear``.

    Meant for ``module.apply(init_linear_weights)``; the RNG is consumed in
    the same order as the reference (``utils.py:8-16``) so seeded
    construction yields identical parameters.
    """
    if not isinstance(module, nn.Linear):
        return
    nn.init.xavier_uniform_(module.weight)
    if module.bias is not None:
        nn.init.zeros_(module.bias)


_EPS = threading.local()


def get_epsilon(dtype: torch.dtype) -> float:
    """Stabilising epsilon: 1e-5 for 16-bit floats, 1e-8 otherwise (``utils.py:19-27``).

    Inside ``epsilon_dtype(d)`` float32 tensors get d's epsilon: a half-precision
    module computed in float32 keeps the epsilon of its own dtype."""
    over = getattr(_EPS, "dtype", None)
    if over is not None and dtype == torch.float32:
        dtype = over
    return 1e-5 if dtype in _LOW_PRECISION else 1e-8


def half_precision_active(*tensors) -> bool:
    """True inside ``epsilon_dtype(d)`` for a 16-bit d (a half-precision module
    computed in float32), or when one of ``tensors`` is 16-bit: the caller's
    accuracy bar is then the half-precision one."""
    if getattr(_EPS, "dtype", None) in _LOW_PRECISION:
        return True
    return any(isinstance(t, torch.Tensor) and t.dtype in _LOW_PRECISION for t in tensors)


@contextlib.contextmanager
def epsilon_dtype(dtype: torch.dtype):
    prev = getattr(_EPS, "dtype", None)
    _EPS.dtype = dtype
    try:
        yield
    finally:
        _EPS.dtype = prev
