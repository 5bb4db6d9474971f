"""ctypes wrapper of the C per-edge restatement (``oracle/blockdiag_ref.c``).

Test infrastructure only.  ``build()`` runs ``make -C oracle``; the library
lives in ``oracle/_build`` (git-ignored).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Sequence

import numpy as np
import torch

from .blockdiag import Binning
from .layout import dim_of, weight_dim

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_bd.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-C", _HERE, "-s"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _ints(v: Sequence[int]):
    a = np.ascontiguousarray(np.asarray([int(x) for x in v], dtype=np.int32))
    return a, _ptr(a), len(v)


def _np(t: torch.Tensor, dt) -> np.ndarray:
    return np.ascontiguousarray(t.detach().cpu().numpy().astype(dt))


def forward(x, table, r, lvals_in, lvals_out, b: Binning) -> torch.Tensor:
    dt = np.float64 if x.dtype == torch.float64 else np.float32
    fn = lib().feqo_fwd_f64 if dt is np.float64 else lib().feqo_fwd_f32
    E, cin, din = x.shape
    _, cout, _, wd = table.shape
    dout = dim_of(lvals_out)
    assert wd == weight_dim(lvals_in, lvals_out)
    xa, ta, ra = _np(x, dt), _np(table, dt), _np(r, dt)
    y = np.zeros((E, cout, dout), dt)
    li, lip, nli = _ints(lvals_in)
    lo, lop, nlo = _ints(lvals_out)
    rc = fn(ctypes.c_int64(E), cin, cout, din, dout, wd, lip, nli, lop, nlo,
            ctypes.c_float(b.p1), ctypes.c_float(b.p2), b.num_bins, int(b.log_bins),
            ctypes.c_float(b.sigma), _ptr(xa), _ptr(ta), _ptr(ra), _ptr(y))
    assert rc == 0
    return torch.from_numpy(y)


def backward(gy, x, table, r, lvals_in, lvals_out, b: Binning):
    dt = np.float64 if x.dtype == torch.float64 else np.float32
    fn = lib().feqo_bwd_f64 if dt is np.float64 else lib().feqo_bwd_f32
    E, cin, din = x.shape
    nbp1, cout, _, wd = table.shape
    dout = dim_of(lvals_out)
    ga, xa, ta, ra = _np(gy, dt), _np(x, dt), _np(table, dt), _np(r, dt)
    gx = np.zeros_like(xa)
    gt = np.zeros_like(ta)
    gr = np.zeros_like(ra)
    li, lip, nli = _ints(lvals_in)
    lo, lop, nlo = _ints(lvals_out)
    rc = fn(ctypes.c_int64(E), cin, cout, din, dout, wd, lip, nli, lop, nlo,
            ctypes.c_float(b.p1), ctypes.c_float(b.p2), b.num_bins, int(b.log_bins),
            ctypes.c_float(b.sigma), _ptr(ga), _ptr(xa), _ptr(ta), _ptr(ra),
            _ptr(gx), _ptr(gt), _ptr(gr))
    assert rc == 0
    return torch.from_numpy(gx), torch.from_numpy(gt), torch.from_numpy(gr)


def binning(r: torch.Tensor, b: Binning):
    """(lo int32, t) per edge from the C restatement of ``compute_binning``."""
    dt = np.float64 if r.dtype == torch.float64 else np.float32
    fn = lib().feqo_binning_f64 if dt is np.float64 else lib().feqo_binning_f32
    ra = _np(r, dt)
    lo = np.zeros(ra.shape[0], np.int32)
    t = np.zeros_like(ra)
    fn(ctypes.c_int64(ra.shape[0]), _ptr(ra), ctypes.c_float(b.p1), ctypes.c_float(b.p2),
       b.num_bins, int(b.log_bins), _ptr(lo), _ptr(t))
    return torch.from_numpy(lo), torch.from_numpy(t)
