"""The reference's compiled-extension interface, served by ``libflasheq.so``.

The reference's ``_BlockDiagonalFunction`` (``flash_eq/cuda/block_diagonal.py:77-174``)
calls a pybind module with two functions (``block_diagonal.cu:1268-1282``,
``:1543-1558``, exported at ``:1758-1761``)::

    forward(features, radial_table, distances, sh_scale, bin_param1, bin_param2,
            num_bins, log_bins, lvals_in, lvals_out, Cout, dim_out, max_in_size) -> [output]
    backward(grad_output, features, radial_table, distances, sh_scale, bin_param1,
             bin_param2, num_bins, log_bins, lvals_in, lvals_out, dim_in, max_in_size,
             max_out_size) -> [grad_features, grad_radial_table, grad_distances]

This module has exactly those two functions, so the reference's
``_get_cuda_module`` (``block_diagonal.py:39-70``) can return it in place of the
pybind module and ``_BlockDiagonalFunction`` runs unchanged on MI355X.  It
depends on nothing but torch, ctypes and the library: set ``FLASHEQ_LIB`` to
the library's path, or keep it at ``../_lib/libflasheq.so`` beside this file.

Behaviour follows the pybind functions:
- inputs must be GPU tensors, contiguous, of one dtype (``CHECK_INPUT``,
  ``block_diagonal.cu:24-26``); violations raise ``RuntimeError``;
- float32 and float64 run their own kernels; float16 is computed in float32
  and returned in float16; other dtypes raise ``RuntimeError`` (the reference
  dispatches float64/float32/float16, ``AT_DISPATCH_FLOATING_TYPES_AND_HALF``);
- outputs are freshly allocated and owned by the caller; ``max_in_size`` /
  ``max_out_size`` / ``dim_in`` are accepted for signature compatibility (the
  kernels derive their sizes from the layout);
- the kernels launch on the current torch stream; the table gradient is
  summed per bin in a fixed order (the reference uses float atomics).
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

__all__ = ["forward", "backward"]

_P, _I32, _I64, _F, _SZ = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
_MAX_BLOCKS, _MAX_SLOTS = 17, 128


class _Layout(ctypes.Structure):
    _fields_ = [("cin", _I32), ("cout", _I32), ("din", _I32), ("dout", _I32), ("wdim", _I32),
                ("nblocks", _I32), ("blk", (_I32 * 6) * _MAX_BLOCKS),
                ("lslot_in", ctypes.c_int8 * _MAX_SLOTS), ("lslot_out", ctypes.c_int8 * _MAX_SLOTS),
                ("has_lpos", _I32)]


class _Binning(ctypes.Structure):
    _fields_ = [("p1", _F), ("p2", _F), ("num_bins", _I32), ("log_bins", _I32), ("sh_scale", _F)]


_lib = None
_lock = threading.Lock()


def _library() -> ctypes.CDLL:
    global _lib
    with _lock:
        if _lib is None:
            path = os.environ.get("FLASHEQ_LIB") or os.path.join(
                os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_lib", "libflasheq.so")
            if not os.path.exists(path):
                raise ImportError(f"libflasheq.so not found at {path} (set FLASHEQ_LIB)")
            lib = ctypes.CDLL(path)
            lib.feq_last_error.restype = ctypes.c_char_p
            lib.feq_layout_init.argtypes = [_P, _P, _I32, _P, _I32, _I32, _I32]
            lib.feq_blockdiag_workspace.argtypes = [_P, _P, _I64]
            lib.feq_blockdiag_workspace.restype = _SZ
            lib.feq_blockdiag_fwd.argtypes = [_P, _P, _I64, _P, _P, _P, _P, _P, _SZ, _P]
            lib.feq_blockdiag_bwd.argtypes = [_P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]
            lib.feq_blockdiag_fwd_f64.argtypes = [_P, _P, _I64, _P, _P, _P, _P, _P]
            lib.feq_blockdiag_bwd_f64.argtypes = [_P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]
            _lib = lib
    return _lib


def _check(rc: int, what: str) -> None:
    if rc:
        raise RuntimeError(f"{what}: {_library().feq_last_error().decode()}")


def _check_input(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _compute_dtype(features, *others) -> torch.dtype:
    dt = features.dtype
    for name, t in others:
        if t.dtype != dt:
            raise RuntimeError(f"{name} has dtype {t.dtype}, expected {dt} (the features' dtype)")
    if dt in (torch.float32, torch.float64):
        return dt
    if dt == torch.float16:
        return torch.float32
    raise RuntimeError(f"block_diagonal: not implemented for '{dt}'")


def _layout(lvals_in, lvals_out, cin: int, cout: int) -> _Layout:
    li = [int(v) for v in torch.as_tensor(lvals_in).tolist()]
    lo = [int(v) for v in torch.as_tensor(lvals_out).tolist()]
    L = _Layout()
    _check(_library().feq_layout_init(ctypes.byref(L), (_I32 * len(li))(*li), len(li),
                                      (_I32 * len(lo))(*lo), len(lo), int(cin), int(cout)),
           "feq_layout_init")
    return L


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def forward(features, radial_table, distances, sh_scale, bin_param1, bin_param2, num_bins,
            log_bins, lvals_in, lvals_out, Cout, dim_out, max_in_size):
    """``block_diagonal_forward_cuda`` (block_diagonal.cu:1268-1282): returns [output]
    (E, Cout, dim_out) in the features' dtype."""
    for t, n in ((features, "features"), (radial_table, "radial_table"), (distances, "distances")):
        _check_input(t, n)
    cdt = _compute_dtype(features, ("radial_table", radial_table), ("distances", distances))
    dev = features.device
    E = features.size(0)
    L = _layout(lvals_in, lvals_out, features.size(1), int(Cout))
    if L.dout != int(dim_out):
        raise RuntimeError(f"dim_out {int(dim_out)} does not match lvals_out (dimension {L.dout})")
    b = _Binning(float(bin_param1), float(bin_param2), int(num_bins), int(bool(log_bins)),
                 float(sh_scale))
    x, T, r = (t.to(cdt).contiguous() for t in (features, radial_table, distances))
    out = torch.zeros(E, int(Cout), int(dim_out), device=dev, dtype=cdt)
    if E:
        lib = _library()
        with torch.cuda.device(dev):
            if cdt == torch.float64:
                rc = lib.feq_blockdiag_fwd_f64(ctypes.byref(L), ctypes.byref(b), E, x.data_ptr(),
                                               T.data_ptr(), r.data_ptr(), out.data_ptr(), _stream(dev))
            else:
                rc = lib.feq_blockdiag_fwd(ctypes.byref(L), ctypes.byref(b), E, x.data_ptr(),
                                           T.data_ptr(), r.data_ptr(), out.data_ptr(), None, 0,
                                           _stream(dev))
        _check(rc, "forward")
    return [out.to(features.dtype)]


def backward(grad_output, features, radial_table, distances, sh_scale, bin_param1, bin_param2,
             num_bins, log_bins, lvals_in, lvals_out, dim_in, max_in_size, max_out_size):
    """``block_diagonal_backward_cuda`` (block_diagonal.cu:1543-1558): returns
    [grad_features, grad_radial_table, grad_distances] in the features' dtype."""
    for t, n in ((grad_output, "grad_output"), (features, "features"),
                 (radial_table, "radial_table"), (distances, "distances")):
        _check_input(t, n)
    cdt = _compute_dtype(features, ("grad_output", grad_output), ("radial_table", radial_table),
                         ("distances", distances))
    dev = features.device
    E = features.size(0)
    L = _layout(lvals_in, lvals_out, features.size(1), radial_table.size(1))
    if L.din != int(dim_in):
        raise RuntimeError(f"dim_in {int(dim_in)} does not match lvals_in (dimension {L.din})")
    b = _Binning(float(bin_param1), float(bin_param2), int(num_bins), int(bool(log_bins)),
                 float(sh_scale))
    g, x, T, r = (t.to(cdt).contiguous() for t in (grad_output, features, radial_table, distances))
    gx, gt, gr = torch.zeros_like(x), torch.zeros_like(T), torch.zeros_like(r)
    lib = _library()
    ws = torch.empty(max(int(lib.feq_blockdiag_workspace(ctypes.byref(L), ctypes.byref(b), E)), 1),
                     dtype=torch.uint8, device=dev)
    fn = lib.feq_blockdiag_bwd_f64 if cdt == torch.float64 else lib.feq_blockdiag_bwd
    with torch.cuda.device(dev):
        rc = fn(ctypes.byref(L), ctypes.byref(b), E, g.data_ptr() if E else None, x.data_ptr(),
                T.data_ptr(), r.data_ptr(), gx.data_ptr(), gt.data_ptr(), gr.data_ptr(),
                ws.data_ptr(), ws.numel(), _stream(dev))
    _check(rc, "backward")
    odt = features.dtype
    return [gx.to(odt), gt.to(odt), gr.to(odt)]
