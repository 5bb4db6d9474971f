"""ctypes binding of ``libflasheq.so`` (the C ABI declared in ``include/flasheq.h``).

The library is the only compute path for the hot-path ops.  Loading fails
loudly: without a GPU the ops raise ``CUDANotAvailableError`` (the reference's
error type, ``flash_eq/cuda/block_diagonal.py:34-55``); with a GPU but no built
library they raise ``ImportError`` naming the build command.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional, Sequence

import torch

from ._build import LIB_PATH

FEQ_MAX_BLOCKS = 17
FEQ_MAX_SLOTS = 128
FEQ_EW_HALF_ACCURACY = 1          # flags of feq_edgewise_*_ex
POOL_MAX_HEADS = 16               # heads of feq_edgewise_*_src_pool


class CUDANotAvailableError(RuntimeError):
    """Raised when a GPU is required but none is visible (reference name kept)."""


class FeqLayout(ctypes.Structure):
    _fields_ = [
        ("cin", ctypes.c_int32), ("cout", ctypes.c_int32),
        ("din", ctypes.c_int32), ("dout", ctypes.c_int32),
        ("wdim", ctypes.c_int32), ("nblocks", ctypes.c_int32),
        ("blk", (ctypes.c_int32 * 6) * FEQ_MAX_BLOCKS),
        ("lslot_in", ctypes.c_int8 * FEQ_MAX_SLOTS),
        ("lslot_out", ctypes.c_int8 * FEQ_MAX_SLOTS),
        ("has_lpos", ctypes.c_int32),
    ]


class FeqBinning(ctypes.Structure):
    _fields_ = [
        ("p1", ctypes.c_float), ("p2", ctypes.c_float),
        ("num_bins", ctypes.c_int32), ("log_bins", ctypes.c_int32),
        ("sh_scale", ctypes.c_float),
    ]


_lib: Optional[ctypes.CDLL] = None
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float
_SZ = ctypes.c_size_t

_SIGS = {
    "feq_last_error": ([], ctypes.c_char_p),
    "feq_abi_version": ([], ctypes.c_int),
    "feq_profile_enable": ([ctypes.c_int], ctypes.c_int),
    "feq_profile_summary": ([ctypes.c_char_p, _SZ], ctypes.c_int),
    "feq_layout_init": ([_P, _P, _I32, _P, _I32, _I32, _I32], ctypes.c_int),
    "feq_bin_edges": ([_P, _I64, _P, _P, _P, _P], ctypes.c_int),
    "feq_blockdiag_workspace": ([_P, _P, _I64], _SZ),
    "feq_blockdiag_fwd": ([_P, _P, _I64, _P, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_blockdiag_bwd": ([_P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_blockdiag_fwd_f64": ([_P, _P, _I64, _P, _P, _P, _P, _P], ctypes.c_int),
    "feq_blockdiag_bwd_f64": ([_P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_edgewise_fwd_workspace": ([_P, _P, _I32, _I64], _SZ),
    "feq_edgewise_workspace": ([_P, _P, _I32, _I64], _SZ),
    "feq_edgewise_fwd": ([_P, _P, _I32, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_edgewise_bwd": ([_P, _P, _I32, _I64, _P, _P, _P, _P, _P, _P, _P,
                          _P, _P, _P, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_edgewise_src_supported": ([_P, _P, _I32], ctypes.c_int),
    "feq_edgewise_fused_supported": ([_P, _P, _I32], ctypes.c_int),
    "feq_edgewise_pq_supported": ([_P, _P, _I32], ctypes.c_int),
    # L, b, rank, E, x, num_src, src, P, Q, dist, C, F, y, ym, flags, ws, ws_bytes, stream
    "feq_edgewise_fwd_ym": ([_P, _P, _I32, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _SZ,
                             _P], ctypes.c_int),
    # L, b, rank, E, gy, x, num_src, src, perm_src, offsets_src, P, Q, dist, C, F, ym,
    # gx, gC, gF, gdist, gP, gQ, flags, ws, ws_bytes, stream
    "feq_edgewise_bwd_pq": ([_P, _P, _I32, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                             _P, _P, _P, _P, _P, _P, _I32, _P, _SZ, _P], ctypes.c_int),
    "feq_edgewise_fwd_src": ([_P, _P, _I32, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
                             ctypes.c_int),
    "feq_edgewise_fwd_src_noalloc": ([_P, _P, _I32, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P],
                                     ctypes.c_int),
    "feq_edgewise_bwd_src": ([_P, _P, _I32, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P,
                              _P, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_edgewise_fwd_src_ex": ([_P, _P, _I32, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _I32, _P,
                                 _SZ, _P], ctypes.c_int),
    "feq_edgewise_bwd_src_nodes_ex": ([_P, _P, _I32, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P,
                                       _P, _P, _P, _P, _P, _P, _I32, _P, _SZ, _P], ctypes.c_int),
    "feq_edgewise_bwd_src_nodes_workspace": ([_P, _P, _I32, _I64], _SZ),
    "feq_edgewise_pool_supported": ([_P, _P, _I32], ctypes.c_int),
    # as feq_edgewise_fwd_src_pool with ym after y_pos
    "feq_edgewise_fwd_src_pool_ym": ([_P, _P, _I32, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _I32, _I32,
                                      _P, _P, _P, _I64, _P, _P, _P, _I32, _P, _SZ, _P], ctypes.c_int),
    # as feq_edgewise_bwd_src_pool with ym after F and grad_P, grad_Q after grad_dist
    "feq_edgewise_bwd_src_pool_pq": ([_P, _P, _I32, _I64, _P, _P, _I32, _I32, _P, _I64, _P, _I64, _P, _P,
                                      _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _SZ, _P],
                                     ctypes.c_int),
    "feq_edgewise_fwd_src_pool_workspace": ([_P, _P, _I32, _I64], _SZ),
    "feq_edgewise_fwd_src_pool": ([_P, _P, _I32, _I64, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _I32, _I32,
                                   _P, _P, _P, _I64, _P, _P, _I32, _P, _SZ, _P], ctypes.c_int),
    "feq_edgewise_bwd_src_pool": ([_P, _P, _I32, _I64, _P, _P, _I32, _I32, _P, _I64, _P, _I64, _P, _P,
                                   _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _P, _SZ, _P],
                                  ctypes.c_int),
    "feq_edgewise_bwd_src_nodes": ([_P, _P, _I32, _I64, _P, _P, _I64, _P, _P, _P, _P, _P, _P,
                                    _P, _P, _P, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_edgewise_hl_supported": ([_P, _P, _I32], ctypes.c_int),
    "feq_edgewise_hl_workspace": ([_P, _P, _I32, _I64, _I32], _SZ),
    # node-side norms and gating: (lvals, nreps, mult, N, ...)
    "feq_sepnorm_fwd": ([_P, _I32, _I32, _I64, _P, _P, _P, _P, _F, _P, _P], ctypes.c_int),
    "feq_sepnorm_fwd_cm": ([_P, _I32, _I32, _I64, _P, _P, _P, _P, _F, _P, _P], ctypes.c_int),
    "feq_sepnorm_bwd_cm": ([_P, _I32, _I32, _I64, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _SZ, _P],
                           ctypes.c_int),
    "feq_sum_tables": ([_P, _I32, _I64, _P, _P], ctypes.c_int),
    "feq_sepnorm_bwd_add": ([_P, _I32, _I32, _I64, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _SZ, _I32,
                             _P], ctypes.c_int),
    "feq_scale_add_cm": ([_P, _P, _P, _I64, _I32, _I32, _P, _P], ctypes.c_int),
    "feq_scale_add_cm_workspace": ([], _SZ),
    "feq_scale_add_cm_bwd": ([_P, _P, _P, _I64, _I32, _I32, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_sepnorm_workspace": ([_P, _I32, _I32, _I64], _SZ),
    "feq_sepnorm_bwd": ([_P, _I32, _I32, _I64, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _SZ, _P],
                        ctypes.c_int),
    "feq_eqnorm_fwd": ([_P, _I32, _I32, _I64, _P, _P, _P, _F, _F, _P, _P], ctypes.c_int),
    "feq_eqnorm_fwd_cm": ([_P, _I32, _I32, _I64, _P, _P, _P, _F, _F, _P, _P], ctypes.c_int),
    "feq_eqnorm_bwd_cm": ([_P, _I32, _I32, _I64, _P, _P, _P, _P, _F, _F, _P, _P, _P, _P, _SZ, _P],
                          ctypes.c_int),
    "feq_eqnorm_bwd_add": ([_P, _I32, _I32, _I64, _P, _P, _P, _P, _F, _F, _P, _P, _P, _P, _P, _SZ, _I32, _P],
                           ctypes.c_int),
    "feq_eqnorm_workspace": ([_P, _I32, _I32, _I64], _SZ),
    "feq_eqnorm_bwd": ([_P, _I32, _I32, _I64, _P, _P, _P, _P, _F, _F, _P, _P, _P, _P, _SZ, _P],
                       ctypes.c_int),
    "feq_gate_norms": ([_P, _I32, _I32, _I64, _I32, _P, _F, _P, _P], ctypes.c_int),
    "feq_gate_apply": ([_P, _I32, _I32, _I64, _I32, _P, _P, _P, _P], ctypes.c_int),
    "feq_gate_bwd_lin": ([_P, _I32, _I32, _I64, _I32, _P, _P, _P, _P, _P], ctypes.c_int),
    "feq_gate_bwd_x": ([_P, _I32, _I32, _I64, _I32, _P, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "feq_edgewise_hl_fwd": ([_P, _P, _I32, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
                            ctypes.c_int),
    "feq_edgewise_hl_bwd": ([_P, _P, _I32, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                             _P, _SZ, _P], ctypes.c_int),
    "feq_wigner_plan_doubles": ([_P, _I32], _SZ),
    "feq_wigner_basis": ([_P, _I32, _P, _P, _I64, _P, _P, _P], ctypes.c_int),
    "feq_wigner_basis_bwd": ([_P, _I32, _P, _P, _I64, _P, _P, _P, _P], ctypes.c_int),
    "feq_wigner_basis_f64": ([_P, _I32, _P, _P, _I64, _P, _P, _P], ctypes.c_int),
    "feq_wigner_basis_bwd_f64": ([_P, _I32, _P, _P, _I64, _P, _P, _P, _P], ctypes.c_int),
    "feq_csr_workspace": ([_I64, _I64], _SZ),
    "feq_csr_by_dst": ([_P, _I64, _I64, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_segment_sum": ([_P, _I64, _P, _P, _I64, _P, _P], ctypes.c_int),
    "feq_gather_rows": ([_P, _I64, _I64, _P, _I64, _P, _P], ctypes.c_int),
    "feq_sum_squares_workspace": ([], _SZ),
    "feq_sum_squares": ([_P, _I64, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_sum_squares_bf16": ([_P, _I64, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_radial_supported": ([_I32, _I32, _I32, _I32], ctypes.c_int),
    "feq_radial_workspace": ([_I32, _I32], _SZ),
    "feq_radial_fwd": ([_P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "feq_radial_bwd": ([_P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
                       ctypes.c_int),
    "feq_eqlinear_supported": ([_I32, _I32], ctypes.c_int),
    "feq_eqlinear_workspace": ([_I32, _I32, _I32], _SZ),
    "feq_eqlinear_fwd": ([_P, _I32, _I64, _I32, _I32, _P, _P, _P, _I32, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_eqlinear_bwd_x": ([_P, _I32, _I64, _I32, _I32, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_eqlinear_bwd_w_workspace": ([_P, _I32, _I64, _I32, _I32], _SZ),
    "feq_eqlinear_bwd_w": ([_P, _I32, _I64, _I32, _I32, _P, _P, _I32, _P, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_transpose": ([_P, _I64, _I64, _I64, _I32, _P, _P], ctypes.c_int),
    "feq_column_sums_workspace": ([_I64, _I64, _I32], _SZ),
    "feq_column_sums": ([_P, _I64, _I64, _I32, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_scale_add": ([_P, _P, _P, _I64, _P, _P], ctypes.c_int),
    "feq_scale_add_bwd": ([_P, _P, _P, _I64, _P, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_dot_f64_workspace": ([], _SZ),
    "feq_dot_f64": ([_P, _P, _I64, _P, _P, _SZ, _P], ctypes.c_int),
    "feq_attn_softmax_fwd": ([_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I32, _I32, _P, _F,
                              _P, _P, _I64, _P, _P, _P], ctypes.c_int),
    "feq_attn_softmax_bwd": ([_P, _I64, _P, _I64, _P, _P, _I64, _P, _P, _I64, _I32, _I32, _P,
                              _P, _P, _I64, _P, _P, _P, _I64, _P, _I64, _P, _P], ctypes.c_int),
    "feq_attn_softmax_fwd_cm": ([_P, _P, _I64, _I64, _I32, _P, _P, _I64, _P, _I64, _I32, _I32, _P, _F,
                                 _P, _P, _I64, _P, _P, _P], ctypes.c_int),
    "feq_attn_softmax_bwd_cm": ([_P, _P, _I64, _I64, _I32, _P, _P, _I64, _P, _P, _I64, _I32, _I32, _P,
                                 _P, _P, _I64, _P, _P, _P, _P, _P, _P], ctypes.c_int),
    "feq_attn_pool_fwd": ([_P, _P, _I64, _I32, _I32, _I32, _P, _P, _I64, _P, _P], ctypes.c_int),
    "feq_attn_pool_bwd": ([_P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P, _P, _P],
                          ctypes.c_int),
    "feq_attn_pool_grad_attn": ([_P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P, _P], ctypes.c_int),
}

EXPORTED_SYMBOLS = tuple(_SIGS)


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the shared library and declare every signature (no GPU needed)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(
            f"flash-eq HIP library not found at {path}.\n"
            "Build it with: python -c 'import __graft_entry__ as g; g.build()' "
            "(or python flash-eq_amd/flash_eq/_build.py)")
    lib = ctypes.CDLL(path)
    for name, (args, res) in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def lib() -> ctypes.CDLL:
    """The library, for compute calls: requires a visible GPU."""
    if not torch.cuda.is_available():
        raise CUDANotAvailableError(
            "flash-eq (MI355X build) requires a ROCm GPU. No GPU was detected: "
            "torch.cuda.is_available() is False.")
    return load_library()


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load_library().feq_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg} (code {rc})")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def make_layout(lvals_in: Sequence[int], lvals_out: Sequence[int], cin: int, cout: int) -> FeqLayout:
    li = (ctypes.c_int32 * len(lvals_in))(*[int(v) for v in lvals_in])
    lo = (ctypes.c_int32 * len(lvals_out))(*[int(v) for v in lvals_out])
    out = FeqLayout()
    rc = load_library().feq_layout_init(ctypes.byref(out), li, len(lvals_in), lo, len(lvals_out),
                                        int(cin), int(cout))
    check(rc, "feq_layout_init")
    return out


def make_binning(p1: float, p2: float, num_bins: int, log_bins: bool, sh_scale: float) -> FeqBinning:
    return FeqBinning(float(p1), float(p2), int(num_bins), int(bool(log_bins)), float(sh_scale))


def require_cuda_tensor(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise CUDANotAvailableError(
            f"{name} must be a GPU tensor: the flash-eq hot path runs only on the GPU "
            f"(got device {t.device}).")


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Caller-owned scratch for the library, from the caching allocator."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def profile_enable(on: bool) -> None:
    """Start (clearing nothing) or stop bracketing every library launch with HIP events."""
    check(load_library().feq_profile_enable(int(bool(on))), "feq_profile_enable")


def profile_summary() -> dict:
    """{kernel name: (launches, total milliseconds)} of the launches recorded so far.

    Waits for the recorded events, then forgets them."""
    buf = ctypes.create_string_buffer(1 << 16)
    check(load_library().feq_profile_summary(buf, len(buf)), "feq_profile_summary")
    out = {}
    for line in buf.value.decode().splitlines():
        name, calls, ms = line.split("\t")
        out[name] = (int(calls), float(ms))
    return out
