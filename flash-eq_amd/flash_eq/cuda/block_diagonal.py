"""The generic block-diagonal op (drop-in for ``flash_eq/cuda/block_diagonal.py:206-274``).

``block_diagonal_cuda`` keeps the reference's signature and autograd contract
(gradients for features, radial table and distances).  It runs the HIP
kernels of ``csrc/blockdiag.hip`` through ``libflasheq.so``; there is no CPU
implementation (as in the reference, a missing GPU raises
``CUDANotAvailableError``).  Unlike the reference it needs no distance sort,
no host synchronisation and no device-side lvals.
"""
from __future__ import annotations

from functools import lru_cache
from typing import Tuple

import torch

from .. import _native as N
from ..ops import BlockDiagonalFn
from .._native import CUDANotAvailableError

__all__ = ["block_diagonal_cuda", "CUDANotAvailableError"]


@lru_cache(maxsize=256)
def _layout(lvals_in: Tuple[int, ...], lvals_out: Tuple[int, ...], cin: int, cout: int):
    return N.make_layout(lvals_in, lvals_out, cin, cout)


def block_diagonal_cuda(features: torch.Tensor, radial_table: torch.Tensor, distances: torch.Tensor,
                        product_repr, bin_param1: float, bin_param2: float, num_bins: int,
                        log_bins: bool = False, sh_scale: float = 0.1) -> torch.Tensor:
    """out[e] = Lambda(r_e) features[e] in the m-first basis.

    features (E, Cin, Din), radial_table (num_bins+1, Cout, Cin, Wdim),
    distances (E,) -> (E, Cout, Dout).
    """
    cout = radial_table.size(1)
    dout = product_repr.rep2.dim()
    if features.size(0) == 0:
        return torch.zeros(0, cout, dout, device=features.device, dtype=features.dtype)
    N.require_cuda_tensor(features, "features")
    lin = tuple(int(l) for l in product_repr.rep1.lvals.tolist())
    lout = tuple(int(l) for l in product_repr.rep2.lvals.tolist())
    layout = _layout(lin, lout, int(features.size(1)), int(cout))
    binning = N.make_binning(bin_param1, bin_param2, num_bins, log_bins, sh_scale)
    return BlockDiagonalFn.apply(features, radial_table, distances.to(features.dtype), layout, binning)
