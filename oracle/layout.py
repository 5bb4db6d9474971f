"""Representation metadata and the m-first block layout (oracle).

Restates, independently of the product package:

* ``m_first_perm``     -- ``_build_m_order_permutation`` (``wigner.py:243-272``).
* ``block_params``     -- ``precompute_block_info`` (``block_diagonal.cu:1191-1266``),
                          equivalently ``_compute_block_sizes`` (``block_diagonal.py:181-203``)
                          and ``_extract_block_diagonal_weights`` (``patch/_conversion.py:99-140``).
* ``weight_dim``       -- ``ProductRepr.nreps`` (``types.py:157-171, 345-347``).

Pinned by ``tests/test_oracle_layout.py`` (hand-derived values and the
Wdim = sum_m n_in n_out (1 or 2) identity).
"""
from __future__ import annotations

from typing import List, Sequence, Tuple


def dim_of(lvals: Sequence[int]) -> int:
    return sum(2 * int(l) + 1 for l in lvals)


def std_index(lvals: Sequence[int], k: int, m: int) -> int:
    """Standard (l-major, m = -l..l) index of order ``m`` in irrep ``k``."""
    off = sum(2 * int(l) + 1 for l in lvals[:k])
    return off + int(lvals[k]) + m


def m_first_perm(lvals: Sequence[int]) -> List[int]:
    """Column permutation std -> m-first: all m=0 first, then (+m, -m) pairs per l."""
    lv = [int(l) for l in lvals]
    perm = [std_index(lv, k, 0) for k in range(len(lv))]
    for m in range(1, max(lv) + 1):
        for k, l in enumerate(lv):
            if l >= m:
                perm += [std_index(lv, k, m), std_index(lv, k, -m)]
    return perm


def weight_dim(lvals_in: Sequence[int], lvals_out: Sequence[int]) -> int:
    """Number of radial weights per (co, ci) channel pair."""
    return sum(2 * min(int(a), int(b)) + 1 for a in lvals_in for b in lvals_out)


def block_params(lvals_in: Sequence[int], lvals_out: Sequence[int]) -> List[Tuple[int, int, int, int, int, int]]:
    """``(m, n_in, n_out, in_off, out_off, w_off)`` for every m with a non-empty block.

    m-blocks with n_in == 0 or n_out == 0 are dropped and do not advance the
    offsets; an m=0 block advances by (n_in, n_out, n_in n_out), an m>0 block
    by twice that (``block_diagonal.cu:1218-1258``).
    """
    li = [int(l) for l in lvals_in]
    lo = [int(l) for l in lvals_out]
    mmax = max(max(li), max(lo))
    out = []
    in_off = out_off = w_off = 0
    for m in range(mmax + 1):
        n_in = sum(1 for l in li if l >= m)
        n_out = sum(1 for l in lo if l >= m)
        if n_in == 0 or n_out == 0:
            continue
        out.append((m, n_in, n_out, in_off, out_off, w_off))
        k = 1 if m == 0 else 2
        in_off += k * n_in
        out_off += k * n_out
        w_off += k * n_in * n_out
    return out


def slot_l(lvals: Sequence[int]) -> List[int]:
    """l value of every m-first component (the per-slot scaling exponent)."""
    lv = [int(l) for l in lvals]
    out = list(lv)
    for m in range(1, max(lv) + 1):
        for l in lv:
            if l >= m:
                out += [l, l]
    return out


def block_l(lvals: Sequence[int], m: int) -> List[int]:
    """l values of the irreps taking part in the m-block, in lvals order."""
    return [int(l) for l in lvals if int(l) >= m]
