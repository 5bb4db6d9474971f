"""Pins of the oracle's layout bookkeeping (oracle/layout.py).

Values are hand-derived from the reference's three independent statements of
the m-first layout: _build_m_order_permutation (wigner.py:243-272),
precompute_block_info (block_diagonal.cu:1191-1266) and
_extract_block_diagonal_weights (patch/_conversion.py:99-140).
"""
import itertools

import pytest

from oracle import layout as OL


def test_perm_l012_hand_derived():
    # std order [l0 m0 | l1 m-1 m0 m1 | l2 m-2 .. m2]; m-first: m=0 of each l,
    # then (+1,-1) of l=1, (+1,-1) of l=2, (+2,-2) of l=2
    assert OL.m_first_perm([0, 1, 2]) == [0, 2, 6, 3, 1, 7, 5, 8, 4]


def test_perm_duplicates_and_gaps():
    assert OL.m_first_perm([1, 1]) == [1, 4, 2, 0, 5, 3]
    assert OL.m_first_perm([0, 2]) == [0, 3, 4, 2, 5, 1]


@pytest.mark.parametrize("lin,lout,wd", [([0, 1, 2], [0, 1, 2], 19), ([0, 1], [0, 1, 2], 10),
                                         (list(range(7)), list(range(7)), 231)])
def test_weight_dim_values(lin, lout, wd):
    assert OL.weight_dim(lin, lout) == wd


@pytest.mark.parametrize("lin,lout", [([0], [0]), ([1, 2], [0, 1, 2]), ([0, 1, 1], [0, 1, 2]),
                                      ([2], [0, 1, 2]), ([1, 2, 2], [0, 1]), (list(range(7)), [3, 1])])
def test_blocks_cover_weights(lin, lout):
    """sum over blocks of n_in n_out (1 or 2) equals sum_pairs (2 min(l,l') + 1)."""
    blocks = OL.block_params(lin, lout)
    total = sum((1 if m == 0 else 2) * ni * no for (m, ni, no, *_r) in blocks)
    assert total == OL.weight_dim(lin, lout)
    # offsets are contiguous in block order
    for (a, b) in zip(blocks, blocks[1:]):
        k = 1 if a[0] == 0 else 2
        assert b[3] == a[3] + k * a[1] and b[4] == a[4] + k * a[2] and b[5] == a[5] + k * a[1] * a[2]


def test_blocks_c2_values():
    assert OL.block_params([0, 1, 2], [0, 1, 2]) == [(0, 3, 3, 0, 0, 0), (1, 2, 2, 3, 3, 9),
                                                    (2, 1, 1, 7, 7, 17)]


def test_slot_l_matches_perm():
    for lv in ([0, 1, 2], [1, 2, 2], [0, 2], list(range(5))):
        perm = OL.m_first_perm(lv)
        std_l = [l for l in lv for _ in range(2 * l + 1)]
        assert OL.slot_l(lv) == [std_l[p] for p in perm]
