"""Seeded construction of the composed modules equals the reference's, bit for bit.

The reference's EquivariantEdgewiseLinear, EquivariantAttention,
EquivariantTransformerBlock and EquivariantTransformer were built under the
seeds recorded in ``tests/golden/make_golden.py: composed`` and their state
dicts stored in ``composed_vectors.npz``.  Building this package's modules
under the same seeds must give the same names, registration order, dtypes and
values: checkpoints load both ways and the RNG consumption order matches.
"""
import os

import numpy as np
import pytest
import torch

import flash_eq as fe

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "composed_vectors.npz"))
R = fe.Repr


def _state(name):
    pre = f"{name}__sd__"
    return {k[len(pre):]: torch.from_numpy(GOLD[k]) for k in GOLD.files if k.startswith(pre)}


def _same(module, name):
    ref = _state(name)
    mine = module.state_dict()
    assert list(mine) == list(ref), "parameter/buffer names or registration order differ"
    for k, v in ref.items():
        assert mine[k].dtype == v.dtype and torch.equal(mine[k], v), k


BUILDERS = {
    "ewl": (21, lambda: fe.EquivariantEdgewiseLinear(R([0, 1], 4), R([0, 1, 2], 3), num_bins=10,
                                                     hidden_dim=16)),
    "ewlL": (22, lambda: fe.EquivariantEdgewiseLinear(R([0, 1, 2], 3), R([0, 1, 2], 3), num_bins=8,
                                                      log_bins=True, min_dist=0.5, max_dist=8.0,
                                                      hidden_dim=16)),
    "att": (31, lambda: fe.EquivariantAttention(R([0, 1, 2], 4), R([0, 1, 2], 4), num_heads=2,
                                                num_bins=10, hidden_dim=16, distance_decay_scale=3.0)),
    "blk": (41, lambda: fe.EquivariantTransformerBlock(R([0, 1, 2], 4), R([0, 1, 2], 4), num_heads=2,
                                                       num_bins=10, hidden_dim=16)),
    "blkN": (42, lambda: fe.EquivariantTransformerBlock(R([0, 1], 4), R([0, 1, 2], 6), num_heads=2,
                                                        num_bins=10, hidden_dim=16,
                                                        distance_decay_scale=2.5)),
    "tf": (51, lambda: fe.EquivariantTransformer(R([0, 1], 4), R([0, 1, 2], 4), R([0], 4),
                                                 num_layers=3, num_heads=2, num_bins=10)),
    "tfS": (51, lambda: fe.EquivariantTransformer(R([0, 1], 4), R([0, 1, 2], 4), R([0], 4),
                                                  num_layers=3, num_heads=2, num_bins=10,
                                                  hidden_dim=16, layer_scale_init=0.6)),
}


@pytest.mark.parametrize("name", sorted(BUILDERS))
def test_seeded_state_dict_matches_reference(name):
    seed, build = BUILDERS[name]
    torch.manual_seed(seed)
    _same(build(), name)
