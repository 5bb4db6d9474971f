"""Pins of the graph-op and radial oracles (oracle/graphops.py, oracle/radial.py)."""
import json
import os

import pytest
import torch

from oracle import graphops as G
from oracle import radial as R

KAT = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "pooling_kat.json")))


@pytest.mark.parametrize("name,fn", [("sum", G.pool_sum), ("mean", G.pool_mean), ("max", G.pool_max)])
def test_pooling_known_answers(name, fn):
    c = KAT[name]
    out = fn(torch.tensor(c["x"], dtype=torch.float64), torch.tensor(c["dst"]), c["num_nodes"])
    assert torch.equal(out, torch.tensor(c["expected"], dtype=torch.float64))


def test_pooling_single_and_all_to_one():
    c = KAT["single"]
    out = G.pool_sum(torch.tensor(c["x"], dtype=torch.float64), torch.tensor(c["dst"]), c["num_nodes"])
    assert torch.equal(out, torch.tensor(c["expected"], dtype=torch.float64))
    a = KAT["all_to_one"]
    x = torch.ones(a["num_edges"], *a["row"], dtype=torch.float64)
    out = G.pool_sum(x, torch.zeros(a["num_edges"], dtype=torch.long), a["num_nodes"])
    assert (out[0] == a["node0_value"]).all() and (out[1:] == 0).all()


def test_pool_sum_loop_matches_vectorised():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(300, 4, 9, generator=g, dtype=torch.float64)
    dst = torch.randint(0, 37, (300,), generator=g)
    assert (G.pool_sum(x, dst, 40) - G.pool_sum_loop(x, dst, 40)).abs().max() < 1e-12


def test_softmax_sums_to_one_and_loop_agrees():
    g = torch.Generator().manual_seed(1)
    E, H, N = 400, 4, 50
    lg = torch.randn(E, H, generator=g, dtype=torch.float64) * 3
    dst = torch.randint(0, N, (E,), generator=g)
    a = G.neighbour_softmax(lg, dst, N)
    b = G.neighbour_softmax_loop(lg, dst, N)
    assert (a - b).abs().max() < 1e-14
    sums = torch.zeros(N, H, dtype=torch.float64).index_add(0, dst, a)
    has = torch.zeros(N, dtype=torch.bool)
    has[dst] = True
    assert (sums[has] - 1).abs().max() < 1e-7          # 1/(1+1e-8/S) with S >= 1
    # shift invariance per destination
    shift = torch.randn(N, H, generator=g, dtype=torch.float64)[dst]
    assert (G.neighbour_softmax(lg + shift, dst, N) - a).abs().max() < 1e-12


def test_envelope_closed_form():
    r = torch.tensor([0.0, 10.0, 5.0], dtype=torch.float64)
    f = R.sinusoidal_basis(r, 0.0, 10.0)
    k = torch.arange(1, 17, dtype=torch.float64) * torch.pi
    assert torch.allclose(f[0], torch.cat([torch.zeros(16, dtype=torch.float64),
                                           torch.ones(16, dtype=torch.float64)]))
    assert f[1].abs().max() < 1e-12                      # e(1) = 0
    assert torch.allclose(f[2], 0.5 * torch.cat([torch.sin(0.5 * k), torch.cos(0.5 * k)]))  # e(1/2) = 1/2
    # e'(0) = e'(1) = 0: first differences vanish to second order
    h = 1e-5
    e = lambda x: 1 - 10 * x ** 3 + 15 * x ** 4 - 6 * x ** 5
    assert abs((e(h) - e(0)) / h) < 1e-8 and abs((e(1.0) - e(1.0 - h)) / h) < 1e-8


def test_table_einsum_matches_loop():
    g = torch.Generator().manual_seed(2)
    C = torch.randn(3, 4, 5, generator=g, dtype=torch.float64)
    F = torch.randn(6, 3, 7, generator=g, dtype=torch.float64)
    T = torch.einsum("koi,bkw->boiw", C, F)
    Tl = sum(C[k][None, :, :, None] * F[:, k][:, None, None, :] for k in range(3))
    assert (T - Tl).abs().max() < 1e-12
