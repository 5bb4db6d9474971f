"""Oracle and drop-in API against vectors written by the reference's own modules.

``tests/golden/reference_vectors.npz`` comes from ``tests/golden/make_golden.py``,
which ran the reference's pure-torch ``WignerDBasis``/``WignerD``, its seeded
module constructors, ``SeparableRadialNet.forward``, the node-side modules,
``_neighbor_softmax`` and ``GraphPooling`` (float32, CPU).  These pin what no
closed form does: the exact frame convention of P/Q and the RNG consumption
order of every constructor.  The GPU half checks the HIP paths against the
same vectors.
"""
import os

import numpy as np
import pytest
import torch

import flash_eq as fe
from oracle import graphops as OG
from oracle import radial as OR
from oracle import wigner as OW

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))
WIGNER_KEYS = sorted(k for k in GOLD.files if k.startswith("wigner__") and k != "wigner__dirs")


def G(key: str) -> torch.Tensor:
    return torch.from_numpy(GOLD[key])


def lvals_of(key: str):
    return [int(x) for x in key.split("__")[1].split("_")]


def state_of(prefix: str) -> dict:
    p = prefix + "__sd__"
    return {k[len(p):]: torch.from_numpy(GOLD[k]) for k in GOLD.files if k.startswith(p)}


def assert_same_state(module: torch.nn.Module, prefix: str) -> None:
    ref = state_of(prefix)
    mine = module.state_dict()
    assert list(mine) == list(ref), "parameter/buffer names or registration order differ"
    for k, v in ref.items():
        assert mine[k].dtype == v.dtype and torch.equal(mine[k], v), k


# ---- oracle ------------------------------------------------------------------------
@pytest.mark.parametrize("key", WIGNER_KEYS)
def test_oracle_wigner_basis_matches_reference(key):
    """Float64 matrix_exp restatement vs the reference's float32 WignerDBasis (incl. zero,
    +-z and near -z directions): only the reference's float32 rounding separates them."""
    mine = OW.basis(lvals_of(key), G("wigner__dirs"))
    assert (mine - G(key).double()).abs().max() < 5e-6


def test_oracle_rot_matches_reference():
    ax, an = G("rot__axis"), G("rot__angle")
    assert (OW.rot([0, 1, 2], ax, an, True) - G("rot__cart").double()).abs().max() < 5e-6
    assert (OW.rot([0, 1, 2], ax, an, False) - G("rot__sph").double()).abs().max() < 5e-6


@pytest.mark.parametrize("prefix", ["ewlA", "ewlB"])
def test_oracle_radial_table_matches_reference(prefix):
    sd = state_of(prefix)
    params = {k.split("radial_weights.")[1]: v.double() for k, v in sd.items()
              if k.split("radial_weights.")[1] not in ("frequencies", "bin_edges")}
    be = sd["radial_weights.bin_edges"].double()
    ref = G(prefix + "__table").double()
    rank, wdim = 4, ref.shape[-1]
    lo, hi = (0.0, 10.0) if prefix == "ewlA" else (0.5, 8.0)
    T = OR.table(params, be, lo, hi, rank, wdim)
    assert (T - ref).abs().max() / ref.abs().max() < 1e-5


def test_oracle_softmax_and_pooling_match_reference():
    dst, logits = G("softmax__dst"), G("softmax__logits").double()
    y = OG.neighbour_softmax(logits, dst, 9)
    assert (y - G("softmax__y").double()).abs().max() < 1e-6
    x, d = G("pool__x").double(), G("softmax__dst")
    assert (OG.pool_sum(x, d, 9) - G("pool__sum").double()).abs().max() < 1e-5
    assert (OG.pool_mean(x, d, 9) - G("pool__mean").double()).abs().max() < 1e-5
    assert (OG.pool_max(x, d, 9) - G("pool__max").double()).abs().max() < 1e-6


# ---- drop-in API, host side ------------------------------------------------------
def test_seeded_edgewise_linear_matches_reference_bitwise():
    torch.manual_seed(0)
    a = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1], 4), fe.Repr([0, 1, 2], 3), num_bins=10)
    assert_same_state(a, "ewlA")
    assert torch.equal(a.radial_weights().detach(), G("ewlA__table"))
    torch.manual_seed(1)
    b = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1, 2], 8), fe.Repr([0, 1, 2], 8), num_bins=20,
                                     log_bins=True, min_dist=0.5, max_dist=8.0)
    assert_same_state(b, "ewlB")
    assert torch.equal(b.radial_weights().detach(), G("ewlB__table"))
    assert np.allclose(np.array(b.radial_weights.binning_params(), dtype=np.float64),
                       GOLD["ewlB__binning"], rtol=0, atol=0)


def test_seeded_attention_matches_reference_bitwise():
    torch.manual_seed(3)
    att = fe.EquivariantAttention(fe.Repr([0, 1, 2], 8), fe.Repr([0, 1, 2], 8), num_heads=2,
                                  num_bins=10)
    assert_same_state(att, "attn")


@pytest.mark.parametrize("name,ctor", [
    ("elin", lambda rp: fe.EquivariantLinear(rp, fe.Repr([0, 1, 2], 5))),
    ("eln", lambda rp: fe.EquivariantLayerNorm(rp)),
    ("sln", lambda rp: fe.SeparableEquivariantLayerNorm(rp)),
    ("gate", lambda rp: fe.EquivariantGating(rp)),
])
def test_node_side_modules_match_reference(name, ctor):
    torch.manual_seed(4)
    m = ctor(fe.Repr([0, 1, 2], 6))
    assert_same_state(m, name)
    y = m(G("node__x"))
    ref = G(name + "__y")
    assert (y.detach() - ref).abs().max() <= 2e-6 * max(1.0, ref.abs().max().item())


def test_repnorm_matches_reference():
    y = fe.RepNorm(fe.Repr([0, 1, 2], 6))(G("node__x"))
    assert (y - G("repnorm__y")).abs().max() < 1e-6


# ---- HIP paths -----------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("key", WIGNER_KEYS)
def test_gpu_wigner_basis_matches_reference(dev, key):
    (M,) = fe.WignerDBasis([fe.Repr(lvals_of(key), 1)]).to(dev)(G("wigner__dirs").to(dev))
    assert (M.cpu().double() - G(key).double()).abs().max() < 5e-6


@pytest.mark.gpu
def test_gpu_wigner_basis_multi_matches_reference(dev):
    reps = [fe.Repr([0, 1], 2), fe.Repr([0, 1, 2], 3), fe.Repr([0, 1], 5), fe.Repr([0], 1)]
    outs = fe.WignerDBasis(reps).to(dev)(G("wigner__dirs").to(dev))
    for i, M in enumerate(outs):
        assert (M.cpu().double() - G(f"wigner_multi__{i}").double()).abs().max() < 5e-6


@pytest.mark.gpu
def test_gpu_softmax_and_pooling_match_reference(dev):
    dst, src = G("softmax__dst"), G("pool__src")
    graph = fe.Graph(src.to(dev), dst.to(dev), 9)
    E, H = G("softmax__logits").shape
    # logits = scale * <Q, K>: Q carries the logit, K = 1, log_scale = 0
    Q = G("softmax__logits").reshape(E, H, 1).to(dev)
    K = torch.ones(E, H, 1, device=dev)
    att = fe.EquivariantEdgeAttention(num_heads=H, qk_dim=1).to(dev)
    with torch.no_grad():
        att.log_scale.zero_()
        w = att.attention_weights(Q, K, graph)
    assert (w.cpu().double() - G("softmax__y").double()).abs().max() < 1e-6
    x = G("pool__x").to(dev)
    for red in ("sum", "mean", "max"):
        y = fe.GraphPooling(red)(x, graph)
        assert (y.cpu().double() - G(f"pool__{red}").double()).abs().max() < 1e-5, red
