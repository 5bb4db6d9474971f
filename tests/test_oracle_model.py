"""Pins the oracle's composed layers to the reference's own outputs and gradients.

``tests/golden/composed_vectors.npz`` holds, for small seeded graphs, what the
reference's EquivariantEdgewiseLinear, EquivariantAttention,
EquivariantTransformerBlock and EquivariantTransformer computed in float64
(``make_golden.py: composed``): the output, and the gradients of sum(y * W)
for a fixed random W with respect to the inputs (features, distances, bases,
coordinates, edge features) and every parameter.  The oracle's restatements
(``oracle/model.py``), run on the same float64 parameters and inputs, must
match to 1e-9 relative: a Q/K swap, a wrong decay sign, a missing residual or
LayerScale, a wrong per-layer P/Q choice or a lost coordinate gradient path
all move these numbers by far more.
"""
import os

import numpy as np
import pytest
import torch

from oracle import model as OM

GOLD = os.path.join(os.path.dirname(__file__), "golden", "composed_vectors.npz")
TOL = 1e-9


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def _state(gold, name):
    pre = f"{name}__sd__"
    return {k[len(pre):]: torch.from_numpy(gold[k]) for k in gold.files if k.startswith(pre)}


def _inputs(gold, name):
    pre = f"{name}__in__"
    out = {}
    for k in gold.files:
        if k.startswith(pre):
            t = torch.from_numpy(gold[k])
            if t.dtype.is_floating_point:
                t = t.clone().requires_grad_(True)
            out[k[len(pre):]] = t
    return out


def _rel(a, b):
    a, b = a.detach().double(), torch.as_tensor(b).double()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


def _check(gold, name, y, params, inputs):
    assert _rel(y, gold[f"{name}__y"]) < TOL
    (y * torch.from_numpy(gold[f"{name}__lossw"])).sum().backward()
    checked = 0
    for k, t in inputs.items():
        key = f"{name}__grad__{k}"
        if key in gold.files:
            assert t.grad is not None, k
            assert _rel(t.grad, gold[key]) < TOL, (k, _rel(t.grad, gold[key]))
            checked += 1
    pre = f"{name}__pgrad__"
    for k in gold.files:
        if k.startswith(pre):
            p = params[k[len(pre):]]
            assert p.grad is not None, k
            assert _rel(p.grad, gold[k]) < TOL, (k, _rel(p.grad, gold[k]))
            checked += 1
    return checked


@pytest.mark.parametrize("name,lin,lout,cin,cout,kw", [
    ("ewl", [0, 1], [0, 1, 2], 4, 3, dict(num_bins=10)),
    ("ewlL", [0, 1, 2], [0, 1, 2], 3, 3, dict(num_bins=8, log=True, min_dist=0.5, max_dist=8.0)),
])
def test_edgewise_linear_matches_reference(gold, name, lin, lout, cin, cout, kw):
    params = OM.leaves({k.replace("radial_weights.", ""): v for k, v in _state(gold, name).items()})
    cfg = OM.edgewise_cfg(lin, lout, cin, cout, **kw)
    I = _inputs(gold, name)
    y = OM.edgewise(params, cfg, I["x"], I["P"], I["Q"], I["r"])
    params = {"radial_weights." + k: v for k, v in params.items()}
    assert _check(gold, name, y, params, I) == 4 + 7      # x, P, Q, r + 7 parameters


@pytest.mark.parametrize("name,with_ef", [("att", False), ("attE", True)])
def test_attention_matches_reference(gold, name, with_ef):
    params = OM.leaves(_state(gold, name))
    cfg = OM.attention_cfg([0, 1, 2], [0, 1, 2], 4, 4, heads=2, decay=3.0, num_bins=10)
    I = _inputs(gold, name)
    from oracle import wigner as W
    P = W.basis([0, 1, 2], I["dirs"].detach())
    y = OM.attention(params, cfg, P, P, I["x"], I["r"], I["src"], I["dst"], 9,
                     I["ef"] if with_ef else None)
    assert _check(gold, name, y, params, I) >= 2 + 11


def test_attention_decay_sign_and_qk_order_are_pinned(gold):
    """The golden output moves when the decay term flips sign or Q/K swap ends."""
    params = OM.leaves(_state(gold, "att"))
    cfg = OM.attention_cfg([0, 1, 2], [0, 1, 2], 4, 4, heads=2, decay=-3.0, num_bins=10)
    I = _inputs(gold, "att")
    from oracle import wigner as W
    P = W.basis([0, 1, 2], I["dirs"].detach())
    y = OM.attention(params, cfg, P, P, I["x"], I["r"], I["src"], I["dst"], 9)
    assert _rel(y, gold["att__y"]) > 1e-3
    cfg["decay"] = 3.0
    y = OM.attention(params, cfg, P, P, I["x"], I["r"], I["dst"], I["src"], 9)
    assert _rel(y, gold["att__y"]) > 1e-3


@pytest.mark.parametrize("name,lin,lout,cin,cout,decay", [
    ("blk", [0, 1, 2], [0, 1, 2], 4, 4, None),
    ("blkN", [0, 1], [0, 1, 2], 4, 6, 2.5),
])
def test_block_matches_reference(gold, name, lin, lout, cin, cout, decay):
    st = _state(gold, name)
    for k in ("layer_scale_attn.gamma", "layer_scale_mlp.gamma"):
        if k in st:
            st[k] = torch.tensor(0.6, dtype=torch.float32)      # as make_golden sets them
    params = OM.leaves(st)
    cfg = OM.block_cfg(lin, lout, cin, cout, heads=2, decay=decay, num_bins=10)
    assert cfg["residual"] == (name == "blk")
    I = _inputs(gold, name)
    from oracle import wigner as W
    P = W.basis(lin, I["dirs"].detach())
    Q = W.basis(lout, I["dirs"].detach())
    y = OM.block(params, cfg, P, Q, I["x"], I["r"], I["src"], I["dst"], 11)
    assert _check(gold, name, y, params, I) >= 2 + 20


def test_transformer_matches_reference_including_coordinate_gradient(gold):
    params = OM.leaves(_state(gold, "tfS"))
    cfg = OM.transformer_cfg([0, 1], [0, 1, 2], [0], 4, 4, 4, num_layers=3, heads=2, num_bins=10)
    I = _inputs(gold, "tfS")
    y = OM.transformer(params, cfg, I["coords"], I["x"], I["src"], I["dst"], 12)
    n = _check(gold, "tfS", y, params, I)
    assert I["coords"].grad is not None and n >= 2 + 60
    assert I["coords"].grad.abs().max() > 1e-6


def test_transformer_seeded_state_dict_names(gold):
    """The default-init transformer's state dict (seed 51) holds every key the
    oracle's transformer reads."""
    st = _state(gold, "tf")
    assert "layers.2.mlp_act.linear.weight" in st and "final_norm.scalar_norm.weight" in st
    assert "layers.0.attn.attention.log_scale" in st
    assert float(st["layers.1.layer_scale_mlp.gamma"]) == pytest.approx(1e-4)
