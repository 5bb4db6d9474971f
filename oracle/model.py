"""Attention layer, transformer block and transformer stack (oracle, float64, CPU).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every function takes the module's parameters as a flat dict keyed by the
reference's ``state_dict`` names (float64 leaves, so torch autograd gives the
parameter gradients) plus a plain config dict, and restates:

* ``attention``    -- ``EquivariantAttention.forward`` (``flash_eq/layers/attention.py:271-314``):
  fused QK projection of the layer-normed node features, Q gathered at dst and K
  at src (``:298-304``), V = edgewise linear of ``x[src] (+ edge_features)``
  (``:307-310``), per-destination softmax with the optional ``-r/decay`` bias
  (``:92-141``), per-head weighting of V's channel groups (``:157-167``), sum
  pooling (``pooling.py:21-30``);
* ``block``        -- ``EquivariantTransformerBlock.forward`` (``transformer.py:213-254``):
  norm1 -> attention -> LayerScale residual (only when the in/out reprs match,
  ``:150-153``) -> norm2 -> mlp_up -> gating -> mlp_down -> LayerScale residual;
* ``transformer``  -- ``EquivariantTransformer.forward`` (``transformer.py:389-431``):
  edge vectors ``coords[src] - coords[dst]``, their norms, the Wigner bases of
  the in/hidden/out reprs, the per-layer P/Q selection (``:414-427``) and the
  final separable norm.  The bases come from ``oracle.wigner.basis``
  (``torch.linalg.matrix_exp`` in float64), so coordinate gradients flow
  through the matrix exponential exactly as in the reference.

Pinned by ``tests/test_oracle_model.py`` against outputs and gradients that the
reference's own modules wrote (``tests/golden/composed_vectors.npz``, made by
``tests/golden/make_golden.py`` with the reference's block-diagonal op replaced
by this oracle's, which is pinned independently).
"""
from __future__ import annotations

from typing import Dict, Optional, Sequence

import torch

from . import graphops as G
from . import wigner as W
from .layer import BlockDiag, equivariant_layer_norm, gating, separable_layer_norm
from .radial import radial_functions
from . import blockdiag as BD


def _sub(params: Dict[str, torch.Tensor], prefix: str) -> Dict[str, torch.Tensor]:
    n = len(prefix)
    return {k[n:]: v for k, v in params.items() if k.startswith(prefix)}


def _scalar_locs(lvals: Sequence[int]):
    offs, locs = 0, []
    for l in lvals:
        if int(l) == 0:
            locs.append(offs)
        offs += 2 * int(l) + 1
    return locs


def linear(f: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor], lvals) -> torch.Tensor:
    """EquivariantLinear (linear.py:242-268): ``weight`` (nreps*out, in) mixes the
    channels of every irrep with its own (out, in) block; the bias (out, nscalar)
    is added to the scalar components in ``find_scalar`` order."""
    nreps = len(lvals)
    w = weight.view(nreps, -1, weight.shape[-1])
    parts, o = [], 0
    for k, l in enumerate(lvals):
        n = 2 * int(l) + 1
        parts.append(torch.einsum("oc,...cd->...od", w[k], f[..., o:o + n]))
        o += n
    out = torch.cat(parts, -1)
    if bias is not None:
        locs = _scalar_locs(lvals)
        out = out.clone()
        out[..., locs] = out[..., locs] + bias
    return out


def edgewise(params: Dict[str, torch.Tensor], cfg: dict, x, P, Q, r) -> torch.Tensor:
    """EquivariantEdgewiseLinear.forward (linear.py:131-160) with the table of
    ``SeparableRadialNet.forward`` (radial.py:259-275): bmm(x, P) -> block
    mix -> bmm(., Q^T).  ``params``: the radial net's parameters."""
    if cfg.get("radial_fp32"):
        # the radial network in float32, as the reference's float32 forward runs
        # it (see oracle/layer.py: edgewise_linear)
        p32 = {k: v.float() for k, v in params.items()}
        F = radial_functions(p32, p32["bin_edges"], cfg["min"], cfg["max"], cfg["rank"],
                             cfg["wdim"]).to(params["channel_patterns"].dtype)
    else:
        F = radial_functions(params, params["bin_edges"], cfg["min"], cfg["max"], cfg["rank"], cfg["wdim"])
    if cfg.get("F_pinned") is not None:
        # the radial functions' values fixed to given ones (another
        # implementation's float32 evaluation), their derivative this network's
        F = cfg["F_pinned"].to(F.dtype) + (F - F.detach())
    T = torch.einsum("koi,bkw->boiw", params["channel_patterns"], F)
    if cfg["log"]:
        b = BD.Binning.log(cfg["num_bins"], cfg["min"], cfg["max"], cfg["sigma"])
    else:
        b = BD.Binning.linear(cfg["num_bins"], cfg["min"], cfg["max"], cfg["sigma"])
    f = torch.bmm(x, P)
    return torch.bmm(BlockDiag.apply(f, T, r, cfg["lin"], cfg["lout"], b), Q.mT)


def attention(params, cfg: dict, P, Qb, x, r, src, dst, num_nodes: int,
              edge_features=None) -> torch.Tensor:
    """EquivariantAttention.forward (attention.py:271-314); keys as its state_dict."""
    lv, mult, H = cfg["lin"], cfg["mult_in"], cfg["heads"]
    eps = cfg.get("eps", 1e-8)
    xn = equivariant_layer_norm(x, lv, params.get("norm_qk.lnorm.weight"),
                                params.get("norm_qk.lnorm.bias"), eps)
    qk = linear(xn, params["linear_qk.weight"], None, lv)
    E = src.shape[0]
    Q = qk[:, :mult][dst].reshape(E, H, -1)
    K = qk[:, mult:][src].reshape(E, H, -1)
    gathered = x[src]
    if edge_features is not None:
        gathered = gathered + edge_features
    V = edgewise(_sub(params, "linear_v.radial_weights."), cfg["v"], gathered, P, Qb, r)
    logits = G.edge_logits(Q, K, params["attention.log_scale"], r, cfg.get("decay"))
    attn = G.neighbour_softmax(logits, dst, num_nodes)
    return G.pool_sum(G.apply_heads(V, attn), dst, num_nodes)


def block(params, cfg: dict, P, Q, x, r, src, dst, num_nodes: int,
          edge_features=None) -> torch.Tensor:
    """EquivariantTransformerBlock.forward (transformer.py:213-254), gating MLP,
    no dropout / drop path (evaluation semantics)."""
    lin, lout, eps = cfg["lin"], cfg["lout"], cfg.get("eps", 1e-8)
    h = separable_layer_norm(x, lin, params.get("norm1.scalar_norm.weight"),
                             params.get("norm1.scalar_norm.bias"), params.get("norm1.higher_norm.weight"),
                             eps)
    a = attention(_sub(params, "attn."), cfg["attn"], P, Q, h, r, src, dst, num_nodes, edge_features)
    if cfg["residual"]:
        g = params.get("layer_scale_attn.gamma")
        x = x + (a * g if g is not None else a)
    else:
        x = a
    h = separable_layer_norm(x, lout, params.get("norm2.scalar_norm.weight"),
                             params.get("norm2.scalar_norm.bias"), params.get("norm2.higher_norm.weight"),
                             eps)
    u = linear(h, params["mlp_up.weight"], params.get("mlp_up.bias"), lout)
    if cfg.get("gating", True):
        u = gating(u, lout, params["mlp_act.linear.weight"], params["mlp_act.linear.bias"], eps)
    m = linear(u, params["mlp_down.weight"], params.get("mlp_down.bias"), lout)
    g = params.get("layer_scale_mlp.gamma")
    return x + (m * g if g is not None else m)


def transformer(params, cfg: dict, coords, x, src, dst, num_nodes: int,
                edge_inputs: dict = None) -> torch.Tensor:
    """EquivariantTransformer.forward (transformer.py:389-431).

    ``edge_inputs`` (optional, no coordinate gradient): the distances ``r`` and
    the bases ``m_in``, ``m_hid``, ``m_out`` given instead of formed from the
    coordinates (another implementation's float32 values, so that a comparison
    covers what the blocks compute from them)."""
    if edge_inputs is not None:
        dt = x.dtype
        r = edge_inputs["r"].to(dt)
        m_in, m_hid, m_out = (edge_inputs[k].to(dt) for k in ("m_in", "m_hid", "m_out"))
    else:
        vec = coords[src] - coords[dst]
        r = vec.norm(dim=-1)
        # (the bases are formed in float64; a float32 evaluation of the composition
        # rounds them, as the reference's float32 matrix_exp would)
        m_in = W.basis(cfg["lin"], vec).to(vec.dtype)
        m_hid = W.basis(cfg["lhid"], vec).to(vec.dtype)
        m_out = W.basis(cfg["lout"], vec).to(vec.dtype)
    L = cfg["num_layers"]
    for i in range(L):
        P = m_in if i == 0 else m_hid
        Q = m_out if i == L - 1 else m_hid
        x = block(_sub(params, f"layers.{i}."), cfg["layers"][i], P, Q, x, r, src, dst, num_nodes)
    lo = cfg["lout"]
    return separable_layer_norm(x, lo, params.get("final_norm.scalar_norm.weight"),
                                params.get("final_norm.scalar_norm.bias"),
                                params.get("final_norm.higher_norm.weight"), cfg.get("eps", 1e-8))


# ---- configs from module hyper-parameters --------------------------------------------------

def edgewise_cfg(lin, lout, cin, cout, num_bins=100, min_dist=0.0, max_dist=10.0, log=False,
                 sigma=0.1, rank=4, radial_fp32=False) -> dict:
    """``radial_fp32``: evaluate the radial network in float32 whatever the
    composition's dtype (linear bins extrapolate beyond max_dist and multiply
    its rounding by |t|; the reference's float32 forward has exactly that)."""
    from .layout import weight_dim
    return dict(lin=list(lin), lout=list(lout), cin=cin, cout=cout, num_bins=num_bins, min=min_dist,
                max=max_dist, log=log, sigma=sigma, rank=rank, wdim=weight_dim(lin, lout),
                radial_fp32=radial_fp32)


def attention_cfg(lin, lout, mult_in, mult_out, heads, decay=None, eps=1e-8, **ew) -> dict:
    """``eps``: the norms' epsilon, ``get_epsilon(dtype)`` in the reference
    (utils.py:19-27): 1e-8 for float32/float64 features, 1e-5 for float16/bfloat16."""
    return dict(lin=list(lin), mult_in=mult_in, heads=heads, decay=decay, eps=eps,
                v=edgewise_cfg(lin, lout, mult_in, mult_out, **ew))


def block_cfg(lin, lout, mult_in, mult_out, heads, decay=None, eps=1e-8, **ew) -> dict:
    return dict(lin=list(lin), lout=list(lout), eps=eps,
                residual=(list(lin) == list(lout) and mult_in == mult_out),
                attn=attention_cfg(lin, lout, mult_in, mult_out, heads, decay, eps, **ew))


def transformer_cfg(lin, lhid, lout, mult_in, mult_hid, mult_out, num_layers, heads, decay=None,
                    eps=1e-8, **ew) -> dict:
    layers = []
    for i in range(num_layers):
        a, ma = (lin, mult_in) if i == 0 else (lhid, mult_hid)
        b, mb = (lout, mult_out) if i == num_layers - 1 else (lhid, mult_hid)
        layers.append(block_cfg(a, b, ma, mb, heads, decay, eps, **ew))
    return dict(lin=list(lin), lhid=list(lhid), lout=list(lout), num_layers=num_layers, eps=eps,
                layers=layers)


def leaves(state: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """float64 copies of a state dict; floating tensors other than the fixed
    buffers become autograd leaves."""
    out = {}
    for k, v in state.items():
        t = torch.as_tensor(v)
        if t.dtype.is_floating_point:
            t = t.double().clone()
            if not k.endswith("bin_edges") and not k.endswith("frequencies"):
                t.requires_grad_(True)
        out[k] = t
    return out
