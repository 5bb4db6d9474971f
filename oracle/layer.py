"""Layer compositions on the oracle pieces (float64, CPU).

``edgewise_linear`` restates ``EquivariantEdgewiseLinear.forward``
(``flash_eq/layers/linear.py:131-160``): ``bmm(x, P)`` -> block-diagonal mix
with the table ``rw()`` -> ``bmm(., Q^T)``.  The block-diagonal step is an
autograd Function whose backward is the oracle's explicit backward (with the
reference's distance-gradient formulas), everything else is torch autograd.

``attention`` restates ``EquivariantAttention.forward`` (attention.py:294-314)
given its sub-results.
"""
from __future__ import annotations

import torch

from . import blockdiag as BD
from . import graphops as G
from . import radial as R


class BlockDiag(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, table, r, lin, lout, b):
        ctx.save_for_backward(x, table, r)
        ctx.meta = (lin, lout, b)
        return BD.forward(x, table, r, lin, lout, b)

    @staticmethod
    def backward(ctx, gy):
        x, table, r = ctx.saved_tensors
        lin, lout, b = ctx.meta
        gx, gt, gr = BD.backward(gy.contiguous(), x, table, r, lin, lout, b,
                                 need_dr=ctx.needs_input_grad[2])
        return gx, gt, (gr if ctx.needs_input_grad[2] else None), None, None, None


def edgewise_linear(x, P, Q, r, params: dict, cfg: dict) -> torch.Tensor:
    """cfg: lin, lout, num_bins, min, max, log, sigma, rank, wdim, bin_edges (float64 tensor).

    ``cfg["radial_fp32"]`` evaluates the radial MLP in float32 (as the
    reference's float32 forward does) before promoting the table to float64:
    beyond max_dist the unclamped interpolation multiplies the MLP's rounding
    by |t|, so float32-vs-float64 MLP evaluation alone differs by ~|t| 1e-7.
    """
    if cfg.get("radial_fp32"):
        p32 = {k: v.float() for k, v in params.items()}
        F = R.radial_functions(p32, cfg["bin_edges"].float(), cfg["min"], cfg["max"],
                               cfg["rank"], cfg["wdim"]).double()
        T = torch.einsum("koi,bkw->boiw", params["channel_patterns"], F)
    else:
        T = R.table(params, cfg["bin_edges"], cfg["min"], cfg["max"], cfg["rank"], cfg["wdim"])
    if cfg["log"]:
        b = BD.Binning.log(cfg["num_bins"], cfg["min"], cfg["max"], cfg["sigma"])
    else:
        b = BD.Binning.linear(cfg["num_bins"], cfg["min"], cfg["max"], cfg["sigma"])
    f = torch.bmm(x, P)
    out = BlockDiag.apply(f, T, r, cfg["lin"], cfg["lout"], b)
    return torch.bmm(out, Q.mT)


def module_cfg(layer) -> dict:
    """Oracle config and float64 parameter copies from a product EquivariantEdgewiseLinear."""
    rw = layer.radial_weights
    params = {k: v.detach().double().cpu().clone().requires_grad_(True)
              for k, v in rw.named_parameters()}
    # the module's frequency buffer: k pi rounded to float32 (radial.py:206-209),
    # which a float64 module keeps (.double() converts the rounded values)
    params["frequencies"] = rw.frequencies.detach().double().cpu()
    cfg = dict(lin=[int(l) for l in layer.in_repr.lvals], lout=[int(l) for l in layer.out_repr.lvals],
               num_bins=rw.num_bins, min=rw.min_val, max=rw.max_val, log=rw.log,
               sigma=layer.solid_harmonic_scale, rank=rw.rank, wdim=rw.weight_dim,
               bin_edges=rw.bin_edges.detach().double().cpu())
    return params, cfg


def rep_norms(f: torch.Tensor, lvals, eps: float) -> torch.Tensor:
    """sqrt(sum over each irrep's components of f^2 + eps) -> (..., nreps) (norm.py:60-72)."""
    out, o = [], 0
    for l in lvals:
        n = 2 * int(l) + 1
        out.append(((f[..., o:o + n] ** 2).sum(-1) + eps).sqrt())
        o += n
    return torch.stack(out, -1)


def equivariant_layer_norm(f, lvals, ln_weight, ln_bias, eps: float = 1e-8):
    """EquivariantLayerNorm (norm.py:148-174): LayerNorm over channels of the irrep norms."""
    norms = rep_norms(f, lvals, eps)                         # (..., mult, nreps)
    idx = torch.tensor([k for k, l in enumerate(lvals) for _ in range(2 * int(l) + 1)])
    if ln_weight is None:                                    # mult = 1: no LayerNorm (norm.py:160-163)
        return f * (1.0 / (norms + eps))[..., idx]
    t = norms.transpose(-2, -1)
    mu = t.mean(-1, keepdim=True)
    var = t.var(-1, unbiased=False, keepdim=True)
    ln = ((t - mu) / torch.sqrt(var + 1e-5) * ln_weight + ln_bias).transpose(-2, -1)
    scale = ln / (norms + eps)
    return f * scale[..., idx]


def equivariant_linear(f, weight, lvals):
    """EquivariantLinear without bias (linear.py:242-268): per-irrep channel mix."""
    nreps = len(lvals)
    w = weight.view(nreps, -1, weight.shape[-1])
    parts, o = [], 0
    for k, l in enumerate(lvals):
        n = 2 * int(l) + 1
        parts.append(torch.einsum("oc,...cd->...od", w[k], f[..., o:o + n]))
        o += n
    return torch.cat(parts, -1)


def _component_irreps(lvals):
    return torch.tensor([k for k, l in enumerate(lvals) for _ in range(2 * int(l) + 1)])


def separable_layer_norm(f, lvals, s_weight, s_bias, h_weight, eps: float = 1e-8):
    """SeparableEquivariantLayerNorm (norm.py:177-246), in the reference's index
    form: LayerNorm over channels of the l = 0 components (norm.py:89-93), one
    RMS over every channel and l > 0 component with a per-channel weight
    (norm.py:109-112), written back at their component positions."""
    offs = [0]
    for l in lvals:
        offs.append(offs[-1] + 2 * int(l) + 1)
    locs = [offs[k] for k, l in enumerate(lvals) if int(l) == 0]
    higher = torch.ones(offs[-1], dtype=torch.bool)
    higher[locs] = False
    out = f.clone()
    if locs:
        x = f[..., locs]
        mu = x.mean(-2, keepdim=True)
        sd = x.std(-2, keepdim=True, unbiased=False)
        out[..., locs] = (x - mu) / (sd + eps) * s_weight + s_bias
    if bool(higher.any()):
        x = f[..., higher]
        rms = torch.sqrt((x ** 2).mean(dim=(-2, -1), keepdim=True) + eps)
        out[..., higher] = x * (h_weight[..., None] / rms)
    return out


def gating(f, lvals, weight, bias, eps: float = 1e-8):
    """EquivariantGating (gating.py:54-76): sigmoid(Linear(flattened irrep norms))
    broadcast over each irrep's components."""
    norms = rep_norms(f, lvals, eps)                         # (..., mult, nreps)
    lead = norms.shape[:-2]
    g = torch.sigmoid(norms.flatten(-2, -1) @ weight.t() + bias).view(*lead, *norms.shape[-2:])
    return f * g[..., _component_irreps(lvals)]


def attention_layer(layer, P, Qb, x, r, src, dst, num_nodes):
    """EquivariantAttention.forward (attention.py:294-314) in float64 from a product layer's weights.

    Returns (out, params) where params are the float64 leaves (for gradients).
    """
    lv = [int(l) for l in layer.in_repr.lvals]
    mult, H = layer.in_repr.mult, layer.num_heads
    ln_w = layer.norm_qk.lnorm.weight.detach().double().cpu().requires_grad_(True)
    ln_b = layer.norm_qk.lnorm.bias.detach().double().cpu().requires_grad_(True)
    wqk = layer.linear_qk.weight.detach().double().cpu().requires_grad_(True)
    ls = layer.attention.log_scale.detach().double().cpu().requires_grad_(True)
    vparams, vcfg = module_cfg(layer.linear_v)
    qk = equivariant_linear(equivariant_layer_norm(x, lv, ln_w, ln_b), wqk, lv)
    E = src.shape[0]
    Q = qk[:, :mult][dst].reshape(E, H, -1)
    K = qk[:, mult:][src].reshape(E, H, -1)
    V = edgewise_linear(x[src], P, Qb, r, vparams, vcfg)
    attn = G.neighbour_softmax(G.edge_logits(Q, K, ls), dst, num_nodes)
    out = G.pool_sum(G.apply_heads(V, attn), dst, num_nodes)
    params = {"norm_qk.lnorm.weight": ln_w, "norm_qk.lnorm.bias": ln_b,
              "linear_qk.weight": wqk, "attention.log_scale": ls}
    params.update({"linear_v.radial_weights." + k: v for k, v in vparams.items() if v.requires_grad})
    return out, params
