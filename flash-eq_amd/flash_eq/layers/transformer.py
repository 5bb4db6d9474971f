"""Equivariant transformer block and stack (drop-in for ``flash_eq/layers/transformer.py``).

Host orchestration in PyTorch; the per-edge work inside runs the HIP kernels
(WignerDBasis, fused edgewise linear, edge softmax, attention pooling).
bfloat16/float16 blocks and models compute in float32 inside (``_precision``).
Module creation order follows ``transformer.py:143-211, 329-387``.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..graph import Graph
from ..representations import Repr, WignerDBasis
from ..ops import FanOutFn, ResidualScaleCmFn, ResidualScaleFn, ScaleFn
from .attention import EquivariantAttention
from .gating import EquivariantGating
from .linear import EquivariantLinear
from .norm import SeparableEquivariantLayerNorm
from ._precision import half_dtype, run_float32


class LayerScale(nn.Module):
    """x * gamma with a learnable scalar gamma (CaiT)."""

    def __init__(self, init_value: float = 1e-4) -> None:
        super().__init__()
        self.gamma = nn.Parameter(torch.tensor(init_value))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda and x.dtype == self.gamma.dtype == torch.float32:
            return ScaleFn.apply(x, self.gamma)   # gradient of gamma as one dot product
        return x * self.gamma


def _residual(x: torch.Tensor, y: torch.Tensor, scale: nn.Module, drop_path: nn.Module) -> torch.Tensor:
    """x + drop_path(scale(y)) (transformer.py:245, :252 of the reference).  With a
    LayerScale and no drop path on float32 GPU tables it is one pass
    (ops.ResidualScaleFn: the sum, the scaling and their gradients fused)."""
    if (isinstance(scale, LayerScale) and isinstance(drop_path, nn.Identity) and x.is_cuda
            and x.dtype == y.dtype == scale.gamma.dtype == torch.float32 and x.shape == y.shape
            and scale.gamma.device == x.device):
        return ResidualScaleFn.apply(x, y, scale.gamma)
    return x + drop_path(scale(y))


class DropPath(nn.Module):
    """Stochastic depth with one keep/drop decision per forward pass."""

    def __init__(self, drop_prob: float = 0.0) -> None:
        super().__init__()
        self.drop_prob = drop_prob

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.drop_prob == 0.0 or not self.training:
            return x
        if torch.rand(1, device=x.device).item() < self.drop_prob:
            return torch.zeros_like(x)
        return x / (1 - self.drop_prob)


class EquivariantTransformerBlock(nn.Module):
    """norm -> attention (-> residual when reprs match) -> norm -> gated MLP -> residual."""

    def __init__(self, in_repr: Repr, out_repr: Repr, num_heads: int = 1, num_bins: int = 100,
                 rank: int = 4, hidden_dim: int = 64, min_dist: float = 0.0,
                 max_dist: float = 10.0, log_bins: bool = False, mlp_ratio: int = 2,
                 dropout: float = 0.0, drop_path: float = 0.0,
                 layer_scale_init: float | None = 1e-4, use_gating: bool = True,
                 use_s2_activation: bool = False, s2_precision: int = 47,
                 distance_decay_scale: float | None = None) -> None:
        super().__init__()
        if use_s2_activation:
            raise NotImplementedError(
                "use_s2_activation=True (S2 grid activation) is not part of the MI355X build")
        self.in_repr = in_repr
        self.out_repr = out_repr
        self.use_s2_activation = use_s2_activation
        self._use_attn_residual = (torch.equal(in_repr.lvals, out_repr.lvals)
                                   and in_repr.mult == out_repr.mult)
        self.norm1 = SeparableEquivariantLayerNorm(in_repr)
        self.attn = EquivariantAttention(
            in_repr=in_repr, out_repr=out_repr, num_heads=num_heads, num_bins=num_bins, rank=rank,
            hidden_dim=hidden_dim, min_dist=min_dist, max_dist=max_dist, log_bins=log_bins,
            dropout=dropout, reduce="sum", distance_decay_scale=distance_decay_scale)
        self.norm2 = SeparableEquivariantLayerNorm(out_repr)
        hidden = Repr(lvals=out_repr.lvals, mult=out_repr.mult * mlp_ratio)
        self.mlp_up = EquivariantLinear(out_repr, hidden, bias=True)
        self.mlp_act: nn.Module = EquivariantGating(hidden) if use_gating else nn.Identity()
        self.mlp_down = EquivariantLinear(hidden, out_repr, bias=True)
        if layer_scale_init is not None and self._use_attn_residual:
            self.layer_scale_attn: nn.Module = LayerScale(layer_scale_init)
        else:
            self.layer_scale_attn = nn.Identity()
        self.layer_scale_mlp: nn.Module = (LayerScale(layer_scale_init)
                                           if layer_scale_init is not None else nn.Identity())
        self.drop_path: nn.Module = DropPath(drop_path) if drop_path > 0.0 else nn.Identity()

    def forward(self, P: torch.Tensor, Q: torch.Tensor, node_features: torch.Tensor,
                distances: torch.Tensor, graph: Graph,
                edge_features: torch.Tensor | None = None) -> torch.Tensor:
        half = half_dtype(node_features)
        if half is not None:
            return run_float32(self, half, (P, Q, node_features, distances, graph),
                               dict(edge_features=edge_features))
        # With the residual connection, the norm also returns the features for
        # it (forward_pair): the residual's gradient is then added inside the
        # norm's backward kernel instead of by autograd in a separate pass.
        if self._use_attn_residual and self.norm1.cm_ok(node_features):
            h, nf = self.norm1.forward_pair(node_features)
        else:
            h, nf = self.norm1(node_features), node_features
        attn_out = self.attn(P, Q, h, distances, graph, edge_features=edge_features)
        if self._use_attn_residual:
            x = _residual(nf, attn_out, self.layer_scale_attn, self.drop_path)
        else:
            x = attn_out
        if (isinstance(self.mlp_act, EquivariantGating) and self.mlp_act.kernels_ok(x)
                and self.mlp_up.fused_ok(x) and self.mlp_down.fused_ok(x)):
            # the MLP runs component-major (dim, N, c) from the norm's output to
            # the residual: the norm writes that layout, the linear maps and the
            # gating keep it, and the residual sum reads it (no transposes)
            cm = (self.norm2.cm_ok(x) and x.dim() == 3 and isinstance(self.layer_scale_mlp, LayerScale)
                  and isinstance(self.drop_path, nn.Identity)
                  and self.layer_scale_mlp.gamma.dtype == torch.float32)
            h, xr = self.norm2.forward_pair(x, cm) if self.norm2.cm_ok(x) else (self.norm2(x), x)
            t = self.mlp_act.forward_cm(self.mlp_up.forward_layout(h, cm, True))
            if cm:
                return ResidualScaleCmFn.apply(xr, self.mlp_down.forward_layout(t, True, True),
                                               self.layer_scale_mlp.gamma)
            mlp_out = self.mlp_down.forward_layout(t, True, False).view(*x.shape[:-2], self.out_repr.mult,
                                                                       x.shape[-1])
            return _residual(xr, mlp_out, self.layer_scale_mlp, self.drop_path)
        mlp_out = self.mlp_down(self.mlp_act(self.mlp_up(self.norm2(x))))
        return _residual(x, mlp_out, self.layer_scale_mlp, self.drop_path)

    def extra_repr(self) -> str:
        return (f"in_repr={self.in_repr}, out_repr={self.out_repr}, "
                f"attn_residual={self._use_attn_residual}")


class EquivariantTransformer(nn.Module):
    """Stack of blocks: in -> hidden -> ... -> hidden -> out, basis computed from coordinates."""

    def __init__(self, in_repr: Repr, hidden_repr: Repr, out_repr: Repr, num_layers: int = 6,
                 num_heads: int = 1, num_bins: int = 100, rank: int = 4, hidden_dim: int = 64,
                 min_dist: float = 0.0, max_dist: float = 10.0, log_bins: bool = False,
                 mlp_ratio: int = 2, dropout: float = 0.0, drop_path: float = 0.0,
                 layer_scale_init: float | None = 1e-4, use_s2_activation: bool = False,
                 s2_precision: int = 47, distance_decay_scale: float | None = None) -> None:
        super().__init__()
        self.in_repr = in_repr
        self.hidden_repr = hidden_repr
        self.out_repr = out_repr
        self.num_layers = num_layers
        self.distance_decay_scale = distance_decay_scale
        self._basis_reprs = [in_repr, hidden_repr, out_repr]
        self.basis = WignerDBasis(self._basis_reprs)
        rates = [x.item() for x in torch.linspace(0, drop_path, num_layers)]
        self.layers = nn.ModuleList()
        for i in range(num_layers):
            layer_in = in_repr if i == 0 else hidden_repr
            layer_out = out_repr if i == num_layers - 1 else hidden_repr
            self.layers.append(EquivariantTransformerBlock(
                in_repr=layer_in, out_repr=layer_out, num_heads=num_heads, num_bins=num_bins,
                rank=rank, hidden_dim=hidden_dim, min_dist=min_dist, max_dist=max_dist,
                log_bins=log_bins, mlp_ratio=mlp_ratio, dropout=dropout, drop_path=rates[i],
                layer_scale_init=layer_scale_init, use_s2_activation=use_s2_activation,
                s2_precision=s2_precision, distance_decay_scale=distance_decay_scale))
        self.final_norm = SeparableEquivariantLayerNorm(out_repr)

    def forward(self, coordinates: torch.Tensor, node_features: torch.Tensor,
                graph: Graph) -> torch.Tensor:
        half = half_dtype(node_features)
        if half is not None:
            return run_float32(self, half, (coordinates, node_features, graph), {})
        # src - dst, as transformer.py:406.  In float32 through the graph's CSR
        # gathers: their backward (the coordinate gradient) is a fixed-order
        # segmented sum, where torch's indexing backward sorts the indices
        # (a radix sort that must not be captured in a HIP graph above 2^20 keys)
        if coordinates.dtype == torch.float32 and coordinates.is_cuda:
            vec = graph.gather_src(coordinates) - graph.gather_dst(coordinates)
        else:
            vec = coordinates[graph.src] - coordinates[graph.dst]
        distances = vec.norm(dim=-1)
        m_in, m_hidden, m_out = self.basis(vec)
        x = node_features
        uses = [(m_in if i == 0 else m_hidden, m_out if i == self.num_layers - 1 else m_hidden)
                for i in range(self.num_layers)]
        if m_hidden.requires_grad and m_hidden.is_cuda and m_hidden.dtype == torch.float32:
            # the hidden bases feed every layer (as P and as Q): their gradients
            # are summed in one pass (FanOutFn) rather than pairwise by autograd
            k = sum((P is m_hidden) + (Q is m_hidden) for P, Q in uses)
            if 1 < k <= 16:
                views = iter(FanOutFn.apply(m_hidden, k))
                uses = [(next(views) if P is m_hidden else P, next(views) if Q is m_hidden else Q)
                        for P, Q in uses]
        for layer, (P, Q) in zip(self.layers, uses):
            x = layer(P, Q, x, distances, graph)
        return self.final_norm(x)

    def extra_repr(self) -> str:
        return (f"in_repr={self.in_repr}, hidden_repr={self.hidden_repr}, "
                f"out_repr={self.out_repr}, num_layers={self.num_layers}")
