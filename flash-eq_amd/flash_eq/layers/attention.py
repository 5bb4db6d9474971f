"""Equivariant graph attention (drop-in for ``flash_eq/layers/attention.py``).

* logits and the per-destination softmax (``attention.py:92-141``) run in one
  HIP kernel over the node segments (``feq_attn_softmax_fwd``): max shift,
  exponentials, the ``+1e-8`` denominator, in CSR order without atomics;
  ``EquivariantAttention`` reads Q and K straight from the node table of its
  fused QK projection (the gathers of ``attention.py:298-304`` happen inside
  the kernels, so no (E, H, Dh) tensor is formed);
* ``EquivariantAttention`` fuses the head weighting of V with the sum pooling
  (``attention.py:143-167`` + ``pooling.py:21-30``) in ``feq_attn_pool_fwd``, so
  the weighted (E, mult, dim) tensor is never written;
* V comes from the fused ``EquivariantEdgewiseLinear``.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import _native as N
from ..graph import Graph
from ..ops import AttnPoolFn, EdgeSoftmaxFn, NodeSoftmaxFn
from ..representations import Repr
from .linear import EquivariantEdgewiseLinear, EquivariantLinear
from .norm import EquivariantLayerNorm
from .pooling import GraphPooling
from ._precision import half_dtype, run_float32


class EquivariantEdgeAttention(nn.Module):
    """Scaled dot-product attention over the edges that share a destination."""

    def __init__(self, num_heads: int, qk_dim: int, dropout: float = 0.0,
                 distance_decay_scale: float | None = None) -> None:
        super().__init__()
        self.num_heads = num_heads
        self.qk_dim = qk_dim
        self.distance_decay_scale = distance_decay_scale
        self.log_scale = nn.Parameter(torch.tensor(qk_dim ** -0.5).log())
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    @property
    def scale(self) -> torch.Tensor:
        return self.log_scale.exp()

    def attention_weights(self, Q: torch.Tensor, K: torch.Tensor, graph: Graph,
                          distances: torch.Tensor | None = None) -> torch.Tensor:
        """Softmax-normalised weights (E, H) after dropout."""
        N.require_cuda_tensor(Q, "Q")
        perm, offsets = graph.csr()
        decay = float(self.distance_decay_scale) if (
            self.distance_decay_scale is not None and distances is not None) else 0.0
        attn = EdgeSoftmaxFn.apply(Q, K, distances if decay > 0 else None, self.log_scale, decay,
                                   perm, offsets, graph.num_nodes)
        return self.dropout(attn)

    def node_attention_weights(self, qk: torch.Tensor, graph: Graph,
                               distances: torch.Tensor | None = None, cm: bool = False) -> torch.Tensor:
        """The same weights (E, H) with Q = qk[dst, :mult] and K = qk[src, mult:]
        read from the (N, 2 mult, dim) node table inside the kernels (``cm``: the
        component-major (dim, N, 2 mult) table)."""
        N.require_cuda_tensor(qk, "qk")
        perm, offsets = graph.csr()
        perm_s, offsets_s = graph.csr_src()
        decay = float(self.distance_decay_scale) if (
            self.distance_decay_scale is not None and distances is not None) else 0.0
        attn = NodeSoftmaxFn.apply(qk, distances if decay > 0 else None, self.log_scale, decay,
                                   self.num_heads, graph.src, graph.dst, perm, offsets, perm_s,
                                   offsets_s, graph.num_nodes, cm)
        return self.dropout(attn)

    def forward(self, Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, graph: Graph,
                distances: torch.Tensor | None = None) -> torch.Tensor:
        """Q, K (E, H, qk_dim); V (E, mult, dim) -> attention-weighted V (E, mult, dim)."""
        attn = self.attention_weights(Q, K, graph, distances)
        return self._apply_attention(V, attn)

    def _apply_attention(self, V: torch.Tensor, attn: torch.Tensor) -> torch.Tensor:
        E, mult, dim = V.shape
        if self.num_heads == 1:
            return V * attn.view(E, 1, 1)
        hd = mult // self.num_heads
        return (V.view(E, self.num_heads, hd, dim) * attn.view(E, self.num_heads, 1, 1)).view(E, mult, dim)

    def extra_repr(self) -> str:
        return f"num_heads={self.num_heads}, qk_dim={self.qk_dim}"


class EquivariantAttention(nn.Module):
    """Equivariant Q/K projections + edgewise V + neighbour softmax + pooling."""

    def __init__(self, in_repr: Repr, out_repr: Repr, num_heads: int = 1, num_bins: int = 100,
                 rank: int = 4, hidden_dim: int = 64, min_dist: float = 0.0,
                 max_dist: float = 10.0, log_bins: bool = False, dropout: float = 0.0,
                 reduce: str = "sum", distance_decay_scale: float | None = None) -> None:
        super().__init__()
        if in_repr.mult % num_heads != 0:
            raise ValueError(f"num_heads ({num_heads}) must divide in_repr.mult ({in_repr.mult})")
        if out_repr.mult % num_heads != 0:
            raise ValueError(f"num_heads ({num_heads}) must divide out_repr.mult ({out_repr.mult})")
        self.in_repr = in_repr
        self.out_repr = out_repr
        self.num_heads = num_heads
        # module creation order follows attention.py:241-269 (seeded init parity)
        self.norm_qk = EquivariantLayerNorm(in_repr)
        self.linear_qk = EquivariantLinear(in_repr, Repr(lvals=in_repr.lvals, mult=in_repr.mult * 2),
                                           bias=False)
        qk_dim = (in_repr.mult // num_heads) * in_repr.dim()
        self.attention = EquivariantEdgeAttention(num_heads=num_heads, qk_dim=qk_dim,
                                                  dropout=dropout,
                                                  distance_decay_scale=distance_decay_scale)
        self.linear_v = EquivariantEdgewiseLinear(in_repr=in_repr, out_repr=out_repr,
                                                  num_bins=num_bins, rank=rank,
                                                  hidden_dim=hidden_dim, min_dist=min_dist,
                                                  max_dist=max_dist, log_bins=log_bins)
        self.pool = GraphPooling(reduce=reduce)

    def forward(self, P: torch.Tensor, Q_basis: torch.Tensor, node_features: torch.Tensor,
                distances: torch.Tensor, graph: Graph,
                edge_features: torch.Tensor | None = None) -> torch.Tensor:
        """node_features (N, mult_in, dim_in) -> (N, mult_out, dim_out)."""
        half = half_dtype(node_features)
        if half is not None:
            return run_float32(self, half, (P, Q_basis, node_features, distances, graph),
                               dict(edge_features=edge_features))
        if (node_features.dim() == 3 and self.norm_qk.cm_ok(node_features)
                and self.linear_qk.fused_ok(node_features)):
            # the norm writes the component-major layout the projection reads;
            # the V projection's gradient of the features is added in the
            # norm's backward kernel (node_features becomes the norm's alias)
            # the attention kernels read the projection's component-major
            # (dim, N, 2 mult) table as it is written
            q_in, node_features = self.norm_qk.forward_pair(node_features, cm=True)
            qk, qk_cm = self.linear_qk.forward_layout(q_in, True, True), True
        else:
            qk, qk_cm = self.linear_qk(self.norm_qk(node_features)), False   # (N, 2 mult, dim)
        if edge_features is None and self.pool.reduce == "sum":
            # V projection, head weighting and sum pooling in one pass over the
            # edges where the fused kernels cover the layer (neither attn * V
            # nor its gradient is formed)
            attn = self.attention.node_attention_weights(qk, graph, distances, qk_cm)
            out = self.linear_v.attention_pool(P, Q_basis, node_features.contiguous(), distances, graph,
                                               attn, self.num_heads)
            if out is not None:
                return out
            V = self.linear_v(P, Q_basis, node_features.contiguous(), distances, graph=graph)
            perm, offsets = graph.csr()
            return AttnPoolFn.apply(V, attn, graph.dst, perm, offsets, graph.num_nodes, self.num_heads)
        if edge_features is not None:
            gathered = graph.gather_src(node_features) + edge_features
            V = self.linear_v(P, Q_basis, gathered, distances)       # (E, mult_out, dim_out)
        else:
            # x[src] gathered inside the fused layer (message-passing form)
            V = self.linear_v(P, Q_basis, node_features.contiguous(), distances, graph=graph)
        attn = self.attention.node_attention_weights(qk, graph, distances, qk_cm)
        if self.pool.reduce == "sum":
            perm, offsets = graph.csr()
            return AttnPoolFn.apply(V, attn, graph.dst, perm, offsets, graph.num_nodes,
                                    self.num_heads)
        return self.pool(self.attention._apply_attention(V, attn), graph)

    def extra_repr(self) -> str:
        return (f"in_repr={self.in_repr}, out_repr={self.out_repr}, "
                f"num_heads={self.num_heads}, reduce='{self.pool.reduce}'")
