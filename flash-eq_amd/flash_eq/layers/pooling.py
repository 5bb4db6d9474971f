"""Edge -> node aggregation (drop-in for ``flash_eq/layers/pooling.py``).

'sum' (the transformer's reduction, ``pooling.py:21-30``) runs the HIP
segmented sum over the graph's cached CSR: one workgroup per node, edges in
a fixed order, no atomics.  'mean' divides that sum by the in-degree from the
CSR offsets.  'max' (``pooling.py:47-58``) is not on the hot path and keeps a
PyTorch scatter_reduce.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import _native as N
from ..graph import Graph
from ..ops import SegmentSumFn

_REDUCTIONS = ("sum", "mean", "max")


def _pool_sum(edge_features: torch.Tensor, graph: Graph) -> torch.Tensor:
    N.require_cuda_tensor(edge_features, "edge_features")
    perm, offsets = graph.csr()
    return SegmentSumFn.apply(edge_features, graph.dst, perm, offsets, graph.num_nodes)


def _pool_mean(edge_features: torch.Tensor, graph: Graph) -> torch.Tensor:
    out = _pool_sum(edge_features, graph)
    _, offsets = graph.csr()
    counts = (offsets[1:] - offsets[:-1]).to(out.dtype).clamp(min=1)
    return out / counts.view(-1, *([1] * (out.dim() - 1)))


def _pool_max(edge_features: torch.Tensor, graph: Graph) -> torch.Tensor:
    _, c, d = edge_features.shape
    idx = graph.dst.view(-1, 1, 1).expand(-1, c, d)
    out = torch.full((graph.num_nodes, c, d), float("-inf"), device=edge_features.device,
                     dtype=edge_features.dtype)
    out.scatter_reduce_(0, idx, edge_features, reduce="amax")
    return out.nan_to_num(neginf=0.0)


_FUNCS = {"sum": _pool_sum, "mean": _pool_mean, "max": _pool_max}


class GraphPooling(nn.Module):
    """Aggregate (E, C, D) edge features onto the destination nodes."""

    def __init__(self, reduce: str = "sum") -> None:
        super().__init__()
        if reduce not in _FUNCS:
            raise ValueError(f"reduce must be one of {list(_REDUCTIONS)}, got '{reduce}'")
        self.reduce = reduce
        self._pool_fn = _FUNCS[reduce]

    def forward(self, edge_features: torch.Tensor, graph: Graph) -> torch.Tensor:
        return self._pool_fn(edge_features, graph)

    def extra_repr(self) -> str:
        return f"reduce='{self.reduce}'"
