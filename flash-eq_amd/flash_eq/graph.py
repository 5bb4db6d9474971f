"""COO graph container (drop-in for ``flash_eq/graph.py:15-97``).

Adds one thing the reference does not have: ``Graph.csr()`` returns the edges
grouped by destination (``perm``, ``offsets``), built once per device by the
HIP radix sort and cached on the object, so every edge->node reduction of the
layers walks contiguous segments instead of scattering with atomics.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Tuple

import torch

from . import _native as N


@dataclass
class Graph:
    """Edge indices ``src``/``dst`` (E,) and the node count."""

    src: torch.Tensor
    dst: torch.Tensor
    num_nodes: int
    _csr_cache: Dict[str, Tuple[torch.Tensor, torch.Tensor]] = field(
        default_factory=dict, init=False, repr=False, compare=False)

    def __post_init__(self) -> None:
        if self.src.dim() != 1:
            raise ValueError(f"src must be 1D, got shape {self.src.shape}")
        if self.dst.dim() != 1:
            raise ValueError(f"dst must be 1D, got shape {self.dst.shape}")
        if self.src.shape[0] != self.dst.shape[0]:
            raise ValueError(
                f"src and dst must have same length, got {self.src.shape[0]} and {self.dst.shape[0]}")
        if self.num_nodes <= 0:
            raise ValueError(f"num_nodes must be positive, got {self.num_nodes}")

    @property
    def num_edges(self) -> int:
        return self.src.shape[0]

    @property
    def device(self) -> torch.device:
        return self.src.device

    @property
    def dtype(self) -> torch.dtype:
        return self.src.dtype

    def to(self, device) -> "Graph":
        return Graph(src=self.src.to(device), dst=self.dst.to(device), num_nodes=self.num_nodes)

    @staticmethod
    def random(num_nodes: int, num_edges: int, device="cpu") -> "Graph":
        """Uniform random src/dst (self-loops and multi-edges allowed), as ``graph.py:79-97``."""
        src = torch.randint(0, num_nodes, (num_edges,), device=device)
        dst = torch.randint(0, num_nodes, (num_edges,), device=device)
        return Graph(src=src, dst=dst, num_nodes=num_nodes)

    def csr(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """(perm int32 (E,), offsets int32 (N+1,)) grouping edges by destination.

        ``perm[offsets[n]:offsets[n+1]]`` are the edges into node n in
        increasing edge id (stable).  Computed on the GPU and cached.
        """
        N.require_cuda_tensor(self.dst, "graph.dst")
        key = str(self.dst.device)
        hit = self._csr_cache.get(key)
        if hit is not None:
            return hit
        dev = self.dst.device
        E, Nn = self.num_edges, self.num_nodes
        dst = self.dst.to(torch.int64).contiguous()
        perm = torch.empty(E, dtype=torch.int32, device=dev)
        offsets = torch.empty(Nn + 1, dtype=torch.int32, device=dev)
        lib = N.lib()
        ws = N.workspace(lib.feq_csr_workspace(E, Nn), dev)
        with torch.cuda.device(dev):
            rc = lib.feq_csr_by_dst(N.ptr(dst) if E else None, E, Nn, N.ptr(perm) if E else None,
                                    N.ptr(offsets), N.ptr(ws), ws.numel(), N.stream_ptr(dev))
        N.check(rc, "feq_csr_by_dst")
        self._csr_cache[key] = (perm, offsets)
        return perm, offsets
