"""COO graph container (drop-in for ``flash_eq/graph.py:15-97``).

Adds what the reference does not have: ``Graph.csr()`` / ``csr_src()`` return
the edges grouped by destination / source (``perm``, ``offsets``), built once
per device by the HIP radix sort and cached on the object, so every edge->node
reduction of the layers walks contiguous segments instead of scattering with
atomics; ``gather_src`` / ``gather_dst`` are ``x[src]`` / ``x[dst]`` whose
backward is such a segmented sum.
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
        return self._csr_of(self.dst, "dst")

    def csr_src(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """The same grouping of the edges by source node (cached)."""
        return self._csr_of(self.src, "src")

    def gather_src(self, node_values: torch.Tensor) -> torch.Tensor:
        """``node_values[src]`` (E, ...) whose backward sums every node's outgoing
        edge rows over the cached CSR by source (no atomics, fixed order)."""
        from .ops import gather_rows
        perm, offsets = self.csr_src()
        return gather_rows(node_values, self.src, perm, offsets)

    def gather_dst(self, node_values: torch.Tensor) -> torch.Tensor:
        """``node_values[dst]`` (E, ...), backward over the CSR by destination."""
        from .ops import gather_rows
        perm, offsets = self.csr()
        return gather_rows(node_values, self.dst, perm, offsets)

    def _csr_of(self, index: torch.Tensor, which: str) -> Tuple[torch.Tensor, torch.Tensor]:
        N.require_cuda_tensor(index, f"graph.{which}")
        key = f"{which}:{index.device}"
        hit = self._csr_cache.get(key)
        if hit is not None:
            return hit
        dev = index.device
        E, Nn = self.num_edges, self.num_nodes
        idx = index.to(torch.int64).contiguous()
        perm = torch.empty(E, dtype=torch.int32, device=dev)
        offsets = torch.empty(Nn + 1, dtype=torch.int32, device=dev)
        lib = N.lib()
        ws = N.workspace(lib.feq_csr_workspace(E, Nn), dev)
        with torch.cuda.device(dev):
            rc = lib.feq_csr_by_dst(N.ptr(idx) if E else None, E, Nn, N.ptr(perm) if E else None,
                                    N.ptr(offsets), N.ptr(ws), ws.numel(), N.stream_ptr(dev))
        N.check(rc, "feq_csr_by_dst")
        self._csr_cache[key] = (perm, offsets)
        return perm, offsets
