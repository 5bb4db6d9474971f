"""flash-eq for AMD Instinct MI355X (gfx950): the equivariant edge hot path.

Drop-in for the public API of hmblair/flash-eq (``flash_eq/__init__.py:17-81``)
restricted to the edge hot path and the modules the transformer needs:
representations and Wigner-D bases, the fused ``EquivariantEdgewiseLinear``,
attention, pooling, norms, gating and the transformer stack.  Per-edge work
runs in hand-written HIP kernels (``libflasheq.so``) reached through a C ABI.
"""
from .representations import (Irrep, ProductIrrep, Repr, ProductRepr, WignerD, WignerDBasis,
                              random_rotation)
from .graph import Graph
from .layers.radial import RadialBasisFunctions, RadialMLP, SeparableRadialNet
from .layers import (
    EquivariantEdgewiseLinear,
    EquivariantAttention,
    EquivariantEdgeAttention,
    RepNorm,
    EquivariantLinear,
    EquivariantGating,
    EquivariantLayerNorm,
    SeparableEquivariantLayerNorm,
    GraphPooling,
    EquivariantTransformerBlock,
    EquivariantTransformer,
)
from ._native import CUDANotAvailableError

__all__ = [
    "Irrep", "ProductIrrep", "Repr", "ProductRepr", "WignerD", "random_rotation",
    "Graph",
    "EquivariantEdgewiseLinear", "EquivariantAttention", "RepNorm", "EquivariantLinear",
    "EquivariantGating", "EquivariantLayerNorm", "SeparableEquivariantLayerNorm",
    "GraphPooling", "EquivariantEdgeAttention",
    "EquivariantTransformerBlock", "EquivariantTransformer",
    "WignerDBasis",
    "RadialBasisFunctions", "RadialMLP", "SeparableRadialNet",
    "CUDANotAvailableError",
]

__version__ = "0.1.0"
