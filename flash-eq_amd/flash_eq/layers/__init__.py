"""Equivariant layers of the edge hot path and their node-side neighbours."""
from .linear import EquivariantEdgewiseLinear, EquivariantLinear
from .attention import EquivariantEdgeAttention, EquivariantAttention
from .norm import RepNorm, EquivariantLayerNorm, SeparableEquivariantLayerNorm
from .pooling import GraphPooling
from .gating import EquivariantGating
from .transformer import EquivariantTransformerBlock, EquivariantTransformer
from .radial import RadialBasisFunctions, RadialMLP, SeparableRadialNet

__all__ = [
    "EquivariantEdgewiseLinear", "EquivariantLinear",
    "EquivariantEdgeAttention", "EquivariantAttention",
    "RepNorm", "EquivariantLayerNorm", "SeparableEquivariantLayerNorm",
    "GraphPooling", "EquivariantGating",
    "EquivariantTransformerBlock", "EquivariantTransformer",
    "RadialBasisFunctions", "RadialMLP", "SeparableRadialNet",
]
