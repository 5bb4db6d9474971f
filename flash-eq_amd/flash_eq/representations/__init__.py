"""SO(3) representations: irreps, representations, Wigner-D matrices and bases."""
from .types import Irrep, ProductIrrep, Repr, ProductRepr
from .wigner import WignerD, WignerDBasis, random_rotation

__all__ = ["Irrep", "ProductIrrep", "Repr", "ProductRepr", "WignerD", "WignerDBasis",
           "random_rotation"]
