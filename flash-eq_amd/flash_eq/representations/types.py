"""Real irreducible representations of SO(3): metadata and generators.

Same public surface and numerics as the reference ``representations/types.py``:

* ``Irrep(l, mult)``: degree ``l``, dimension ``2l+1``; its so(3) generators
  are built in complex128 in the |l, m> basis, conjugated into the real
  spherical-harmonic basis and rounded to float32 (``types.py:74-135``).
* ``Repr(lvals, mult)``: ordered list of irreps, duplicates allowed
  (``types.py:178-305``).
* ``ProductRepr(rep1, rep2)``: tensor-product bookkeeping; ``nreps()`` is the
  radial weight width ``sum_{l in rep1, l' in rep2} (2 min(l, l') + 1)``
  (``types.py:157-171``, ``:308-350``).
"""
from __future__ import annotations

import math
from typing import Any, Iterator, List, Sequence

import torch

__all__ = ["Irrep", "ProductIrrep", "Repr", "ProductRepr"]


def _sqrt_f32(n: int) -> float:
    """Correctly rounded float32 square root of a non-negative integer."""
    return float(torch.tensor(float(n), dtype=torch.float32).sqrt())


class Irrep:
    """Degree-``l`` real irrep of SO(3) with multiplicity ``mult``."""

    REAL_DTYPE = torch.float32
    COMPLEX_DTYPE = torch.complex128

    def __init__(self, l: int, mult: int = 1) -> None:
        if not isinstance(l, int) or l < 0:
            raise ValueError(f"Degree l must be a non-negative integer, got {l}")
        if not isinstance(mult, int) or mult < 1:
            raise ValueError(f"Multiplicity must be a positive integer, got {mult}")
        self.l = l
        self.mult = mult

    def __eq__(self, other: Any) -> bool:
        return isinstance(other, Irrep) and (self.l, self.mult) == (other.l, other.mult)

    def __hash__(self) -> int:
        return hash((self.l, self.mult))

    def dim(self) -> int:
        return 2 * self.l + 1

    def mvals(self) -> torch.Tensor:
        return torch.arange(-self.l, self.l + 1)

    # -- ladder operators in the complex |l, m> basis, m = -l..l ------------
    # The ladder entries are float32 square roots of integers, as in the
    # reference (sqrt of an integer tensor); this fixes the last bit of the
    # float32 generators built from them.
    def raising(self) -> torch.Tensor:
        """J+ with the reference's sign: entry (m+1, m) = -sqrt(l(l+1) - m(m+1))."""
        l = self.l
        out = torch.zeros(self.dim(), self.dim(), dtype=torch.float32)
        for m in range(-l, l):
            out[m + 1 + l, m + l] = -_sqrt_f32(l * (l + 1) - m * (m + 1))
        return out

    def lowering(self) -> torch.Tensor:
        """J-: entry (m-1, m) = sqrt(l(l+1) - m(m-1))."""
        l = self.l
        out = torch.zeros(self.dim(), self.dim(), dtype=torch.float32)
        for m in range(-l + 1, l + 1):
            out[m - 1 + l, m + l] = _sqrt_f32(l * (l + 1) - m * (m - 1))
        return out

    def toreal(self) -> torch.Tensor:
        """Unitary map from complex to real spherical harmonics (``types.py:114-135``).

        Row ``l+m`` holds the real harmonic of order ``m``; an overall phase
        ``(-i)^l`` is applied, matching the reference convention.
        """
        l, d = self.l, self.dim()
        h = 1.0 / math.sqrt(2.0)
        q = torch.zeros(d, d, dtype=torch.complex128)
        for m in range(1, l + 1):
            sgn = -1.0 if (m % 2) else 1.0
            # negative order: combination of |m| and -|m| with -i weight
            q[l - m, l + m] = h
            q[l - m, l - m] = -1j * h
            # positive order: (-1)^m weighted combination
            q[l + m, l + m] = sgn * h
            q[l + m, l - m] = 1j * sgn * h
        q[l, l] = 1.0
        return ((-1j) ** l) * q

    def _generators(self) -> torch.Tensor:
        """Real-basis generators stacked in the slot order ``[Lz, Lx, Ly]``.

        ``Jx = (J+ + J-)/2``, ``Jy = -i (J+ - J-)/2``, ``Jz = i diag(m)``;
        conjugation by the real map sends Jx -> Lx, Jy -> Lz, Jz -> Ly
        (``types.py:86-112``).
        """
        rp = self.raising().to(self.COMPLEX_DTYPE)
        lo = self.lowering().to(self.COMPLEX_DTYPE)
        jx = 0.5 * (rp + lo)
        jy = -0.5j * (rp - lo)
        jz = 1j * torch.diag(self.mvals().to(self.COMPLEX_DTYPE))
        q = self.toreal()
        qh = q.t().conj()

        def real_part(j: torch.Tensor) -> torch.Tensor:
            return (qh @ j @ q).real.to(self.REAL_DTYPE)

        return torch.stack([real_part(jy), real_part(jx), real_part(jz)], dim=0)

    def __str__(self) -> str:
        return f"Irrep(l={self.l}, mult={self.mult})"


class ProductIrrep:
    """Clebsch-Gordan decomposition bookkeeping of ``rep1 x rep2``."""

    def __init__(self, rep1: Irrep, rep2: Irrep) -> None:
        self.rep1 = rep1
        self.rep2 = rep2
        self.lmin = abs(rep1.l - rep2.l)
        self.lmax = rep1.l + rep2.l
        self.reps = [Irrep(l) for l in range(self.lmin, self.lmax + 1)]

    def dim(self) -> int:
        return sum(r.dim() for r in self.reps)

    def maxdim(self) -> int:
        return max(r.dim() for r in self.reps)

    def nreps(self) -> int:
        return len(self.reps)

    def __str__(self) -> str:
        return f"ProductIrrep({self.rep1.l} x {self.rep2.l})"


class Repr:
    """Ordered collection of irreps sharing one multiplicity."""

    def __init__(self, lvals: Sequence[int], mult: int = 1) -> None:
        if not hasattr(lvals, "__len__"):
            raise TypeError(f"lvals must be a sequence, got {type(lvals).__name__}")
        if len(lvals) == 0:
            raise ValueError("lvals must contain at least one degree")
        if not isinstance(mult, int) or mult < 1:
            raise ValueError(f"Multiplicity must be a positive integer, got {mult}")
        self.irreps = [Irrep(int(l), mult) for l in lvals]
        self.lvals = torch.tensor([ir.l for ir in self.irreps], dtype=torch.long)
        self.mult = mult
        offs = [0]
        for ir in self.irreps:
            offs.append(offs[-1] + ir.dim())
        self._cumdims = torch.tensor(offs)

    def nreps(self) -> int:
        return len(self.irreps)

    def __iter__(self) -> Iterator[Irrep]:
        return iter(self.irreps)

    def __eq__(self, other: Any) -> bool:
        return (isinstance(other, Repr) and self.mult == other.mult
                and torch.equal(self.lvals, other.lvals))

    def __hash__(self) -> int:
        return hash((tuple(self.lvals.tolist()), self.mult))

    def dim(self) -> int:
        return int(self._cumdims[-1])

    def lmax(self) -> int:
        return max(ir.l for ir in self.irreps)

    def cumdims(self) -> torch.Tensor:
        return self._cumdims

    def mvals(self) -> torch.Tensor:
        return torch.cat([ir.mvals() for ir in self.irreps])

    def indices(self) -> List[int]:
        """Irrep index of every component (``types.py:250-263``)."""
        out: List[int] = []
        for k, ir in enumerate(self.irreps):
            out += [k] * ir.dim()
        return out

    def l_indices(self) -> torch.Tensor:
        return self.lvals[self.indices()]

    def find_scalar(self) -> tuple[int, List[int]]:
        """(count, component offsets) of the l=0 irreps (``types.py:279-301``)."""
        offs = self._cumdims.tolist()
        locs = [offs[k] for k, ir in enumerate(self.irreps) if ir.l == 0]
        return len(locs), locs

    def __str__(self) -> str:
        return "Repr(lvals=[" + ", ".join(str(ir.l) for ir in self.irreps) + "])"


class ProductRepr:
    """Tensor product ``rep1 x rep2`` of two representations."""

    def __init__(self, rep1: Repr, rep2: Repr) -> None:
        self.rep1 = rep1
        self.rep2 = rep2
        self.reps = [ProductIrrep(a, b) for a in rep1 for b in rep2]

    def dim(self) -> int:
        return sum(r.dim() for r in self.reps)

    def __eq__(self, other: Any) -> bool:
        return isinstance(other, ProductRepr) and self.rep1 == other.rep1 and self.rep2 == other.rep2

    def __hash__(self) -> int:
        return hash((hash(self.rep1), hash(self.rep2)))

    def lmax(self) -> int:
        return max(r.lmax for r in self.reps)

    def nreps(self) -> int:
        return sum(r.nreps() for r in self.reps)

    def __str__(self) -> str:
        return f"ProductRepr({self.rep1} x {self.rep2})"
