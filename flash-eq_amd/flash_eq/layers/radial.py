"""Radial weight networks (drop-in for ``flash_eq/layers/radial.py``).

``SeparableRadialNet`` produces the binned radial weights
``T[b, o, i, w] = sum_k C[k, o, i] F[b, k, w]`` (``radial.py:133-283``).  The
fused edgewise kernel consumes the two factors (``channel_patterns`` C and
``radial_functions()`` F) directly; ``forward()`` still materialises the full
table for callers of the generic block-diagonal op.  Parameters are created
and initialised in the reference's order so seeded construction matches.
"""
from __future__ import annotations

import math
import weakref

import torch
import torch.nn as nn

from ..utils import get_epsilon, init_linear_weights


# SeparableRadialNet -> (bin-edge buffer refs and versions, basis): see _edge_basis
_BASIS_CACHE: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()


class RadialBasisFunctions(nn.Module):
    """Gaussian RBF expansion with learnable centres/widths (``radial.py:19-64``)."""

    def __init__(self, num_functions: int, r_min: float = 0.0, r_max: float = 10.0) -> None:
        super().__init__()
        self.num_functions = num_functions
        self.mu = nn.Parameter(torch.linspace(r_min, r_max, num_functions))
        width = (r_max - r_min) / max(num_functions - 1, 1)
        self.sigma = nn.Parameter(torch.full((num_functions,), width))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dim() > 1 and x.size(-1) == 1:
            x = x.squeeze(-1)
        eps = get_epsilon(self.sigma.dtype)
        z = (x[..., None] - self.mu) / self.sigma.abs().clamp(min=eps)
        return torch.exp(-z * z)


class RadialMLP(nn.Module):
    """RBF + MLP mapping distances to (N, out, in, num_basis) weights (``radial.py:67-130``)."""

    def __init__(self, hidden_dim: int, num_basis: int, in_mult: int, out_mult: int,
                 num_layers: int = 2, r_max: float = 10.0) -> None:
        super().__init__()
        self.num_basis = num_basis
        self.in_mult = in_mult
        self.out_mult = out_mult
        self.rbf = RadialBasisFunctions(hidden_dim, r_min=0.0, r_max=r_max)
        layers: list = [nn.Linear(hidden_dim, hidden_dim), nn.SiLU()]
        for _ in range(num_layers - 1):
            layers += [nn.Linear(hidden_dim, hidden_dim), nn.SiLU()]
        layers.append(nn.Linear(hidden_dim, out_mult * in_mult * num_basis))
        self.mlp = nn.Sequential(*layers)
        self.apply(init_linear_weights)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n = x.size(0)
        return self.mlp(self.rbf(x)).view(n, self.out_mult, self.in_mult, self.num_basis)


class SeparableRadialNet(nn.Module):
    """Rank-K separable binned radial weights W[o,i,w](r) = sum_k C_k[o,i] f_k(r, w)."""

    bin_edges: torch.Tensor
    frequencies: torch.Tensor

    def __init__(self, num_bins: int = 100, out_mult: int = 16, in_mult: int = 16,
                 weight_dim: int = 7, rank: int = 4, num_freqs: int = 16, hidden_dim: int = 64,
                 min_val: float = 0.0, max_val: float = 10.0, log: bool = False) -> None:
        super().__init__()
        if log and min_val <= 0:
            raise ValueError("min_val must be > 0 for log spacing")
        self.num_bins = num_bins
        self.out_mult = out_mult
        self.in_mult = in_mult
        self.weight_dim = weight_dim
        self.rank = rank
        self.min_val = min_val
        self.max_val = max_val
        self.log = log
        # creation order (and hence RNG consumption) follows radial.py:200-240
        self.channel_patterns = nn.Parameter(torch.empty(rank, out_mult, in_mult))
        nn.init.xavier_uniform_(self.channel_patterns)
        self.register_buffer("frequencies",
                             torch.arange(1, num_freqs + 1, dtype=torch.float32) * torch.pi)
        self.trunk = nn.Sequential(
            nn.Linear(2 * num_freqs, hidden_dim), nn.SiLU(),
            nn.Linear(hidden_dim, hidden_dim), nn.SiLU(),
        )
        self.head = nn.Linear(hidden_dim, rank * weight_dim)
        if log:
            lo = float(torch.tensor(min_val).log10())
            hi = float(torch.tensor(max_val).log10())
            self.register_buffer("bin_edges", torch.logspace(lo, hi, num_bins + 1))
            self._log_min = float(torch.tensor(min_val).log())
            self._inv_log_range = 1.0 / float(torch.tensor(max_val / min_val).log())
        else:
            self.register_buffer("bin_edges", torch.linspace(min_val, max_val, num_bins + 1))
        self.apply(init_linear_weights)

    def _sinusoidal_basis(self, r: torch.Tensor) -> torch.Tensor:
        """[sin(k pi x) e(x), cos(k pi x) e(x)], x = clamp((r-min)/(max-min)), e = 1-10x^3+15x^4-6x^5."""
        x = ((r - self.min_val) / (self.max_val - self.min_val)).clamp(0.0, 1.0)
        env = 1.0 - 10.0 * x ** 3 + 15.0 * x ** 4 - 6.0 * x ** 5
        ang = x.unsqueeze(-1) * self.frequencies
        return torch.cat([torch.sin(ang) * env.unsqueeze(-1), torch.cos(ang) * env.unsqueeze(-1)], -1)

    def _edge_basis(self) -> torch.Tensor:
        """The sinusoidal basis at the bin edges, formed from buffers only and
        kept until a buffer changes.

        The cache (outside the module's state, so pickling and deepcopy are
        unaffected) holds weak references to the very buffer objects it was
        formed from and their in-place versions: a replaced buffer (``.to()``,
        the float32 copies of a half-precision module run in float32) misses.
        A basis formed under ``torch.inference_mode()`` is an inference tensor,
        which autograd cannot save for a later backward: it is never kept."""
        be, fq = self.bin_edges, self.frequencies
        cached = _BASIS_CACHE.get(self)
        if cached is not None:
            rbe, vbe, rfq, vfq, basis = cached
            if rbe() is be and rfq() is fq and vbe == be._version and vfq == fq._version:
                return basis
        basis = self._sinusoidal_basis(be)
        if basis.is_inference():
            _BASIS_CACHE.pop(self, None)
        else:
            _BASIS_CACHE[self] = (weakref.ref(be), be._version, weakref.ref(fq), fq._version, basis)
        return basis

    def _fused_mlp_ok(self, basis: torch.Tensor) -> bool:
        t = self.trunk
        if not (basis.is_cuda and len(t) == 4 and isinstance(t[0], nn.Linear) and isinstance(t[1], nn.SiLU)
                and isinstance(t[2], nn.Linear) and isinstance(t[3], nn.SiLU)):
            return False
        params = (t[0].weight, t[0].bias, t[2].weight, t[2].bias, self.head.weight, self.head.bias)
        if any(p is None or p.dtype != torch.float32 or not p.is_cuda for p in params) or basis.dtype != torch.float32:
            return False
        from ..ops import radial_mlp_supported
        return radial_mlp_supported(basis.shape[0], basis.shape[1], t[0].out_features, self.head.out_features)

    def radial_functions(self) -> torch.Tensor:
        """F[b, k, w]: the radial factor at every bin edge, shape (num_bins+1, rank, weight_dim).
        On the GPU in float32 the network runs as the fused kernels of
        ``RadialMLPFn`` (one workgroup forward, one backward)."""
        basis = self._edge_basis()
        if self._fused_mlp_ok(basis):
            from ..ops import RadialMLPFn
            t = self.trunk
            F = RadialMLPFn.apply(basis, t[0].weight, t[0].bias, t[2].weight, t[2].bias, self.head.weight,
                                  self.head.bias)
        else:
            F = self.head(self.trunk(basis))
        return F.view(-1, self.rank, self.weight_dim)

    def forward(self) -> torch.Tensor:
        """Full table (num_bins+1, out_mult, in_mult, weight_dim) (``radial.py:259-275``)."""
        return torch.einsum("koi,bkw->boiw", self.channel_patterns, self.radial_functions())

    def binning_params(self) -> tuple:
        """(min, num_bins/(max-min)) for linear bins, (log min, 1/log(max/min)) for log bins."""
        if self.log:
            return (self._log_min, self._inv_log_range)
        return (self.min_val, self.num_bins / (self.max_val - self.min_val))

    def bin_indices(self, values: torch.Tensor):
        """Bin index and clamped interpolation weight (``radial.py:285-296``)."""
        if self.log:
            nrm = ((values.float().clamp(min=self.min_val).log() - self._log_min)
                   * self._inv_log_range * self.num_bins)
        else:
            nrm = (values.float() - self.min_val) * (self.num_bins / (self.max_val - self.min_val))
        nrm = nrm.clamp(0.0, self.num_bins)
        lo = nrm.floor().int().clamp(max=self.num_bins - 1)
        return lo, (nrm - lo.float()).clamp(0.0, 1.0)
