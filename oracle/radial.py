"""SeparableRadialNet table formula (oracle, float64 autograd).

Restates ``flash_eq/layers/radial.py:242-283``: sinusoidal features
``[sin(k pi x) e(x), cos(k pi x) e(x)]`` with ``x = clamp((r-min)/(max-min), 0, 1)``
and the quintic envelope ``e = 1 - 10x^3 + 15x^4 - 6x^5`` evaluated at the bin
edges, trunk Linear-SiLU-Linear-SiLU, head Linear, then
``T[b,o,i,w] = sum_k C[k,o,i] F[b,k,w]``.

Pinned by ``tests/test_oracle_graphops.py::test_envelope_closed_form`` (e(0)=1,
e(1)=0, e'(0)=e'(1)=0) and by the einsum identity against a loop.
"""
from __future__ import annotations

import torch


def sinusoidal_basis(r: torch.Tensor, min_val: float, max_val: float, num_freqs: int = 16,
                     freqs: torch.Tensor = None):
    """``freqs``: the module's ``frequencies`` buffer (k pi rounded to float32,
    radial.py:206-209); by default k pi in the dtype of r."""
    x = ((r - min_val) / (max_val - min_val)).clamp(0.0, 1.0)
    env = 1.0 - 10.0 * x ** 3 + 15.0 * x ** 4 - 6.0 * x ** 5
    if freqs is None:
        freqs = torch.arange(1, num_freqs + 1, dtype=torch.float32).to(r.dtype) * torch.pi
    else:
        freqs = freqs.to(r.dtype)
    ang = x[:, None] * freqs
    return torch.cat([torch.sin(ang) * env[:, None], torch.cos(ang) * env[:, None]], -1)


def radial_functions(params: dict, bin_edges: torch.Tensor, min_val: float, max_val: float,
                     rank: int, wdim: int) -> torch.Tensor:
    """F (num_bins+1, rank, wdim) from trunk/head parameters (keys as the module's state_dict)."""
    silu = torch.nn.functional.silu
    h = sinusoidal_basis(bin_edges, min_val, max_val, freqs=params.get("frequencies"))
    h = silu(h @ params["trunk.0.weight"].T + params["trunk.0.bias"])
    h = silu(h @ params["trunk.2.weight"].T + params["trunk.2.bias"])
    f = h @ params["head.weight"].T + params["head.bias"]
    return f.view(-1, rank, wdim)


def table(params: dict, bin_edges, min_val, max_val, rank, wdim) -> torch.Tensor:
    F = radial_functions(params, bin_edges, min_val, max_val, rank, wdim)
    return torch.einsum("koi,bkw->boiw", params["channel_patterns"], F)
