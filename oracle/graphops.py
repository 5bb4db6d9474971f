"""Edge->node reductions and the neighbour softmax (oracle, float64).

Restates ``flash_eq/layers/pooling.py:21-64`` and
``flash_eq/layers/attention.py:92-167``.  Vectorised forms use
``index_add``/``scatter_reduce`` (library routines); the ``*_loop`` forms are
per-node brute force for tiny graphs.

Pinned by ``tests/test_oracle_graphops.py``: the reference's pooling
known-answer tests (tests/test_layers.py:470-602, stored as data in
``tests/golden/pooling_kat.json``), loop-vs-vectorised agreement, softmax rows
summing to 1 per destination (test_attention.py:77-108) and shift invariance.
"""
from __future__ import annotations

import torch


def pool_sum(x: torch.Tensor, dst: torch.Tensor, num_nodes: int) -> torch.Tensor:
    out = torch.zeros((num_nodes,) + tuple(x.shape[1:]), dtype=x.dtype)
    return out.index_add(0, dst.long(), x)


def pool_sum_loop(x, dst, num_nodes):
    out = torch.zeros((num_nodes,) + tuple(x.shape[1:]), dtype=x.dtype)
    for e in range(x.shape[0]):
        out[int(dst[e])] += x[e]
    return out


def pool_mean(x, dst, num_nodes):
    s = pool_sum(x, dst, num_nodes)
    cnt = torch.zeros(num_nodes, dtype=x.dtype).index_add(0, dst.long(), torch.ones(x.shape[0], dtype=x.dtype))
    return s / cnt.clamp(min=1).view(-1, *([1] * (x.dim() - 1)))


def pool_max(x, dst, num_nodes):
    _, c, d = x.shape
    out = torch.full((num_nodes, c, d), float("-inf"), dtype=x.dtype)
    out = out.scatter_reduce(0, dst.long().view(-1, 1, 1).expand(-1, c, d), x, reduce="amax")
    return out.nan_to_num(neginf=0.0)


def edge_logits(Q, K, log_scale, distances=None, decay=None):
    lg = (Q * K).sum(-1) * torch.exp(log_scale)
    if decay is not None and distances is not None:
        lg = lg - distances.unsqueeze(-1) / decay
    return lg


def neighbour_softmax(logits: torch.Tensor, dst: torch.Tensor, num_nodes: int) -> torch.Tensor:
    """exp(l - max_dst) / (sum_dst exp(l - max_dst) + 1e-8) per head (attention.py:108-141)."""
    E, H = logits.shape
    idx = dst.long().unsqueeze(-1).expand(E, H)
    mx = torch.full((num_nodes, H), float("-inf"), dtype=logits.dtype)
    mx = mx.scatter_reduce(0, idx, logits, reduce="amax", include_self=False)
    ex = torch.exp(logits - mx.gather(0, idx))
    s = torch.zeros(num_nodes, H, dtype=logits.dtype).scatter_add(0, idx, ex)
    return ex / (s.gather(0, idx) + 1e-8)


def neighbour_softmax_loop(logits, dst, num_nodes):
    out = torch.zeros_like(logits)
    for n in range(num_nodes):
        sel = (dst == n).nonzero().flatten()
        if sel.numel() == 0:
            continue
        l = logits[sel]
        ex = torch.exp(l - l.max(0).values)
        out[sel] = ex / (ex.sum(0) + 1e-8)
    return out


def apply_heads(V: torch.Tensor, attn: torch.Tensor) -> torch.Tensor:
    """V (E, mult, dim) weighted by attn (E, H): channel c belongs to head c // (mult/H)."""
    E, mult, dim = V.shape
    H = attn.shape[1]
    return (V.view(E, H, mult // H, dim) * attn.view(E, H, 1, 1)).view(E, mult, dim)
