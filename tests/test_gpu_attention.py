"""GPU parity of the attention kernels (csrc/attention.hip) against the float64
oracle: the node form (Q, K read from the fused QK projection's node table at
dst / src inside the kernels) and the edge form of the logits + softmax, the
head-weighted sum pooling, and all their gradients.

Shapes cover both chunk widths (16-byte chunks when the head length is a
multiple of 4 floats, single floats otherwise), head groups of 1..8 lanes,
more than 64 heads (two head passes), nodes without edges and edges whose
destination lies outside the graph (zero weights and gradients).
"""
import pytest
import torch

import flash_eq as fe
from flash_eq.ops import AttnPoolFn
from helpers import rel_err
from oracle import graphops as G

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _graph(Nn, E, g, empty_tail=3):
    """Random edges; the last ``empty_tail`` nodes have no incoming edges."""
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn - empty_tail, (E,), generator=g)
    return src, dst


@pytest.mark.parametrize("Nn,E,mult,dim,H", [
    (300, 6000, 64, 9, 8),      # config 3's heads: Dh = 72, 16-byte chunks, 8-lane groups
    (200, 3000, 6, 3, 3),       # Dh = 6: single floats, 16-lane groups (one idle group)
    (40, 900, 130, 1, 65),      # 65 heads of 2 floats: two head passes of 64
    (50, 700, 16, 9, 1),        # one head of 144 floats: 64-lane group
])
@pytest.mark.parametrize("cm", [False, True])
def test_node_form_matches_oracle(dev, Nn, E, mult, dim, H, cm):
    """cm: the table component-major (dim, N, 2 mult), as the fused QK
    projection writes it (feq_attn_softmax_fwd_cm / _bwd_cm)."""
    g = torch.Generator().manual_seed(Nn + E + H)
    src, dst = _graph(Nn, E, g)
    qk = torch.randn(Nn, 2 * mult, dim, generator=g)
    r = torch.rand(E, generator=g) * 8
    graph = fe.Graph(src.to(dev), dst.to(dev), Nn)
    Dh = mult // H * dim
    att = fe.EquivariantEdgeAttention(num_heads=H, qk_dim=Dh, distance_decay_scale=2.5).to(dev)
    qin = qk.permute(2, 0, 1).contiguous() if cm else qk
    qin = qin.to(dev).requires_grad_(True)
    rg = r.to(dev).requires_grad_(True)
    a = att.node_attention_weights(qin, graph, rg, cm)
    qd, rd = qk.double().requires_grad_(True), r.double().requires_grad_(True)
    ls = att.log_scale.detach().double().cpu().requires_grad_(True)
    Qe = qd[dst, :mult].reshape(E, H, Dh)
    Ke = qd[src, mult:].reshape(E, H, Dh)
    aref = G.neighbour_softmax(G.edge_logits(Qe, Ke, ls, rd, 2.5), dst, Nn)
    assert a.shape == (E, H)
    assert rel_err(a, aref) < TOL
    ga = torch.randn(E, H, generator=g)
    a.backward(ga.to(dev))
    aref.backward(ga.double())
    qgrad = qin.grad.permute(1, 2, 0) if cm else qin.grad
    assert rel_err(qgrad, qd.grad) < TOL
    assert rel_err(rg.grad, rd.grad) < TOL
    assert rel_err(att.log_scale.grad, ls.grad) < TOL
    # nodes without incoming edges: zero Q gradient; nodes without outgoing
    # edges: zero K gradient
    no_in = torch.bincount(dst, minlength=Nn) == 0
    assert torch.all(qgrad.cpu()[no_in, :mult] == 0)
    no_out = torch.bincount(src, minlength=Nn) == 0
    assert torch.all(qgrad.cpu()[no_out, mult:] == 0)


def test_node_form_equals_edge_form(dev):
    """The in-kernel gathers give the same weights and gradients as gathering
    Q, K to the edges first (edge form), to float32 rounding."""
    g = torch.Generator().manual_seed(11)
    Nn, E, mult, dim, H = 500, 8000, 32, 9, 4
    src, dst = _graph(Nn, E, g)
    graph = fe.Graph(src.to(dev), dst.to(dev), Nn)
    qk = torch.randn(Nn, 2 * mult, dim, generator=g).to(dev)
    Dh = mult // H * dim
    att = fe.EquivariantEdgeAttention(num_heads=H, qk_dim=Dh).to(dev)
    q1 = qk.clone().requires_grad_(True)
    a1 = att.node_attention_weights(q1, graph)
    q2 = qk.clone().requires_grad_(True)
    Qe = q2[graph.dst, :mult].reshape(E, H, Dh)
    Ke = q2[graph.src, mult:].reshape(E, H, Dh)
    a2 = att.attention_weights(Qe, Ke, graph)
    assert rel_err(a1, a2) < 1e-6
    ga = torch.randn(E, H, generator=g).to(dev)
    a1.backward(ga)
    a2.backward(ga)
    assert rel_err(q1.grad, q2.grad) < 1e-6


def test_out_of_range_destination_gets_zero_weight(dev):
    """An edge whose destination lies outside the graph is never part of a
    softmax: weight 0, zero gradients (edge and node form)."""
    g = torch.Generator().manual_seed(12)
    Nn, E, H, Dh = 50, 400, 2, 8
    src, dst = _graph(Nn, E, g, empty_tail=0)
    dst[::37] = Nn + 5
    graph = fe.Graph(src.to(dev), dst.to(dev), Nn)
    att = fe.EquivariantEdgeAttention(num_heads=H, qk_dim=Dh).to(dev)
    Q = torch.randn(E, H, Dh, generator=g).to(dev).requires_grad_(True)
    K = torch.randn(E, H, Dh, generator=g).to(dev).requires_grad_(True)
    a = att.attention_weights(Q, K, graph)
    bad = (dst >= Nn).to(dev)
    assert torch.all(a[bad] == 0)
    good = ~bad
    aref = G.neighbour_softmax(G.edge_logits(Q.detach()[good].double().cpu(),
                                             K.detach()[good].double().cpu(),
                                             att.log_scale.detach().double().cpu()),
                               dst[good.cpu()], Nn)
    assert rel_err(a[good], aref) < TOL
    a.backward(torch.randn(E, H, generator=g).to(dev))
    assert torch.all(Q.grad[bad] == 0) and torch.all(K.grad[bad] == 0)
    qk = torch.randn(Nn, 2 * H, Dh, generator=g).to(dev).requires_grad_(True)
    a2 = att.node_attention_weights(qk, graph)
    assert torch.all(a2[bad] == 0)


@pytest.mark.parametrize("mult,dim,H", [(64, 9, 8), (6, 3, 3), (8, 5, 2)])
def test_pool_matches_oracle(dev, mult, dim, H):
    """Head weighting + sum pooling and its gradients; (6, 3, 3) and (8, 5, 2)
    have head lengths that are not multiples of 4 (single-float chunks)."""
    g = torch.Generator().manual_seed(mult + dim + H)
    Nn, E = 120, 2500
    src, dst = _graph(Nn, E, g)
    graph = fe.Graph(src.to(dev), dst.to(dev), Nn)
    V = torch.randn(E, mult, dim, generator=g)
    A = torch.rand(E, H, generator=g)
    Vg, Ag = V.to(dev).requires_grad_(True), A.to(dev).requires_grad_(True)
    perm, offsets = graph.csr()
    out = AttnPoolFn.apply(Vg, Ag, graph.dst, perm, offsets, Nn, H)
    Vd, Ad = V.double().requires_grad_(True), A.double().requires_grad_(True)
    ref = G.pool_sum(G.apply_heads(Vd, Ad), dst, Nn)
    assert rel_err(out, ref) < TOL
    go = torch.randn(out.shape, generator=g)
    out.backward(go.to(dev))
    ref.backward(go.double())
    assert rel_err(Vg.grad, Vd.grad) < TOL
    assert rel_err(Ag.grad, Ad.grad) < TOL
