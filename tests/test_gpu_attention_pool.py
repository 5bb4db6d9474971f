"""The V projection of EquivariantAttention fused with the head weighting and
sum pooling (layer.attention_pool: feq_edgewise_fwd_src_pool /
feq_edgewise_bwd_src_pool / feq_attn_pool_grad_attn) against the unfused
composition that the reference spells out (attention.py:307-314,
pooling.py:21-30): V = layer(x[src]) per edge, then sum over e -> n of
attn[e, head(c)] V[e] (AttnPoolFn).

The per-edge arithmetic is the same; the fused forward sums attn * V per
destination in CSR order (partial rows for nodes crossing a 16-edge tile), the
fused backward scales grad_out[dst] by attn inside the layer's kernels, so
output and gradients agree to float32 rounding of reordered sums (2e-6).  The
composed block and model tests against the float64 oracle (test_gpu_model.py,
test_gpu_composed.py) run this path for their [0,1,2]x64 layers.
"""
import pytest
import torch

import flash_eq as fe
from flash_eq.ops import AttnPoolFn
from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 2e-6


@pytest.fixture(autouse=True)
def split_kernels(monkeypatch):
    monkeypatch.delenv("FEQ_EW_PATH", raising=False)
    monkeypatch.delenv("FEQ_FORCE_GENERIC", raising=False)


def _setup(dev, lin, lout, cin, cout, N, E, heads, seed, bad_dst=0):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, N - 2, (E,), generator=g)          # the last two nodes send nothing
    dst = torch.randint(0, N - 3, (E,), generator=g)          # the last three receive nothing
    dst, _ = torch.sort(dst)                                  # runs of edges per node, as kNN graphs
    dst = dst[torch.randperm(E, generator=g)] if seed % 2 else dst
    if bad_dst:
        idx = torch.randperm(E, generator=g)[:bad_dst]
        dst[idx[: bad_dst // 2]] = -1
        dst[idx[bad_dst // 2:]] = N
    torch.manual_seed(seed)
    layer = fe.EquivariantEdgewiseLinear(fe.Repr(lin, cin), fe.Repr(lout, cout), num_bins=40).to(dev)
    d = torch.randn(E, 3, generator=g).to(dev)
    P, Q = fe.WignerDBasis([fe.Repr(lin, 1), fe.Repr(lout, 1)]).to(dev)(d)
    x = torch.randn(N, cin, P.shape[-1], generator=g)
    r = (torch.rand(E, generator=g) * 11).to(dev)
    attn = torch.rand(E, heads, generator=g)
    gout = torch.randn(N, cout, Q.shape[-1], generator=g).to(dev)
    return layer, fe.Graph(src.to(dev), dst.to(dev), N), P, Q, x, r, attn, gout


def _run(layer, graph, P, Q, x, r, attn, gout, heads, fused):
    dev = P.device
    xg = x.to(dev).requires_grad_(True)
    rg = r.clone().requires_grad_(True)
    ag = attn.to(dev).requires_grad_(True)
    if fused:
        out = layer.attention_pool(P, Q, xg, rg, graph, ag, heads)
        assert out is not None, "the fused kernels must cover this layout"
    else:
        V = layer(P, Q, xg, rg, graph=graph)
        perm, offsets = graph.csr()
        out = AttnPoolFn.apply(V, ag, graph.dst, perm, offsets, graph.num_nodes, heads)
    for p in layer.parameters():
        p.grad = None
    out.backward(gout)
    grads = [p.grad.clone() for p in layer.radial_weights.parameters()]
    return out.detach(), xg.grad, rg.grad, ag.grad, grads


@pytest.mark.parametrize("E,N,heads,seed", [(3000, 200, 8, 1), (3000, 200, 8, 2), (1037, 500, 4, 3),
                                            (17, 9, 16, 4), (5000, 40, 2, 5)])
def test_pooled_matches_unfused(dev, E, N, heads, seed):
    print(f"pooled vs unfused [0,1,2]x64 E={E} N={N} heads={heads} seed={seed}", flush=True)
    layer, graph, P, Q, x, r, attn, gout = _setup(dev, [0, 1, 2], [0, 1, 2], 64, 64, N, E, heads, seed)
    ref = _run(layer, graph, P, Q, x, r, attn, gout, heads, False)
    got = _run(layer, graph, P, Q, x, r, attn, gout, heads, True)
    names = ["out", "grad_x", "grad_r", "grad_attn"]
    for n, a, b in zip(names, got[:4], ref[:4]):
        assert rel_err(a, b) < TOL, (n, rel_err(a, b))
    for i, (a, b) in enumerate(zip(got[4], ref[4])):
        assert rel_err(a, b) < TOL, ("radial parameter", i, rel_err(a, b))
    # nodes without incoming edges get zero rows
    assert torch.count_nonzero(got[0][N - 3:]) == 0


def test_pooled_out_of_range_destinations(dev):
    """Edges whose dst lies outside [0, N) add nothing and get zero gradients,
    as the unfused pooling drops them."""
    layer, graph, P, Q, x, r, attn, gout = _setup(dev, [0, 1, 2], [0, 1, 2], 64, 64, 150, 2500, 8, 7,
                                                  bad_dst=300)
    ref = _run(layer, graph, P, Q, x, r, attn, gout, 8, False)
    got = _run(layer, graph, P, Q, x, r, attn, gout, 8, True)
    for a, b in zip(got[:4], ref[:4]):
        assert rel_err(a, b) < TOL
    bad = ((graph.dst < 0) | (graph.dst >= 150)).cpu()
    assert torch.count_nonzero(got[3].cpu()[bad]) == 0
    assert torch.count_nonzero(got[2].cpu()[bad]) == 0


@pytest.mark.parametrize("lin,lout,cin", [([0, 1], [0, 1, 2], 32), ([0, 1, 2], [0, 1], 64),
                                          ([0, 1], [0, 1], 64)])
def test_pooled_embedded_layout(dev, lin, lout, cin):
    """Small layouts run zero-embedded in the [0,1] / [0,1,2] -> [0,1,2] x64
    kernels from 4096 edges ([0,1]x32 -> [0,1,2]x64 is the first layer of
    config 4); an output with fewer slots than the kernels' is sliced after the
    pooling, and its gradient enters zero-padded."""
    print(f"pooled embedded {lin} -> {lout} cin={cin}", flush=True)
    layer, graph, P, Q, x, r, attn, gout = _setup(dev, lin, lout, cin, 64, 700, 6000, 8, 9)
    ref = _run(layer, graph, P, Q, x, r, attn, gout, 8, False)
    got = _run(layer, graph, P, Q, x, r, attn, gout, 8, True)
    for n, a, b in zip(["out", "grad_x", "grad_r", "grad_attn"], got[:4], ref[:4]):
        assert rel_err(a, b) < TOL, (n, rel_err(a, b))
    for a, b in zip(got[4], ref[4]):
        assert rel_err(a, b) < TOL


def test_pooled_deterministic_and_dispatch(dev):
    """Two runs give the same bits; the layer forms V only for the attention
    weights' gradient (none without it), and the scalar-output layout is left
    to the unfused path."""
    layer, graph, P, Q, x, r, attn, gout = _setup(dev, [0, 1, 2], [0, 1, 2], 64, 64, 300, 4000, 8, 11)
    a = _run(layer, graph, P, Q, x, r, attn, gout, 8, True)
    b = _run(layer, graph, P, Q, x, r, attn, gout, 8, True)
    for u, v in zip(a[:4], b[:4]):
        assert torch.equal(u, v)
    for u, v in zip(a[4], b[4]):
        assert torch.equal(u, v)
    with torch.no_grad():
        out = layer.attention_pool(P, Q, x.to(dev), r, graph, attn.to(dev), 8)
    assert rel_err(out, a[0]) < TOL
    torch.manual_seed(0)
    scalar = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1, 2], 64), fe.Repr([0], 8), num_bins=40).to(dev)
    P0, Q0 = fe.WignerDBasis([fe.Repr([0, 1, 2], 1), fe.Repr([0], 1)]).to(dev)(torch.randn(4000, 3, device=dev))
    assert scalar.attention_pool(P0, Q0, x.to(dev), r, graph, attn.to(dev)[:, :8], 8) is None


def test_attention_layer_takes_pooled_form(dev):
    """EquivariantAttention at [0,1,2]x64, 8 heads: the fused pooled form, and
    the same output and gradients as the unfused composition forced through
    edge_features = 0."""
    torch.manual_seed(21)
    rep = fe.Repr([0, 1, 2], 64)
    att = fe.EquivariantAttention(rep, rep, num_heads=8, distance_decay_scale=3.0).to(dev)
    g = torch.Generator().manual_seed(22)
    N, E = 256, 4096
    src = torch.randint(0, N, (E,), generator=g).to(dev)
    dst = torch.randint(0, N, (E,), generator=g).to(dev)
    graph = fe.Graph(src, dst, N)
    vec = (torch.randn(E, 3, generator=g) * 3).to(dev)
    (P,) = fe.WignerDBasis([rep]).to(dev)(vec)
    r = vec.norm(dim=-1)
    x = torch.randn(N, 64, 9, generator=g).to(dev)
    go = torch.randn(N, 64, 9, generator=g).to(dev)

    def run(edge_feats):
        xg = x.clone().requires_grad_(True)
        for p in att.parameters():
            p.grad = None
        out = att(P, P, xg, r, graph, edge_features=edge_feats)
        out.backward(go)
        return out.detach(), xg.grad, [p.grad.clone() for p in att.parameters()]

    fused = run(None)
    unfused = run(torch.zeros(E, 64, 9, device=dev))
    assert rel_err(fused[0], unfused[0]) < TOL
    assert rel_err(fused[1], unfused[1]) < 1e-5
    for a, b in zip(fused[2], unfused[2]):
        assert rel_err(a, b) < 1e-5
