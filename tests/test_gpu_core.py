"""GPU parity of the core kernels against the oracle (through the C ABI).

Bars: bit-exact for bin indices and graph index sets; <= 1e-5 relative
(max|a-b| / max|ref|) for float32 results against the float64 oracle.
"""
import math

import pytest
import torch

import flash_eq as fe
from flash_eq import _native as N
from flash_eq import ops
from flash_eq.cuda import block_diagonal_cuda
from helpers import rel_err
from oracle import blockdiag as BD
from oracle import graphops as G
from oracle import wigner as OW
from oracle.layout import dim_of, weight_dim

pytestmark = pytest.mark.gpu
TOL = 1e-5


# ---------------------------------------------------------------- binning --
def test_linear_bins_bit_exact(dev):
    g = torch.Generator().manual_seed(0)
    r = torch.cat([torch.rand(200000, generator=g) * 14 - 2, torch.linspace(0, 10, 1001),
                   torch.tensor([0.0, 10.0, 9.999999, 1e-30, -0.0])])
    for nb, lo_v, hi_v in ((100, 0.0, 10.0), (64, 0.0, 10.0), (50, 0.5, 7.0)):
        b = BD.Binning.linear(nb, lo_v, hi_v)
        lo_ref, t_ref, _ = BD.bin_state(r, b)
        lo, t = ops.bin_edges(r.to(dev), N.make_binning(b.p1, b.p2, nb, False, 0.1))
        assert torch.equal(lo.cpu().long(), lo_ref)
        # t agrees to float32 rounding: the GPU fuses p1 + lo*width into one FMA (as nvcc
        # does by default), so the bin edge may differ by 1 ulp, i.e. t by ulp(edge)/width
        width = (hi_v - lo_v) / nb
        bound = 2 * 2.0 ** -23 * max(abs(lo_v), abs(hi_v)) / width + 1e-6
        assert ((t.cpu() - t_ref).abs() / t_ref.abs().clamp(min=1.0)).max() < bound


def test_log_bins_bit_exact(dev):
    """Log-bin indices bit for bit: the kernels and the oracle both take float32
    log/exp rounded from float64, so the index depends on the float32 inputs
    alone; includes distances exactly at (and one ulp either side of) bin edges."""
    g = torch.Generator().manual_seed(1)
    r = torch.rand(200000, generator=g) * 12
    b = BD.Binning.log(50, 0.5, 10.0)
    edges = torch.exp(torch.linspace(math.log(0.5), math.log(10.0), 51, dtype=torch.float64)).float()
    r = torch.cat([r, edges, torch.nextafter(edges, edges + 1), torch.nextafter(edges, edges - 1),
                   torch.tensor([0.0, 0.49, 0.5, 10.0, 11.0])])
    lo_ref, t_ref, _ = BD.bin_state(r, b)
    lo, t = ops.bin_edges(r.to(dev), N.make_binning(b.p1, b.p2, 50, True, 0.1))
    assert torch.equal(lo.cpu().long(), lo_ref.long())
    assert (t.cpu() - t_ref).abs().max() < 1e-5


# ---------------------------------------------------------------- wigner ---
@pytest.mark.parametrize("lvals", [[0, 1, 2], [0, 1], [0], [1, 2, 2], list(range(7)), [3, 0, 5]])
def test_wigner_basis_matches_matrix_exp(dev, lvals):
    g = torch.Generator().manual_seed(2)
    d = torch.randn(3000, 3, generator=g) * 4
    d[:6] = torch.tensor([[0.0, 0.0, 0.0], [0.0, 0.0, -1.0], [0.0, 0.0, 3.0], [1e-7, 0.0, -1.0],
                          [0.0, 1e-6, 1.0], [2.0, -1.0, 0.0]])
    ref = OW.basis(lvals, d)
    out = fe.WignerDBasis([fe.Repr(lvals, 3)])(d.to(dev))[0]
    assert out.dtype == torch.float32 and out.shape == ref.shape
    assert (out.cpu().double() - ref).abs().max().item() < 1e-5


def test_wigner_basis_dedup_and_order(dev):
    d = torch.randn(100, 3)
    a, b, c = fe.WignerDBasis([fe.Repr([0, 1], 2), fe.Repr([0, 1, 2], 4), fe.Repr([0, 1], 8)])(d.to(dev))
    assert a is c and b.shape == (100, 9, 9)
    ref = OW.basis([0, 1, 2], d)
    assert (b.cpu().double() - ref).abs().max() < 1e-5


def test_wigner_basis_empty(dev):
    (m,) = fe.WignerDBasis([fe.Repr([0, 1, 2])])(torch.zeros(0, 3, device=dev))
    assert m.shape == (0, 9, 9)


# ------------------------------------------------------- generic block op --
CONFIGS = [([0, 1, 2], [0, 1, 2]), ([0, 1], [0, 1, 2]), ([1], [0, 1]), ([1, 2], [0, 1, 2]),
           ([0, 1, 2], [1, 2]), ([2], [0, 1, 2]), ([0, 1], [2]), ([0, 0], [0, 0]),
           ([1, 1], [1, 1]), ([0, 1, 1], [0, 1, 2]), ([1, 2, 2], [0, 1]), ([0, 2], [0, 2]),
           ([1, 2, 3], [1, 2, 3])]


@pytest.mark.parametrize("lin,lout", CONFIGS)
@pytest.mark.parametrize("log", [False, True])
def test_block_diagonal_op_parity(dev, lin, lout, log):
    g = torch.Generator().manual_seed(3)
    E, cin, cout, nb = 300, 5, 6, 20
    din, wd = dim_of(lin), weight_dim(lin, lout)
    b = BD.Binning.log(nb, 0.5, 10.0) if log else BD.Binning.linear(nb, 0.0, 10.0)
    x = torch.randn(E, cin, din, generator=g)
    T = torch.randn(nb + 1, cout, cin, wd, generator=g)
    r = torch.rand(E, generator=g) * 12 + (0.3 if log else 0.0)
    pr = fe.ProductRepr(fe.Repr(lin, cin), fe.Repr(lout, cout))
    xg, Tg, rg = (t.to(dev).requires_grad_(True) for t in (x, T, r))
    y = block_diagonal_cuda(xg, Tg, rg, pr, b.p1, b.p2, nb, log_bins=log, sh_scale=0.1)
    yref = BD.forward(x.double(), T.double(), r.double(), lin, lout, b)
    assert rel_err(y, yref) < TOL
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev))
    gx, gt, gr = BD.backward(gy.double(), x.double(), T.double(), r.double(), lin, lout, b)
    assert rel_err(xg.grad, gx) < TOL
    assert rel_err(Tg.grad, gt) < TOL
    # the distance gradient of an edge is a sum of Cout*Cin*Wdim signed terms that
    # largely cancel, so its float32 rounding relative to its own size is ~1e-5
    assert rel_err(rg.grad, gr) < 1e-4


# ------------------------------------------------------------------ graph --
def _kat(name):
    import json, os
    return json.load(open(os.path.join(os.path.dirname(__file__), "golden", "pooling_kat.json")))[name]


@pytest.mark.parametrize("reduce", ["sum", "mean", "max"])
def test_pooling_known_answers(dev, reduce):
    c = _kat(reduce)
    dst = torch.tensor(c["dst"], device=dev)
    g = fe.Graph(torch.zeros_like(dst), dst, c["num_nodes"])
    out = fe.GraphPooling(reduce)(torch.tensor(c["x"], device=dev), g)
    assert torch.equal(out.cpu(), torch.tensor(c["expected"]))


def test_pooling_edge_cases(dev):
    pool = fe.GraphPooling("sum")
    g0 = fe.Graph(torch.zeros(0, dtype=torch.long, device=dev), torch.zeros(0, dtype=torch.long, device=dev), 5)
    out = pool(torch.zeros(0, 4, 9, device=dev), g0)
    assert out.shape == (5, 4, 9) and (out == 0).all()
    c = _kat("single")
    dst = torch.tensor(c["dst"], device=dev)
    out = pool(torch.tensor(c["x"], device=dev), fe.Graph(torch.zeros_like(dst), dst, 5))
    assert torch.equal(out.cpu(), torch.tensor(c["expected"]))
    x = torch.ones(100, 2, 3, device=dev)
    z = torch.zeros(100, dtype=torch.long, device=dev)
    out = pool(x, fe.Graph(z, z, 10))
    assert (out[0] == 100).all() and (out[1:] == 0).all()


def test_csr_index_sets_bit_exact(dev):
    g = torch.Generator().manual_seed(4)
    dst = torch.randint(0, 977, (50000,), generator=g)
    graph = fe.Graph(torch.zeros_like(dst).to(dev), dst.to(dev), 1000)
    perm, offsets = graph.csr()
    ref_perm = torch.argsort(dst, stable=True)
    counts = torch.bincount(dst, minlength=1000)
    ref_off = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    assert torch.equal(perm.cpu().long(), ref_perm)
    assert torch.equal(offsets.cpu().long(), ref_off)


def test_sum_pooling_random_and_grad(dev):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(20000, 16, 9, generator=g)
    dst = torch.randint(0, 700, (20000,), generator=g)
    graph = fe.Graph(dst.to(dev), dst.to(dev), 700)
    xg = x.to(dev).requires_grad_(True)
    out = fe.GraphPooling("sum")(xg, graph)
    assert rel_err(out, G.pool_sum(x.double(), dst, 700)) < TOL
    go = torch.randn(out.shape, generator=g)
    out.backward(go.to(dev))
    assert torch.equal(xg.grad.cpu(), go[dst])


def test_edge_softmax_parity_and_sum_to_one(dev):
    g = torch.Generator().manual_seed(6)
    E, H, Dh, Nn = 6000, 8, 12, 300
    Q = torch.randn(E, H, Dh, generator=g)
    K = torch.randn(E, H, Dh, generator=g)
    r = torch.rand(E, generator=g) * 8
    dst = torch.randint(0, Nn, (E,), generator=g)
    graph = fe.Graph(dst.to(dev), dst.to(dev), Nn)
    att = fe.EquivariantEdgeAttention(num_heads=H, qk_dim=Dh, distance_decay_scale=3.0).to(dev)
    Qg, Kg, rg = Q.to(dev).requires_grad_(True), K.to(dev).requires_grad_(True), r.to(dev).requires_grad_(True)
    a = att.attention_weights(Qg, Kg, graph, rg)
    Qd, Kd, rd = (t.double().requires_grad_(True) for t in (Q, K, r))
    ls = att.log_scale.detach().double().cpu().requires_grad_(True)
    aref = G.neighbour_softmax(G.edge_logits(Qd, Kd, ls, rd, 3.0), dst, Nn)
    assert rel_err(a, aref) < TOL
    sums = torch.zeros(Nn, H, dtype=torch.float64).index_add(0, dst, a.detach().cpu().double())
    has = torch.bincount(dst, minlength=Nn) > 0
    assert (sums[has] - 1).abs().max() < 1e-5
    ga = torch.randn(E, H, generator=g)
    a.backward(ga.to(dev))
    aref.backward(ga.double())
    assert rel_err(Qg.grad, Qd.grad) < TOL
    assert rel_err(Kg.grad, Kd.grad) < TOL
    assert rel_err(rg.grad, rd.grad) < TOL
    assert rel_err(att.log_scale.grad, ls.grad) < TOL


@pytest.mark.parametrize("row_shape", [(64, 9), (3, 5), (4,), (3,), (17,)])
def test_gather_src_dst_and_grad(dev, row_shape):
    """Graph.gather_src / gather_dst equal x[src] / x[dst] exactly; their backward
    (segmented sums over the cached CSRs) matches a float64 index_add, including
    nodes without edges.  (64, 9) and (4,) rows take the 16-byte kernels, rows
    of at most 16 other floats (coordinates) a row per thread, (17,) the
    workgroup-per-row kernels."""
    g = torch.Generator().manual_seed(21)
    N, E = 37, 400
    src = torch.randint(0, N - 3, (E,), generator=g)      # the last nodes have no edges
    dst = torch.randint(0, N, (E,), generator=g)
    graph = fe.Graph(src.to(dev), dst.to(dev), N)
    x = torch.randn(N, *row_shape, generator=g)
    for which, idx in (("src", src), ("dst", dst)):
        xg = x.to(dev).requires_grad_(True)
        out = graph.gather_src(xg) if which == "src" else graph.gather_dst(xg)
        assert torch.equal(out.detach().cpu(), x[idx]), which
        gout = torch.randn(out.shape, generator=g)
        out.backward(gout.to(dev))
        ref = torch.zeros((N,) + tuple(row_shape), dtype=torch.float64).index_add_(0, idx, gout.double())
        assert rel_err(xg.grad, ref) < 1e-6, which
        assert torch.all(xg.grad[N - 3:].cpu() == 0) or which == "dst"
