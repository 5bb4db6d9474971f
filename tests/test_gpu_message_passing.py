"""The message-passing form of the fused layer: layer(P, Q, x, r, graph=graph)
reads row src[e] of the node table inside the kernels (feq_edgewise_fwd_src)
and sums the input gradient per source node inside the input-gradient kernel
(feq_edgewise_bwd_src_nodes, walking the CSR by source).

It does the same per-edge arithmetic on the same values as layer(P, Q,
graph.gather_src(x), r), whose parity with the float64 oracle
test_gpu_edgewise.py checks, so the output and the radial and distance
gradients agree bit for bit.  The node gradient sums the same per-edge rows in
CSR order, through one partial sum per 16-edge tile for nodes whose edges cross
a tile boundary, so it agrees to float32 rounding (1e-6) and is itself the same
on every run.  The reference gathers with x[src] before the layer
(layers/attention.py:307-310).
"""
import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from flash_eq import ops
from helpers import rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def split_kernels(monkeypatch):
    """Every test starts on the default (split-fp16) kernel family."""
    monkeypatch.delenv("FEQ_EW_PATH", raising=False)
    monkeypatch.delenv("FEQ_FORCE_GENERIC", raising=False)


def _setup(dev, lin, lout, cin, cout, N, E, seed):
    g = torch.Generator().manual_seed(seed)
    src = torch.randint(0, N - 2, (E,), generator=g)          # the last two nodes send nothing
    dst = torch.randint(0, N, (E,), generator=g)
    torch.manual_seed(seed)
    layer = fe.EquivariantEdgewiseLinear(fe.Repr(lin, cin), fe.Repr(lout, cout), num_bins=40).to(dev)
    d = torch.randn(E, 3, generator=g).to(dev)
    P, Q = fe.WignerDBasis([fe.Repr(lin, 1), fe.Repr(lout, 1)]).to(dev)(d)
    x = torch.randn(N, cin, P.shape[-1], generator=g)
    r = (torch.rand(E, generator=g) * 11).to(dev)
    gy = torch.randn(E, cout, Q.shape[-1], generator=g).to(dev)
    return layer, fe.Graph(src.to(dev), dst.to(dev), N), P, Q, x, r, gy


def _run(layer, graph, P, Q, x, r, gy, fused):
    dev = P.device
    xg = x.to(dev).requires_grad_(True)
    rg = r.clone().requires_grad_(True)
    y = layer(P, Q, xg, rg, graph=graph) if fused else layer(P, Q, graph.gather_src(xg), rg)
    for p in layer.parameters():
        p.grad = None
    y.backward(gy)
    grads = [p.grad.clone() for p in layer.radial_weights.parameters()]
    return y.detach(), xg.grad, rg.grad, grads


@pytest.mark.parametrize("E", [1000, 1037, 5])
@pytest.mark.parametrize("lin,lout,cin,cout", [([0, 1, 2], [0, 1, 2], 64, 64),
                                               ([0, 1], [0, 1, 2], 32, 64)])
def test_message_passing_matches_gather(dev, lin, lout, cin, cout, E):
    """Bit-identical to gather + layer, ragged last tiles and nodes without
    outgoing edges included.  [0,1]x32 has forward kernels only, so the whole op
    falls back to the gather; its backward then runs the generic kernels, whose
    radial-function gradient is summed with float atomics (run-to-run order), so
    the radial-parameter gradients are compared to 1e-6 there."""
    args = _setup(dev, lin, lout, cin, cout, N=97, E=E, seed=E + cin)
    layer = args[0]
    fused = ops.edgewise_src_supported(layer.layout(), layer.binning(), layer.rank)
    assert fused == (cin == 64)
    a = _run(*args, fused=True)
    b = _run(*args, fused=False)
    assert torch.equal(a[0], b[0])
    assert torch.equal(a[1], b[1]) if not fused else rel_err(a[1], b[1]) < 1e-6
    assert torch.all(a[1][-2:] == 0)
    assert torch.equal(a[2], b[2]) if fused else rel_err(a[2], b[2]) < 1e-6
    for ga, gb in zip(a[3], b[3]):
        assert torch.equal(ga, gb) if fused else rel_err(ga, gb) < 1e-6


def test_message_passing_dispatch(dev):
    """[0,1,2]x64 runs the split kernels with the gather inside: no gather kernel
    forward; backward, the node sums inside the input-gradient kernel and its
    fix-up pass (no separate segmented sum)."""
    layer, graph, P, Q, x, r, gy = _setup(dev, [0, 1, 2], [0, 1, 2], 64, 64, N=97, E=1000, seed=3)
    assert ops.edgewise_src_supported(layer.layout(), layer.binning(), layer.rank)
    graph.csr_src()
    torch.cuda.synchronize()
    NAT.profile_summary()
    NAT.profile_enable(True)
    _run(layer, graph, P, Q, x, r, gy, fused=True)
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    names = NAT.profile_summary()
    assert "k_gather_rows" not in names and "k_segment_sum" not in names, names
    for k in ("k_ews_fwd", "k_ews_bwd_x", "k_ews_bwd_c", "k_ews_node_fix"):
        assert k in names, (k, names)


@pytest.mark.parametrize("case", ["hub", "sparse", "ragged"])
def test_node_sums_inside_the_kernel(dev, case):
    """Out-degrees that exercise every path of the per-node sums: a hub node
    whose 70 edges span five tiles, nodes with one edge, nodes without edges,
    runs that start and end inside a tile, and a ragged last tile.  The node
    gradient equals the float64 sum of the per-edge gradients (from the
    per-edge entry point) to float32 rounding, and two runs give the same bits."""
    g = torch.Generator().manual_seed({"hub": 1, "sparse": 2, "ragged": 3}[case])
    N = 61
    if case == "hub":
        src = torch.cat([torch.full((70,), 7), torch.randint(0, N, (230,), generator=g)])
    elif case == "sparse":
        src = torch.arange(0, N, 2).repeat(3)[:77]          # odd nodes send nothing
    else:
        src = torch.randint(0, 5, (16 * 9 + 5,), generator=g)   # five busy nodes, ragged end
    E = src.numel()
    src = src[torch.randperm(E, generator=g)]
    dst = torch.randint(0, N, (E,), generator=g)
    torch.manual_seed(9)
    layer = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1, 2], 64), fe.Repr([0, 1, 2], 64), num_bins=40).to(dev)
    d = torch.randn(E, 3, generator=g).to(dev)
    (P,) = fe.WignerDBasis([fe.Repr([0, 1, 2], 1)]).to(dev)(d)
    x = torch.randn(N, 64, 9, generator=g).to(dev)
    r = (torch.rand(E, generator=g) * 11).to(dev)
    gy = torch.randn(E, 64, 9, generator=g).to(dev)
    graph = fe.Graph(src.to(dev), dst.to(dev), N)
    runs = []
    for _ in range(2):
        xg = x.clone().requires_grad_(True)
        layer(P, P, xg, r, graph=graph).backward(gy)
        runs.append(xg.grad)
    assert torch.equal(runs[0], runs[1])
    # per-edge gradients from the dense form, summed per source node in float64
    xe = x[src.to(dev)].requires_grad_(True)
    layer(P, P, xe, r).backward(gy)
    ref = torch.zeros(N, 64, 9, dtype=torch.float64, device=dev)
    ref.index_add_(0, src.to(dev), xe.grad.double())
    assert rel_err(runs[0], ref) < 1e-6
    deg = torch.bincount(src, minlength=N).to(dev)
    assert torch.all(runs[0][deg == 0] == 0)


def test_message_passing_out_of_range_rows_read_zero(dev):
    """Source indices outside [0, N) read zero rows (as feq_gather_rows): output
    and radial gradient equal those of an explicit table with a zero row for them
    bit for bit; the channel-pattern kernel drops such edges instead of zeroing
    their rows (their rows still enter its per-column fp16 scales), so its
    gradient agrees to fp32 accuracy."""
    layer, graph, P, Q, x, r, gy = _setup(dev, [0, 1, 2], [0, 1, 2], 64, 64, N=97, E=1000, seed=4)
    N = x.shape[0]
    src = graph.src.clone()
    src[::7] = -1
    src[3::11] = N + 5
    bad = (src < 0) | (src >= N)
    perm, offsets = fe.Graph(torch.where(bad, torch.zeros_like(src), src), graph.dst, N).csr_src()
    xd = x.to(dev)
    rw = layer.radial_weights
    C, F = rw.channel_patterns, rw.radial_functions()
    L, B = layer.layout(), layer.binning()

    y = ops.edgewise_linear_src(xd, src, perm, offsets, P, Q, r, C, F, L, B, rw.rank)
    gC, gF = torch.autograd.grad(y, [C, F], gy)
    x_ext = torch.cat([xd, torch.zeros_like(xd[:1])])
    rows = torch.where(bad, torch.full_like(src, N), src)
    # with grad_x requested, so that the reference also runs the split kernels
    xe = x_ext[rows].contiguous().requires_grad_(True)
    y_ref = ops.edgewise_linear(xe, P, Q, r, C, F, L, B, rw.rank)
    gC_ref, gF_ref, _ = torch.autograd.grad(y_ref, [C, F, xe], gy)
    assert torch.equal(y, y_ref)
    assert rel_err(gC, gC_ref) < 1e-6
    assert torch.equal(gF, gF_ref)


def test_message_passing_fallback(dev, monkeypatch):
    """With the split kernels switched off (FEQ_EW_PATH=generic) the layer
    gathers first and runs the generic kernels: same results within fp32
    tolerance."""
    args = _setup(dev, [0, 1, 2], [0, 1, 2], 64, 64, N=97, E=300, seed=5)
    a = _run(*args, fused=True)
    monkeypatch.setenv("FEQ_EW_PATH", "generic")
    layer = args[0]
    assert not ops.edgewise_src_supported(layer.layout(), layer.binning(), layer.rank)
    b = _run(*args, fused=True)
    assert rel_err(a[0], b[0]) < 1e-5
    assert rel_err(a[1], b[1]) < 1e-5
    for ga, gb in zip(a[3], b[3]):
        assert rel_err(ga, gb) < 1e-5
