"""A training step of the fused layer (message-passing form, sum-of-squares
loss, backward into node features and every parameter) captured in a HIP graph:
each replay, with eager work and synchronisations between replays, must give
the eager step's loss and gradients."""
import pytest
import torch

import flash_eq as fe
from flash_eq.capture import capture_step
from flash_eq.ops import SumSquaresFn
from helpers import rel_err

pytestmark = pytest.mark.gpu


def test_sum_squares_matches_torch(dev):
    g = torch.Generator().manual_seed(5)
    for n in (0, 1, 7, 1000, 3 * 1024 * 256 + 5, 9 * 1024 * 1024 * 4 + 3 * 1024 + 7):   # the last: 8-load steps
        y = torch.randn(n, generator=g).to(dev).requires_grad_(True)
        s = SumSquaresFn.apply(y)
        ref = (y.detach().double() ** 2).sum()
        assert abs(s.item() - ref.item()) <= 1e-6 * max(ref.item(), 1.0)
        s.backward()
        assert torch.equal(y.grad, 2 * y.detach())
    y = torch.randn(1001, generator=g).to(dev)[1:]          # not 16-byte aligned
    assert abs(SumSquaresFn.apply(y).item() - (y.double() ** 2).sum().item()) < 1e-3


def test_sum_squares_bf16(dev):
    """bfloat16 input: float32 squares and sums (8 values per 16-byte load), gradient 2y in bf16."""
    g = torch.Generator().manual_seed(6)
    for n in (0, 1, 9, 4001, 2 * 1024 * 256 * 8 + 13, 9 * 1024 * 1024 * 8 + 13):
        y = torch.randn(n, generator=g).to(dev, torch.bfloat16).requires_grad_(True)
        s = SumSquaresFn.apply(y)
        assert s.dtype == torch.float32
        ref = (y.detach().double() ** 2).sum()
        assert abs(s.item() - ref.item()) <= 1e-6 * max(ref.item(), 1.0)
        s.backward()
        assert y.grad.dtype == torch.bfloat16 and torch.equal(y.grad, 2 * y.detach())
    y = torch.randn(1003, generator=g).to(dev, torch.bfloat16)[3:]   # 6-byte offset: scalar loads
    assert abs(SumSquaresFn.apply(y).item() - (y.double() ** 2).sum().item()) < 1e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sum_squares_gradient(dev, dtype):
    """The loss and its gradient y * (2 g).to(y.dtype) for a non-unit upstream
    gradient, lengths with a scalar tail, unaligned (offset) inputs and an
    empty input; the loss within 1e-6 of the float64 sum."""
    g = torch.Generator().manual_seed(8)
    for n, off in ((0, 0), (5, 0), (1029, 0), (3 * 1024 * 256 * 8 + 11, 0), (4001, 3)):
        base = torch.randn(n + off, generator=g).to(dev, dtype)
        y = base[off:].clone().requires_grad_(True) if off == 0 else base[off:].detach().requires_grad_(True)
        s = SumSquaresFn.apply(y)
        ref_s = (y.detach().double() ** 2).sum().item()
        assert abs(s.item() - ref_s) <= 1e-6 * max(ref_s, 1.0), (n, off)
        up = torch.tensor(0.37, device=dev)
        s.backward(up)
        ref = y.detach() * (2.0 * up).to(dtype)
        assert y.grad.dtype == dtype and torch.equal(y.grad, ref), (n, off)


def test_captured_step_replays_match_eager(dev):
    torch.manual_seed(2)
    rep = fe.Repr([0, 1, 2], 64)
    layer = fe.EquivariantEdgewiseLinear(rep, rep, num_bins=100, max_dist=10.0).to(dev)
    g = torch.Generator().manual_seed(12)
    Nn, E = 400, 6000
    src = torch.randint(0, Nn, (E,), generator=g).to(dev)
    dst = torch.randint(0, Nn, (E,), generator=g).to(dev)
    vec = (torch.randn(E, 3, generator=g) * 3).to(dev)
    dist = vec.norm(dim=-1).clamp(max=10.0)
    (P,) = fe.WignerDBasis([rep]).to(dev)(vec)
    feats = torch.randn(Nn, 64, 9, generator=g).to(dev).requires_grad_(True)
    graph = fe.Graph(src, dst, Nn)
    graph.csr_src()
    leaves = [feats] + list(layer.parameters())

    def step():
        y = layer(P, P, feats, dist, graph=graph)
        loss = SumSquaresFn.apply(y)
        loss.backward()
        return loss

    for t in leaves:
        t.grad = None
    ref_loss = step().detach().clone()
    ref = [t.grad.clone() for t in leaves]

    cg, loss = capture_step(step, leaves)
    other = torch.randn(Nn, 64, 9, device=dev)
    for it in range(4):
        cg.replay()
        torch.cuda.synchronize()
        assert rel_err(loss, ref_loss) < 1e-6, it
        for t, r in zip(leaves, ref):
            assert rel_err(t.grad, r) < 1e-6, it
        # eager work between replays, on other inputs
        y2 = layer(P, P, other, dist, graph=graph)
        SumSquaresFn.apply(y2).item()


def test_captured_block_step_replays_match_eager(dev):
    """Config 3's transformer block ([0,1,2]x64, 8 heads, WignerDBasis inside the
    step) recorded in one HIP graph: every replay gives the eager step's loss and
    gradients (log_scale, LayerScale, norms, linear maps, radial net, features)."""
    torch.manual_seed(3)
    rep = fe.Repr([0, 1, 2], 64)
    block = fe.EquivariantTransformerBlock(rep, rep, num_heads=8, max_dist=10.0,
                                           distance_decay_scale=4.0).to(dev)
    with torch.no_grad():
        block.layer_scale_attn.gamma.fill_(0.5)
        block.layer_scale_mlp.gamma.fill_(0.5)
    basis = fe.WignerDBasis([rep]).to(dev)
    g = torch.Generator().manual_seed(13)
    Nn, E = 512, 8192
    src = torch.randint(0, Nn, (E,), generator=g).to(dev)
    dst = torch.randint(0, Nn, (E,), generator=g).to(dev)
    xyz = (torch.rand(Nn, 3, generator=g) * 12).to(dev)
    feats = torch.randn(Nn, 64, 9, generator=g).to(dev).requires_grad_(True)
    graph = fe.Graph(src, dst, Nn)
    graph.csr()
    graph.csr_src()
    leaves = [feats] + list(block.parameters())

    def step():
        vec = xyz[graph.src] - xyz[graph.dst]
        (P,) = basis(vec)
        out = block(P, P, feats, vec.norm(dim=-1), graph)
        loss = SumSquaresFn.apply(out)
        loss.backward()
        return loss

    for t in leaves:
        t.grad = None
    ref_loss = step().detach().clone()
    ref = [t.grad.clone() for t in leaves]
    names = ["features"] + [n for n, _ in block.named_parameters()]

    cg, loss = capture_step(step, leaves)
    other = torch.randn(Nn, 64, 9, device=dev)
    for it in range(4):
        cg.replay()
        torch.cuda.synchronize()
        assert rel_err(loss, ref_loss) < 1e-6, it
        for n, t, r in zip(names, leaves, ref):
            assert rel_err(t.grad, r) < 1e-5, (it, n)
        # eager work between replays, on other inputs
        with torch.no_grad():
            vec = xyz[graph.src] - xyz[graph.dst]
            (P2,) = basis(vec)
            SumSquaresFn.apply(block(P2, P2, other, vec.norm(dim=-1), graph)).item()


def test_captured_model_step_with_coordinate_gradients(dev):
    """A transformer step whose coordinates require grad (force training)
    recorded in one HIP graph: the edge vectors come from the graph's CSR
    gathers (their backward a fixed-order segmented sum, no index sort), the
    bases' gradients from the split kernels (grad_P, grad_Q) and the Wigner
    backward.  Every replay gives the eager step's loss and gradients for the
    coordinates, the features and the parameters."""
    torch.manual_seed(5)
    model = fe.EquivariantTransformer(fe.Repr([0, 1], 32), fe.Repr([0, 1, 2], 64), fe.Repr([0], 8),
                                      num_layers=2, num_heads=8, max_dist=10.0).to(dev)
    g = torch.Generator().manual_seed(17)
    Nn, E = 512, 8192
    src = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.randint(0, Nn, (E,), generator=g)
    dst = torch.where(dst == src, (dst + 1) % Nn, dst)   # no self-loops: |0|'s gradient is NaN
    src, dst = src.to(dev), dst.to(dev)
    xyz = (torch.rand(Nn, 3, generator=g) * 12).to(dev).requires_grad_(True)
    feats = torch.randn(Nn, 32, 4, generator=g).to(dev).requires_grad_(True)
    graph = fe.Graph(src, dst, Nn)
    graph.csr()
    graph.csr_src()
    leaves = [xyz, feats] + list(model.parameters())

    def step():
        loss = SumSquaresFn.apply(model(xyz, feats, graph))
        loss.backward()
        return loss

    for t in leaves:
        t.grad = None
    ref_loss = step().detach().clone()
    ref = [t.grad.clone() for t in leaves]
    names = ["coordinates", "features"] + [n for n, _ in model.named_parameters()]
    cg, loss = capture_step(step, leaves)
    for it in range(3):
        cg.replay()
        torch.cuda.synchronize()
        assert rel_err(loss, ref_loss) < 1e-6, it
        for n, t, r in zip(names, leaves, ref):
            assert rel_err(t.grad, r) < 1e-5, (it, n)
        with torch.no_grad():      # eager work between replays
            SumSquaresFn.apply(model(xyz + 0.5, feats, graph)).item()


@pytest.mark.parametrize("num_keys", [100, 50000])
def test_captured_csr_build_above_2pow20_edges(dev, num_keys):
    """The stable grouping by key (feq_csr_by_dst) recorded in a HIP graph at
    E = 1.3M > 2^20, the size above which the radix sort's default would switch
    to a form that records memset nodes: every replay, with eager work between
    replays, gives the stable argsort and the segment offsets (keys out of
    range sorted past the last one).  num_keys = 100 is the bin count of the
    radial-function gradient's sorted form; 50000 a node count."""
    from flash_eq import _native as N
    g = torch.Generator().manual_seed(31 + num_keys)
    E = 1_300_000
    keys = torch.randint(0, num_keys, (E,), generator=g)
    keys[torch.randint(0, E, (1000,), generator=g)] = -1
    keys[torch.randint(0, E, (1000,), generator=g)] = num_keys
    in_range = (keys >= 0) & (keys < num_keys)
    ref_perm = torch.argsort(torch.where(in_range, keys, num_keys), stable=True)
    counts = torch.bincount(keys[in_range], minlength=num_keys)
    ref_off = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    kd = keys.to(dev)
    lib = N.lib()
    ws = N.workspace(lib.feq_csr_workspace(E, num_keys), dev)
    perm = torch.full((E,), -7, dtype=torch.int32, device=dev)
    offsets = torch.full((num_keys + 1,), -7, dtype=torch.int32, device=dev)

    def build():
        rc = lib.feq_csr_by_dst(N.ptr(kd), E, num_keys, N.ptr(perm), N.ptr(offsets), N.ptr(ws),
                                ws.numel(), N.stream_ptr(dev))
        N.check(rc, "feq_csr_by_dst")

    build()
    torch.cuda.synchronize()
    assert torch.equal(perm.cpu().long(), ref_perm)
    assert torch.equal(offsets.cpu().long(), ref_off)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        build()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    cg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(cg):
        build()
    for it in range(4):
        perm.fill_(-7)
        offsets.fill_(-7)
        cg.replay()
        torch.cuda.synchronize()
        assert torch.equal(perm.cpu().long(), ref_perm), it
        assert torch.equal(offsets.cpu().long(), ref_off), it
        # eager work between replays: the same build on other keys
        kd2 = torch.randint(0, num_keys, (E,), device=dev)
        p2 = torch.empty(E, dtype=torch.int32, device=dev)
        o2 = torch.empty(num_keys + 1, dtype=torch.int32, device=dev)
        N.check(lib.feq_csr_by_dst(N.ptr(kd2), E, num_keys, N.ptr(p2), N.ptr(o2), N.ptr(ws),
                                   ws.numel(), N.stream_ptr(dev)), "feq_csr_by_dst")
        torch.cuda.synchronize()
        assert int(o2[-1]) == E, it
