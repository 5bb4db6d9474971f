"""The scalar-output kernels (csrc/edgewise_scalar.hip): EquivariantEdgewiseLinear
from [0,1,2]x64 to [0]xC (C = 8, 1), the value projection of a transformer's last
block when its output representation is scalar (the c4 model's [0]x8).

Parity with the float64 oracle (oracle/layer.py: bmm(x, P), the materialised
radial table, bmm(., Q^T)) at the float32 bar for the output and every
gradient, with Wigner-D bases and with dense ones; the message-passing form
against the gather form; determinism; and the launch log, which shows that the
dedicated kernels ran instead of the zero-embedded [0,1,2]x64 ones."""
import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from flash_eq import ops
from helpers import rel_err
from oracle import layer as OL
from oracle import wigner as OW
from test_gpu_edgewise import _run_parity

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(autouse=True)
def default_path(monkeypatch):
    monkeypatch.delenv("FEQ_EW_PATH", raising=False)
    monkeypatch.delenv("FEQ_FORCE_GENERIC", raising=False)


@pytest.mark.parametrize("cout", [8, 1])
@pytest.mark.parametrize("E", [1000, 37, 4003])
def test_scalar_output_parity(dev, cout, E):
    _run_parity(dev, [0, 1, 2], [0], cin=64, cout=cout, E=E, seed=E + cout)


def test_scalar_output_parity_log_bins(dev):
    _run_parity(dev, [0, 1, 2], [0], cin=64, cout=8, E=2003, seed=5, log=True, rmin=0.05)


def test_scalar_output_parity_dense_basis(dev):
    """Bases with entries off the degree blocks (the kernels take P's m = 0
    columns whole) and Q[0, 0] other than 1."""
    torch.manual_seed(12)
    layer = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1, 2], 64), fe.Repr([0], 8), num_bins=50).to(dev)
    E = 300
    g = torch.Generator().manual_seed(13)
    x = torch.randn(E, 64, 9, generator=g)
    P = torch.randn(E, 9, 9, generator=g) * 0.4
    Q = torch.randn(E, 1, 1, generator=g)
    r = torch.rand(E, generator=g) * 12
    xg = x.to(dev).requires_grad_(True)
    rg = r.to(dev).requires_grad_(True)
    y = layer(P.to(dev), Q.to(dev), xg, rg)
    params, cfg = OL.module_cfg(layer)
    xd, rd = x.double().requires_grad_(True), r.double().requires_grad_(True)
    yref = OL.edgewise_linear(xd, P.double(), Q.double(), rd, params, cfg)
    assert rel_err(y, yref) < TOL
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev))
    yref.backward(gy.double())
    assert rel_err(xg.grad, xd.grad) < TOL
    assert rel_err(rg.grad, rd.grad) < 1e-4
    for name, p in layer.radial_weights.named_parameters():
        assert rel_err(p.grad, params[name].grad) < TOL, name


def _mp_setup(dev, E, N, seed):
    g = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)
    layer = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1, 2], 64), fe.Repr([0], 8), num_bins=40).to(dev)
    src = torch.randint(0, N - 2, (E,), generator=g).to(dev)      # the last two nodes send nothing
    graph = fe.Graph(src, torch.randint(0, N, (E,), generator=g).to(dev), N)
    d = torch.randn(E, 3, generator=g).to(dev)
    P, Q = fe.WignerDBasis([fe.Repr([0, 1, 2], 1), fe.Repr([0], 1)]).to(dev)(d)
    x = torch.randn(N, 64, 9, generator=g).to(dev)
    r = (torch.rand(E, generator=g) * 11).to(dev)
    gy = torch.randn(E, 8, 1, generator=g).to(dev)
    return layer, graph, P, Q, x, r, gy


def _mp_run(layer, graph, P, Q, x, r, gy, fused):
    xg = x.clone().requires_grad_(True)
    rg = r.clone().requires_grad_(True)
    y = layer(P, Q, xg, rg, graph=graph) if fused else layer(P, Q, graph.gather_src(xg), rg)
    for p in layer.parameters():
        p.grad = None
    y.backward(gy)
    return [y.detach(), xg.grad, rg.grad] + [p.grad.clone() for p in layer.radial_weights.parameters()]


@pytest.mark.parametrize("E", [1000, 1037, 5])
def test_scalar_output_message_passing(dev, E):
    """Node sums inside the kernel (CSR-by-source tiles) against the gather form:
    the output, the distance and radial-function gradients per edge are the same
    bits; the node gradient and the channel patterns' gradient (summed in
    another edge order) agree to float32 rounding."""
    args = _mp_setup(dev, E, N=97, seed=E)
    layer = args[0]
    assert ops.edgewise_src_supported(layer.layout(), layer.binning(), layer.rank)
    a = _mp_run(*args, fused=True)
    b = _mp_run(*args, fused=False)
    assert torch.equal(a[0], b[0])
    assert rel_err(a[1], b[1]) < 1e-6
    assert torch.all(a[1][-2:] == 0)
    assert torch.equal(a[2], b[2])
    for ga, gb in zip(a[3:], b[3:]):
        assert rel_err(ga, gb) < 1e-6


def test_scalar_output_deterministic_and_dispatched(dev):
    args = _mp_setup(dev, 3000, N=200, seed=4)
    NAT.profile_summary()
    NAT.profile_enable(True)
    try:
        runs = [_mp_run(*args, fused=True) for _ in range(2)]
        torch.cuda.synchronize()
        names = NAT.profile_summary()
    finally:
        NAT.profile_enable(False)
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    for k in ("k_ew0_fwd", "k_ew0_bwd", "k_ews_node_fix"):
        assert k in names, (k, names)
    assert "k_ews_fwd" not in names and "k_ews_bwd_x" not in names, names


def test_scalar_output_out_of_range_rows_and_empty(dev):
    """Source indices outside [0, N) read zero rows (their edges output Q00 * 0 and
    scatter nothing); no edges gives empty outputs, zero radial gradients and
    zero node gradients.  Checked against the gather form with zero rows."""
    E, N = 400, 50
    layer, graph, P, Q, x, r, gy = _mp_setup(dev, E, N, seed=31)
    src = graph.src.clone()
    src[::7] = N + 5
    src[3::11] = -2
    g2 = fe.Graph(src, graph.dst, N)
    xg = x.clone().requires_grad_(True)
    y = layer(P, Q, xg, r, graph=g2)
    y.backward(gy)
    valid = (src >= 0) & (src < N)
    xz = torch.cat([x, torch.zeros(1, 64, 9, device=dev)])
    xr = xz[torch.where(valid, src, torch.full_like(src, N))].clone().requires_grad_(True)
    yref = layer(P, Q, xr, r)
    assert torch.equal(y, yref)
    yref.backward(gy)
    gref = torch.zeros_like(x).index_add_(0, src[valid], xr.grad[valid])
    assert rel_err(xg.grad, gref) < 1e-6
    # no edges
    e0 = torch.zeros(0, dtype=torch.long, device=dev)
    g0 = fe.Graph(e0, e0, N)
    x0 = x.clone().requires_grad_(True)
    for p in layer.parameters():
        p.grad = None
    y0 = layer(P[:0], Q[:0], x0, r[:0], graph=g0)
    assert y0.shape == (0, 8, 1)
    y0.sum().backward()
    assert torch.count_nonzero(x0.grad) == 0
    for p in layer.radial_weights.parameters():
        assert p.grad is None or torch.count_nonzero(p.grad) == 0
