"""GPU parity of the fused EquivariantEdgewiseLinear against the float64 oracle.

The oracle composes bmm(x, P) -> block-diagonal mix with the materialised
SeparableRadialNet table (explicit reference backward) -> bmm(., Q^T); the
product runs one fused HIP kernel per direction with the separable factors.
Gradients compared: edge features, distances, P, Q and every radial-network
parameter.  Equivariance is reported with the reference's metric.
"""
import pytest
import torch

import flash_eq as fe
from helpers import equivariance_err, rel_err
from oracle import layer as OL
from oracle import wigner as OW

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _inputs(lin, lout, E, cin, seed, rmax=12.0, rmin=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(E, cin, sum(2 * l + 1 for l in lin), generator=g)
    d = torch.randn(E, 3, generator=g)
    r = torch.rand(E, generator=g) * (rmax - rmin) + rmin
    gy_seed = torch.Generator().manual_seed(seed + 1)
    return x, d, r, gy_seed


def _run_parity(dev, lin, lout, cin, cout, E, seed=0, log=False, grad_pq=False, rmin=0.0, rvals=None,
                rank=4):
    torch.manual_seed(seed)
    kw = dict(log_bins=True, min_dist=0.5) if log else {}
    layer = fe.EquivariantEdgewiseLinear(fe.Repr(lin, cin), fe.Repr(lout, cout), num_bins=50, rank=rank, **kw)
    x, d, r, g = _inputs(lin, lout, E, cin, seed, rmin=rmin)
    if rvals is not None:      # distances drawn from a few values: neighbouring edges share bins
        r = torch.tensor(rvals)[torch.randint(len(rvals), (E,), generator=g)]
    P = OW.basis(lin, d).float()
    Q = OW.basis(lout, d).float()
    layer = layer.to(dev)
    xg = x.to(dev).requires_grad_(True)
    rg = r.to(dev).requires_grad_(True)
    Pg = P.to(dev).requires_grad_(grad_pq)
    Qg = Q.to(dev).requires_grad_(grad_pq)
    y = layer(Pg, Qg, xg, rg)
    params, cfg = OL.module_cfg(layer)
    xd, rd = x.double().requires_grad_(True), r.double().requires_grad_(True)
    Pd, Qd = P.double().requires_grad_(grad_pq), Q.double().requires_grad_(grad_pq)
    yref = OL.edgewise_linear(xd, Pd, Qd, rd, params, cfg)
    assert y.shape == yref.shape
    assert rel_err(y, yref) < TOL, rel_err(y, yref)
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev))
    yref.backward(gy.double())
    assert rel_err(xg.grad, xd.grad) < TOL
    assert rel_err(rg.grad, rd.grad) < 1e-4
    for name, p in layer.radial_weights.named_parameters():
        assert rel_err(p.grad, params[name].grad) < TOL, name
    if grad_pq:
        assert rel_err(Pg.grad, Pd.grad) < TOL
        assert rel_err(Qg.grad, Qd.grad) < TOL


@pytest.mark.parametrize("lin,lout", [([0, 1, 2], [0, 1, 2]), ([0, 1], [0, 1, 2]), ([1, 2], [0, 1]),
                                      ([0, 1, 1], [0, 1, 2]), ([1, 2, 2], [0, 1]), ([2], [0, 1, 2]),
                                      ([0], [0]), ([1, 2, 3], [1, 2, 3])])
def test_edgewise_parity(dev, lin, lout):
    _run_parity(dev, lin, lout, cin=6, cout=5, E=400)


PATHS = ("split", "generic")


def _select(monkeypatch, path):
    """Kernel family of the fused layer: split-fp16 MFMA (default) or generic."""
    monkeypatch.delenv("FEQ_FORCE_GENERIC", raising=False)
    if path == "split":
        monkeypatch.delenv("FEQ_EW_PATH", raising=False)
    else:
        monkeypatch.setenv("FEQ_EW_PATH", path)


@pytest.fixture(params=PATHS)
def impl(request, monkeypatch):
    _select(monkeypatch, request.param)
    return request.param


def test_edgewise_parity_c1_shape(dev, impl):
    """BASELINE config 1 layer shape: [0,1]x32 -> [0,1,2]x64, E=500."""
    _run_parity(dev, [0, 1], [0, 1, 2], cin=32, cout=64, E=500, seed=1)


def test_edgewise_parity_c2_shape(dev, impl):
    """BASELINE config 2 layer shape ([0,1,2]x64, num_bins=100 range) at a reduced E."""
    _run_parity(dev, [0, 1, 2], [0, 1, 2], cin=64, cout=64, E=1500, seed=2)


def test_edgewise_parity_c2_ragged_tiles(dev, impl):
    """E not a multiple of the 16-edge tile; permuted lvals with the c2 dimensions."""
    _run_parity(dev, [0, 1, 2], [0, 1, 2], cin=64, cout=64, E=4003, seed=8)
    _run_parity(dev, [2, 0, 1], [1, 2, 0], cin=64, cout=64, E=37, seed=9)


def test_kernel_families_agree_at_scale(dev, monkeypatch):
    """c2 shape at E = 40,000: the split-fp16 path against the generic kernels."""
    torch.manual_seed(3)
    rp = fe.Repr([0, 1, 2], 64)
    layer = fe.EquivariantEdgewiseLinear(rp, rp).to(dev)
    E = 40000
    g = torch.Generator().manual_seed(10)
    (P,) = fe.WignerDBasis([rp]).to(dev)(torch.randn(E, 3, generator=g).to(dev))
    x = torch.randn(E, 64, 9, generator=g).to(dev)
    r = (torch.rand(E, generator=g) * 11).to(dev)
    gy = torch.randn(E, 64, 9, generator=g).to(dev)
    outs = {}
    for mode in PATHS:
        _select(monkeypatch, mode)
        layer.zero_grad()
        xg, rg = x.clone().requires_grad_(True), r.clone().requires_grad_(True)
        y = layer(P, P, xg, rg)
        y.backward(gy)
        outs[mode] = (y.detach(), xg.grad, rg.grad,
                      [p.grad.clone() for p in layer.radial_weights.parameters()])
    b = outs["generic"]
    for mode in ("split",):
        a = outs[mode]
        assert rel_err(a[0], b[0]) < 2e-6 and rel_err(a[1], b[1]) < 2e-6, mode
        assert rel_err(a[2], b[2]) < 2e-5, mode
        for pa, pb in zip(a[3], b[3]):
            assert rel_err(pa, pb) < 2e-5, mode


@pytest.mark.parametrize("path", PATHS)
def test_backward_is_deterministic(dev, monkeypatch, path):
    """Two backward passes give the same bits on either kernel family (the
    radial-function gradient is binned and the channel-pattern partials summed
    in a fixed order; no atomics)."""
    _select(monkeypatch, path)
    torch.manual_seed(5)
    rp = fe.Repr([0, 1, 2], 16)
    layer = fe.EquivariantEdgewiseLinear(rp, rp, num_bins=20).to(dev)
    g = torch.Generator().manual_seed(6)
    E = 3000
    (P,) = fe.WignerDBasis([rp]).to(dev)(torch.randn(E, 3, generator=g).to(dev))
    x = torch.randn(E, 16, 9, generator=g).to(dev)
    r = (torch.rand(E, generator=g) * 9).to(dev)
    gy = torch.randn(E, 16, 9, generator=g).to(dev)
    runs = []
    for _ in range(2):
        layer.zero_grad()
        xg, rg = x.clone().requires_grad_(True), r.clone().requires_grad_(True)
        layer(P, P, xg, rg).backward(gy)
        runs.append([xg.grad, rg.grad] + [p.grad.clone() for p in layer.radial_weights.parameters()])
    for a, b in zip(*runs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("lin,lout,cin,cout,E", [([0, 1, 2], [0, 1, 2], 64, 64, 1000),
                                                 ([0, 1], [0, 1, 2], 32, 64, 1000)])
def test_split_path_is_dispatched(dev, monkeypatch, lin, lout, cin, cout, E):
    """The default forward of the compiled shapes runs the split-fp16 kernel."""
    from flash_eq import _native as NAT
    _select(monkeypatch, "split")
    layer = fe.EquivariantEdgewiseLinear(fe.Repr(lin, cin), fe.Repr(lout, cout)).to(dev)
    g = torch.Generator().manual_seed(11)
    d = torch.randn(E, 3, generator=g).to(dev)
    P, Q = fe.WignerDBasis([fe.Repr(lin, 1), fe.Repr(lout, 1)]).to(dev)(d)
    x = torch.randn(E, cin, P.shape[-1], generator=g).to(dev).requires_grad_(True)
    r = (torch.rand(E, generator=g) * 9).to(dev)
    torch.cuda.synchronize()
    NAT.profile_summary()
    NAT.profile_enable(True)
    y = layer(P, Q, x, r)
    y.backward(torch.ones_like(y))
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    names = NAT.profile_summary()
    assert "k_ews_fwd" in names and "k_ews_prep" in names, names
    if cin % 64 == 0:
        assert "k_ews_bwd_x" in names and "k_ews_bwd_c" in names, names


@pytest.mark.parametrize("lin,lout,cin,cout", [([0, 1, 2], [0, 1, 2], 64, 64), ([0, 1], [0, 1, 2], 32, 64)])
def test_edgewise_parity_general_basis(dev, lin, lout, cin, cout):
    """P and Q need not be Wigner-D matrices: tiles whose matrices have entries off
    the degree blocks take the dense rotations, the others the block-sparse ones."""
    torch.manual_seed(12)
    layer = fe.EquivariantEdgewiseLinear(fe.Repr(lin, cin), fe.Repr(lout, cout), num_bins=50)
    E = 100
    x, d, r, g = _inputs(lin, lout, E, cin, 12)
    P = OW.basis(lin, d).float()
    Q = OW.basis(lout, d).float()
    gen = torch.Generator().manual_seed(13)
    for lo, hi in ((16, 32), (70, 71)):          # one full dense tile, one tile with a single edge
        P[lo:hi] = torch.randn(hi - lo, *P.shape[1:], generator=gen) * 0.4
        Q[lo:hi] = torch.randn(hi - lo, *Q.shape[1:], generator=gen) * 0.4
    layer = layer.to(dev)
    xg = x.to(dev).requires_grad_(True)
    y = layer(P.to(dev), Q.to(dev), xg, r.to(dev))
    params, cfg = OL.module_cfg(layer)
    xd = x.double().requires_grad_(True)
    yref = OL.edgewise_linear(xd, P.double(), Q.double(), r.double(), params, cfg)
    assert rel_err(y, yref) < TOL, rel_err(y, yref)
    gy = torch.randn(y.shape, generator=g)
    y.backward(gy.to(dev))
    yref.backward(gy.double())
    assert rel_err(xg.grad, xd.grad) < TOL
    for name, p in layer.radial_weights.named_parameters():
        assert rel_err(p.grad, params[name].grad) < TOL, name


def test_edgewise_parity_log_bins(dev):
    _run_parity(dev, [0, 1, 2], [0, 1], cin=8, cout=8, E=600, seed=3, log=True, rmin=0.1)


@pytest.mark.parametrize("lin,cin", [([0, 1, 2], 64), ([0, 1], 32)])
def test_edgewise_parity_log_bins_split_kernels(dev, monkeypatch, lin, cin):
    """Logarithmic bins through the split-fp16 kernels (c1/c2 layouts), with
    distances below min_dist and beyond max_dist; the launch log shows that the
    split kernels ran."""
    from flash_eq import _native as NAT
    _select(monkeypatch, "split")
    NAT.profile_summary()
    NAT.profile_enable(True)
    try:
        _run_parity(dev, lin, [0, 1, 2], cin=cin, cout=64, E=2003, seed=21, log=True, rmin=0.05)
        torch.cuda.synchronize()
        names = NAT.profile_summary()
    finally:
        NAT.profile_enable(False)
    assert "k_ews_fwd" in names, names
    if cin % 64 == 0:
        assert "k_ews_bwd_x" in names and "k_ews_bwd_c" in names, names


def test_edgewise_grad_wrt_basis(dev):
    _run_parity(dev, [0, 1], [0, 1, 2], cin=4, cout=3, E=200, seed=4, grad_pq=True)


def test_edgewise_empty_and_single_edge(dev):
    r4 = fe.Repr([0, 1, 2], 4)
    layer = fe.EquivariantEdgewiseLinear(r4, r4).to(dev)
    P = torch.zeros(0, 9, 9, device=dev)
    out = layer(P, P, torch.zeros(0, 4, 9, device=dev), torch.zeros(0, device=dev))
    assert out.shape == (0, 4, 9)
    _run_parity(dev, [0, 1, 2], [0, 1, 2], cin=4, cout=4, E=1, seed=5)


def test_zero_distance_self_loop(dev):
    """r = 0: l>0 outputs vanish (test_self_loops.py:42-66), dr is NaN like the reference."""
    torch.manual_seed(6)
    r4 = fe.Repr([0, 1, 2], 4)
    layer = fe.EquivariantEdgewiseLinear(r4, r4).to(dev)
    E = 8
    d = torch.randn(E, 3)
    P = OW.basis([0, 1, 2], d).float().to(dev)
    x = torch.randn(E, 4, 9, device=dev)
    r = torch.rand(E, device=dev) * 5 + 0.5
    r[0] = 0.0
    rg = r.clone().requires_grad_(True)
    y = layer(P, P, x, rg)
    assert y[0, :, 1:].abs().max() < 1e-6 and y[0, :, 0].abs().max() > 1e-3
    (y ** 2).sum().backward()
    assert torch.isnan(rg.grad[0]) and torch.isfinite(rg.grad[1:]).all()


@pytest.mark.parametrize("rvals,rank", [(None, 4), ([2.0, 2.1, 2.3, 7.3], 4), (None, 3)])
def test_binned_gradient_many_edges_per_wave(dev, rvals, rank):
    """E large enough that each wave of the binned radial-function gradient adds
    several whole batches of edges and a partial one.  Rank 4 gives c2's rows
    (K * wdim = 76 columns, lanes on column pairs); rank 3 an odd row of 57
    (a lane per column).  With clustered distances neighbouring edges mostly
    fall in the same or adjacent bins."""
    _run_parity(dev, [0, 1, 2], [0, 1, 2], cin=8, cout=8, E=40000, seed=11, rvals=rvals, rank=rank)


def test_out_of_range_distances_extrapolate(dev):
    _run_parity(dev, [0, 1], [0, 1], cin=4, cout=4, E=300, seed=7)   # r up to 12 > max_dist 10


@pytest.mark.parametrize("lin,lout", [([0, 1, 2], [0, 1, 2]), ([0, 1], [0, 1, 2]), ([1, 2, 2], [0, 1])])
def test_equivariance(dev, lin, lout):
    """Reference protocol (test_equivariance.py:47-99): rotate inputs and directions."""
    torch.manual_seed(42)
    mult, N, E = 4, 20, 50
    rin, rout = fe.Repr(lin, mult), fe.Repr(lout, mult)
    layer = fe.EquivariantEdgewiseLinear(rin, rout, num_bins=50).to(dev)
    basis = fe.WignerDBasis([rin, rout]).to(dev)
    nf = torch.randn(N, mult, rin.dim(), device=dev)
    src = torch.randint(0, N, (E,), device=dev)
    r = torch.rand(E, device=dev) * 5
    dirs = torch.randn(E, 3, device=dev)
    dirs = dirs / dirs.norm(dim=-1, keepdim=True)
    axis, angle = fe.random_rotation(device=dev)
    D_in = fe.WignerD(rin).to(dev).rot(axis, angle)
    D_out = fe.WignerD(rout).to(dev).rot(axis, angle)
    R = fe.WignerD(fe.Repr([1])).to(dev).rot(axis, angle, cartesian=True)
    P, Q = basis(dirs)
    out1 = torch.einsum("ij,ecj->eci", D_out, layer(P, Q, nf[src], r))
    P2, Q2 = basis(dirs @ R.T)
    out2 = layer(P2, Q2, torch.einsum("ij,ncj->nci", D_in, nf)[src], r)
    err = equivariance_err(out1, out2)
    print(f"equivariance error {lin}->{lout}: {err:.2e}")
    assert err < 1e-4


def test_gradient_equivariance(dev):
    torch.manual_seed(101)
    lv, mult, N, E = [0, 1, 2], 4, 10, 30
    rp = fe.Repr(lv, mult)
    layer = fe.EquivariantEdgewiseLinear(rp, rp, num_bins=50).to(dev)
    basis = fe.WignerDBasis([rp]).to(dev)
    axis, angle = fe.random_rotation(device=dev)
    D = fe.WignerD(rp).to(dev).rot(axis, angle)
    R = fe.WignerD(fe.Repr([1])).to(dev).rot(axis, angle, cartesian=True)
    src = torch.randint(0, N, (E,), device=dev)
    r = torch.rand(E, device=dev) * 5
    dirs = torch.randn(E, 3, device=dev)
    (P,) = basis(dirs)
    nf = torch.randn(N, mult, 9, device=dev, requires_grad=True)
    (layer(P, P, nf[src], r) ** 2).sum().backward()
    g1 = torch.einsum("ij,ncj->nci", D, nf.grad)
    nf2 = torch.einsum("ij,ncj->nci", D, nf.detach()).requires_grad_(True)
    (P2,) = basis(dirs @ R.T)
    (layer(P2, P2, nf2[src], r) ** 2).sum().backward()
    assert equivariance_err(g1, nf2.grad) < 1e-4


def test_distance_gradient_finite_difference(dev):
    """dL/dr vs central differences (test_equivariance.py:324-395 protocol), linear and log bins."""
    for log in (False, True):
        torch.manual_seed(123)
        rp = fe.Repr([0, 1], 2)
        kw = dict(log_bins=True, min_dist=0.5) if log else {}
        layer = fe.EquivariantEdgewiseLinear(rp, rp, num_bins=50, max_dist=10.0, **kw).to(dev)
        E = 10
        (P,) = fe.WignerDBasis([rp]).to(dev)(torch.randn(E, 3, device=dev))
        x = torch.randn(E, 2, 4, device=dev)
        r = torch.rand(E, device=dev) * 5.0 + (0.5 if log else 0.0) + 0.5
        rg = r.clone().requires_grad_(True)
        (layer(P, P, x, rg) ** 2).sum().backward()
        eps = 1e-3
        fd = torch.zeros(E, device=dev)
        with torch.no_grad():
            for i in range(E):
                rp_, rm_ = r.clone(), r.clone()
                rp_[i] += eps
                rm_[i] -= eps
                fd[i] = ((layer(P, P, x, rp_) ** 2).sum() - (layer(P, P, x, rm_) ** 2).sum()) / (2 * eps)
        rel = ((rg.grad - fd).abs() / (fd.abs() + 1e-8)).max().item()
        assert rel < 0.10, (log, rel)
