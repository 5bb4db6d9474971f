"""The generic block-diagonal op (``feq_blockdiag_*``) beyond float32 parity:
float64 kernels, deterministic table gradients, the reference's pybind
interface (``flash_eq.cuda._pybind_compat``), float16 through that interface,
and sizes at which the per-bin table-gradient slices split the input channels.

float64 results are compared with the float64 oracle (``oracle/blockdiag.py``,
pinned by ``tests/test_oracle_blockdiag.py``) at 1e-12; float16 inputs are
computed in float32, compared on the same float16 values at 2e-3 (the output
rounding to float16).
"""
import pytest
import torch

import flash_eq as fe
from flash_eq.cuda import _pybind_compat as PB
from flash_eq.cuda import block_diagonal_cuda
from helpers import rel_err
from oracle import blockdiag as BD
from oracle.layout import dim_of, weight_dim

pytestmark = pytest.mark.gpu


def _case(lin, lout, cin, cout, nb, E, log, seed):
    g = torch.Generator().manual_seed(seed)
    b = BD.Binning.log(nb, 0.5, 10.0) if log else BD.Binning.linear(nb, 0.0, 10.0)
    x = torch.randn(E, cin, dim_of(lin), generator=g, dtype=torch.float64)
    T = torch.randn(nb + 1, cout, cin, weight_dim(lin, lout), generator=g, dtype=torch.float64)
    r = torch.rand(E, generator=g, dtype=torch.float64) * 12 + (0.3 if log else 0.0)
    gy = torch.randn(E, cout, dim_of(lout), generator=g, dtype=torch.float64)
    return b, x, T, r, gy


@pytest.mark.parametrize("lin,lout,log", [([0, 1, 2], [0, 1, 2], False), ([0, 1], [0, 1, 2], True),
                                          ([1, 2, 2], [0, 1], False), ([0, 1, 2, 3], [2, 3], True)])
def test_float64_matches_oracle(dev, lin, lout, log):
    b, x, T, r, gy = _case(lin, lout, 5, 6, 20, 400, log, seed=11)
    pr = fe.ProductRepr(fe.Repr(lin, 5), fe.Repr(lout, 6))
    xg, Tg, rg = (t.to(dev).requires_grad_(True) for t in (x, T, r))
    y = block_diagonal_cuda(xg, Tg, rg, pr, b.p1, b.p2, 20, log_bins=log, sh_scale=0.1)
    assert y.dtype == torch.float64
    yref = BD.forward(x, T, r, lin, lout, b)
    assert rel_err(y, yref) < 1e-12
    y.backward(gy.to(dev))
    gx, gt, gr = BD.backward(gy, x, T, r, lin, lout, b)
    assert rel_err(xg.grad, gx) < 1e-12
    assert rel_err(Tg.grad, gt) < 1e-12
    assert rel_err(rg.grad, gr) < 1e-9


def test_table_gradient_is_deterministic_and_bin_grouped(dev):
    """Two backward passes give the same bits; a bin no edge touches has a zero row."""
    b, x, T, r, gy = _case([0, 1, 2], [0, 1, 2], 16, 16, 30, 5000, False, seed=12)
    r = r.clamp(max=6.0)                         # rows 19..30 receive nothing
    pr = fe.ProductRepr(fe.Repr([0, 1, 2], 16), fe.Repr([0, 1, 2], 16))
    grads = []
    for _ in range(2):
        xg, Tg, rg = (t.float().to(dev).requires_grad_(True) for t in (x, T, r))
        y = block_diagonal_cuda(xg, Tg, rg, pr, b.p1, b.p2, 30, sh_scale=0.1)
        y.backward(gy.float().to(dev))
        grads.append((xg.grad.clone(), Tg.grad.clone(), rg.grad.clone()))
    for a, c in zip(*grads):
        assert torch.equal(a, c)
    assert grads[0][1][19:].abs().max() == 0
    _, gt, _ = BD.backward(gy, x, T, r, [0, 1, 2], [0, 1, 2], b)
    assert rel_err(grads[0][1], gt) < 1e-5


def test_table_gradient_slices_of_input_channels(dev):
    """Cin * Wdim beyond one workgroup's 4096 weights: slices over input channels."""
    lv = [0, 1, 2, 3]
    b, x, T, r, gy = _case(lv, lv, 300, 2, 8, 64, False, seed=13)
    pr = fe.ProductRepr(fe.Repr(lv, 300), fe.Repr(lv, 2))
    xg, Tg = x.to(dev).requires_grad_(True), T.to(dev).requires_grad_(True)
    y = block_diagonal_cuda(xg, Tg, r.to(dev), pr, b.p1, b.p2, 8, sh_scale=0.1)
    y.backward(gy.to(dev))
    gx, gt, _ = BD.backward(gy, x, T, r, lv, lv, b, need_dr=False)
    assert rel_err(Tg.grad, gt) < 1e-12 and rel_err(xg.grad, gx) < 1e-12


def _pb_args(lin, lout, b, nb, dev, log=False):
    li = torch.tensor(lin, dtype=torch.int32, device=dev)
    lo = torch.tensor(lout, dtype=torch.int32, device=dev)
    return 0.1, b.p1, b.p2, nb, log, li, lo


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.float64, 1e-12)])
def test_pybind_interface_matches_oracle(dev, dtype, tol):
    lin, lout, nb = [0, 1], [0, 1, 2], 20
    b, x, T, r, gy = _case(lin, lout, 4, 7, nb, 300, True, seed=14)
    sh, p1, p2, nbins, log, li, lo = _pb_args(lin, lout, b, nb, dev, log=True)
    xd, Td, rd, gd = (t.to(dev, dtype) for t in (x, T, r, gy))
    (y,) = PB.forward(xd, Td, rd, sh, p1, p2, nbins, log, li, lo, 7, dim_of(lout), 2)
    assert y.dtype == dtype and y.shape == (300, 7, 9)
    assert rel_err(y, BD.forward(x, T, r, lin, lout, b)) < tol
    gx, gt, gr = PB.backward(gd, xd, Td, rd, sh, p1, p2, nbins, log, li, lo, dim_of(lin), 2, 5)
    rx, rt, rr = BD.backward(gy, x, T, r, lin, lout, b)
    assert rel_err(gx, rx) < tol and rel_err(gt, rt) < tol
    assert rel_err(gr, rr) < (1e-4 if dtype == torch.float32 else 1e-9)


def test_pybind_interface_half_and_errors(dev):
    lin, lout, nb = [0, 1, 2], [0, 1, 2], 10
    b, x, T, r, gy = _case(lin, lout, 3, 3, nb, 200, False, seed=15)
    sh, p1, p2, nbins, log, li, lo = _pb_args(lin, lout, b, nb, dev)
    xh, Th, rh = (t.to(dev, torch.float16) for t in (x, T, r))
    (y,) = PB.forward(xh, Th, rh, sh, p1, p2, nbins, log, li, lo, 3, 9, 3)
    assert y.dtype == torch.float16
    ref = BD.forward(xh.double().cpu(), Th.double().cpu(), rh.double().cpu(), lin, lout, b)
    assert rel_err(y, ref) < 2e-3
    with pytest.raises(RuntimeError):          # bfloat16 is outside the reference's dispatch
        PB.forward(xh.bfloat16(), Th.bfloat16(), rh.bfloat16(), sh, p1, p2, nbins, log, li, lo, 3, 9, 3)
    with pytest.raises(RuntimeError):          # CHECK_INPUT: contiguous
        PB.forward(xh.transpose(1, 2), Th, rh, sh, p1, p2, nbins, log, li, lo, 3, 9, 3)
    with pytest.raises(RuntimeError):          # one dtype
        PB.forward(xh.float(), Th, rh, sh, p1, p2, nbins, log, li, lo, 3, 9, 3)
    with pytest.raises(RuntimeError):          # CUDA tensors
        PB.forward(xh.cpu(), Th, rh, sh, p1, p2, nbins, log, li, lo, 3, 9, 3)


def test_zero_edges(dev):
    lin = [0, 1]
    b, x, T, r, gy = _case(lin, lin, 2, 2, 5, 0, False, seed=16)
    pr = fe.ProductRepr(fe.Repr(lin, 2), fe.Repr(lin, 2))
    sh, p1, p2, nbins, log, li, lo = _pb_args(lin, lin, b, 5, dev)
    (y,) = PB.forward(x.to(dev), T.to(dev), r.to(dev), sh, p1, p2, nbins, log, li, lo, 2, 4, 2)
    assert y.shape == (0, 2, 4)
    gx, gt, gr = PB.backward(gy.to(dev), x.to(dev), T.to(dev), r.to(dev), sh, p1, p2, nbins, log, li,
                             lo, 4, 2, 2)
    assert gt.shape == T.shape and gt.abs().max() == 0
    assert block_diagonal_cuda(x.float().to(dev), T.float().to(dev), r.float().to(dev), pr, b.p1, b.p2,
                               5).shape == (0, 2, 4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_sh_scale_zero_like_patched_conv(dev, dtype):
    """PatchedConvSE3 (patch/_patched_conv.py:93-104) calls the op with sh_scale = 0.
    For r > 0 the solid-harmonic factor is r / r = 1 (no suppression); at r = 0 the
    reference's s = 0 / 0 is NaN, and its ipow(s, l_in + l_out) (block_diagonal.cu:202-219)
    is 1 for l_in + l_out = 0 and NaN otherwise.  With lvals_in = [0] and lvals_out =
    [0, 1] an r = 0 edge therefore has a finite l = 0 output, a NaN (l = 1, m = 0)
    output and zero (l = 1, m = +-1) outputs, which no m-block reaches (m-first slots
    0, 1, 2, 3)."""
    lin, lout, nb = [0], [0, 1], 12
    g = torch.Generator().manual_seed(18)
    b = BD.Binning.linear(nb, 0.0, 10.0, sigma=0.0)
    E = 200
    x = torch.randn(E, 3, 1, generator=g, dtype=torch.float64)
    T = torch.randn(nb + 1, 4, 3, weight_dim(lin, lout), generator=g, dtype=torch.float64)
    r = torch.rand(E, generator=g, dtype=torch.float64) * 12
    r[::17] = 0.0
    pr = fe.ProductRepr(fe.Repr(lin, 3), fe.Repr(lout, 4))
    y = block_diagonal_cuda(x.to(dev, dtype), T.to(dev, dtype), r.to(dev, dtype), pr, b.p1, b.p2, nb,
                            sh_scale=0.0).double().cpu()
    ref = BD.forward(x, T, r, lin, lout, b)
    zero = r == 0
    assert torch.isnan(ref[zero][..., 1]).all() and torch.isfinite(ref[zero][..., 0]).all()
    assert (ref[zero][..., 2:] == 0).all() and not torch.isnan(ref[~zero]).any()
    assert torch.equal(torch.isnan(y), torch.isnan(ref))
    fin = torch.isfinite(ref)
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    assert ((y[fin] - ref[fin]).abs().max() / ref[fin].abs().max()).item() < tol
    # r > 0: identical to the layer without suppression at all (s = 1)
    pos = ~zero
    ones = BD.forward(x[pos], T, r[pos], lin, lout, BD.Binning.linear(nb, 0.0, 10.0, sigma=1e-30))
    assert ((y[pos] - ones).abs().max() / ones.abs().max()).item() < tol
