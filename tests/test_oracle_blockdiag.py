"""Pins of the block-diagonal oracle (oracle/blockdiag.py, oracle/blockdiag_ref.c).

Independent checks, each able to catch a dropped term, sign or index slip:
* three forms agree: bin-grouped dense-per-m (torch), per-edge loops (C) and a
  per-edge dense Lambda brute force;
* the sign/layout convention: a dense m-first Lambda with [[a,b],[-b,a]]
  blocks, flattened with the extraction rule of patch/_conversion.py:99-140
  (a = Lambda[re_o, re_i], b = Lambda[re_o, im_i]), must act as Lambda itself;
* explicit gradients equal autograd of the forward (features, table) and
  central finite differences (distances, linear and log bins);
* t = 0 exactly at a bin edge reproduces row T[b]; r = 0 zeroes every l > 0
  output (test_self_loops.py:42-66) and makes dr NaN when an l>0 pair exists.
"""
import pytest
import torch

from oracle import blockdiag as BD
from oracle import cref
from oracle.layout import block_params, dim_of, weight_dim

CONFIGS = [([0, 1, 2], [0, 1, 2]), ([0, 1], [0, 1, 2]), ([1], [0, 1]), ([1, 2], [0, 1, 2]),
           ([0, 1, 2], [1, 2]), ([2], [0, 1, 2]), ([0, 1], [2]), ([0, 0], [0, 0]),
           ([1, 1], [1, 1]), ([0, 1, 1], [0, 1, 2]), ([1, 2, 2], [0, 1]), ([0, 2], [0, 2]),
           ([1, 2, 3], [1, 2, 3])]


def _case(lin, lout, E=24, cin=3, cout=4, nb=16, log=False, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    din, wd = dim_of(lin), weight_dim(lin, lout)
    b = BD.Binning.log(nb, 0.5, 10.0) if log else BD.Binning.linear(nb, 0.0, 10.0)
    x = torch.randn(E, cin, din, generator=g, dtype=dtype)
    T = torch.randn(nb + 1, cout, cin, wd, generator=g, dtype=dtype)
    r = torch.rand(E, generator=g, dtype=dtype) * 11.0 + (0.2 if log else 0.0)
    return x, T, r, b


@pytest.mark.parametrize("lin,lout", CONFIGS)
@pytest.mark.parametrize("log", [False, True])
def test_three_forms_agree(lin, lout, log):
    x, T, r, b = _case(lin, lout, log=log)
    y = BD.forward(x, T, r, lin, lout, b)
    yc = cref.forward(x, T, r, lin, lout, b)
    lam = BD.dense_lambda(T, r, lin, lout, b)
    yd = (lam @ x.reshape(x.shape[0], -1, 1)).reshape(y.shape)
    assert (y - yc).abs().max() < 1e-12 and (y - yd).abs().max() < 1e-12
    gy = torch.randn_like(y)
    g1 = BD.backward(gy, x, T, r, lin, lout, b)
    g2 = cref.backward(gy, x, T, r, lin, lout, b)
    for a, c in zip(g1, g2):
        assert (a - c).abs().max() < 1e-11 * (1 + c.abs().max())


@pytest.mark.parametrize("lin,lout", [([0, 1, 2], [0, 1, 2]), ([1, 2, 2], [0, 1]), ([0, 1], [2])])
def test_sign_convention_from_extraction_rule(lin, lout):
    """A dense m-first Lambda, flattened by the reference's extraction rule, acts as itself."""
    g = torch.Generator().manual_seed(11)
    cin, cout, nb = 2, 3, 4
    din, dout, wd = dim_of(lin), dim_of(lout), weight_dim(lin, lout)
    lam = torch.zeros(cout, dout, cin, din, dtype=torch.float64)
    row = torch.zeros(cout, cin, wd, dtype=torch.float64)
    for (m, ni, no, ioff, ooff, woff) in block_params(lin, lout):
        for o in range(no):
            for i in range(ni):
                a = torch.randn(cout, cin, generator=g, dtype=torch.float64)
                if m == 0:
                    lam[:, ooff + o, :, ioff + i] = a
                    row[:, :, woff + o * ni + i] = lam[:, ooff + o, :, ioff + i]
                else:
                    bb = torch.randn(cout, cin, generator=g, dtype=torch.float64)
                    ro, io, ri, ii = ooff + 2 * o, ooff + 2 * o + 1, ioff + 2 * i, ioff + 2 * i + 1
                    lam[:, ro, :, ri], lam[:, ro, :, ii] = a, bb
                    lam[:, io, :, ri], lam[:, io, :, ii] = -bb, a
                    # extraction (patch/_conversion.py:129-132): a = re/re, b = re/im
                    row[:, :, woff + 2 * (o * ni + i)] = lam[:, ro, :, ri]
                    row[:, :, woff + 2 * (o * ni + i) + 1] = lam[:, ro, :, ii]
    T = row.unsqueeze(0).repeat(nb + 1, 1, 1, 1)
    b = BD.Binning(0.0, nb / 10.0, nb, False, 0.0)     # sigma = 0: scale 1 for r > 0
    x = torch.randn(7, cin, din, generator=g, dtype=torch.float64)
    r = torch.rand(7, generator=g, dtype=torch.float64) * 9 + 0.5
    y = BD.forward(x, T, r, lin, lout, b)
    ref = torch.einsum("odci,eci->eod", lam, x)
    assert (y - ref).abs().max() < 1e-12
    assert (cref.forward(x, T, r, lin, lout, b) - ref).abs().max() < 1e-12


@pytest.mark.parametrize("lin,lout", [([0, 1, 2], [0, 1, 2]), ([1, 2], [0, 1]), ([0, 1, 1], [0, 1, 2])])
def test_explicit_grads_match_autograd(lin, lout):
    x, T, r, b = _case(lin, lout, E=12)
    xg = x.clone().requires_grad_(True)
    Tg = T.clone().requires_grad_(True)
    y = BD.forward(xg, Tg, r, lin, lout, b)
    gy = torch.randn_like(y)
    (y * gy).sum().backward()
    gx, gt, _ = BD.backward(gy, x, T, r, lin, lout, b)
    assert (gx - xg.grad).abs().max() < 1e-11
    assert (gt - Tg.grad).abs().max() < 1e-11


@pytest.mark.parametrize("log", [False, True])
def test_distance_grad_finite_differences(log):
    lin, lout = [0, 1, 2], [0, 1]
    x, T, r, b = _case(lin, lout, E=20, log=log, seed=5)
    # keep away from bin edges and from the log clamp region
    lo, t, _ = BD.bin_state(r, b)
    r = torch.where((t > 0.05) & (t < 0.95), r, r + 0.3 / (b.num_bins / 10.0))
    lo, t, _ = BD.bin_state(r, b)
    keep = (t > 0.05) & (t < 0.95) & (r > 0.6)
    x, r = x[keep], r[keep]
    y = BD.forward(x, T, r, lin, lout, b)
    gy = torch.randn_like(y)
    _, _, gr = BD.backward(gy, x, T, r, lin, lout, b)
    h = 1e-6
    fd = ((BD.forward(x, T, r + h, lin, lout, b) - BD.forward(x, T, r - h, lin, lout, b)) * gy
          ).sum((1, 2)) / (2 * h)
    assert (gr - fd).abs().max() < 1e-5 * (1 + fd.abs().max())


def test_bin_edge_reproduces_row():
    lin, lout = [0, 1, 2], [0, 1, 2]
    x, T, _, b = _case(lin, lout, E=10, nb=10)
    r = torch.tensor([1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0, 9.0, 3.0], dtype=torch.float64)
    lo, t, _ = BD.bin_state(r, b)
    assert torch.equal(lo, torch.tensor([1, 2, 3, 4, 5, 6, 7, 8, 9, 3])) and (t == 0).all()
    y = BD.forward(x, T, r, lin, lout, b)
    for e in range(10):
        Te = T[lo[e]].unsqueeze(0).repeat(T.shape[0], 1, 1, 1)
        ye = BD.forward(x[e:e + 1], Te, r[e:e + 1], lin, lout, b)
        assert (y[e:e + 1] - ye).abs().max() < 1e-13


def test_zero_distance_suppresses_higher_l_and_nan_grad():
    lin, lout = [0, 1, 2], [0, 1, 2]
    x, T, r, b = _case(lin, lout, E=6)
    r[0] = 0.0
    y = BD.forward(x, T, r, lin, lout, b)
    assert y[0, :, 3:].abs().max() == 0 and y[0, :, :3].abs().max() > 0   # slots 0..2 are m=0
    # m=0 slots of l>0 irreps: slot 1 (l=1), slot 2 (l=2) also vanish
    assert y[0, :, 1:3].abs().max() == 0 and y[0, :, 0].abs().max() > 0
    _, _, gr = BD.backward(torch.randn_like(y), x, T, r, lin, lout, b)
    assert torch.isnan(gr[0]) and torch.isfinite(gr[1:]).all()
    _, _, gr0 = BD.backward(*[torch.randn(6, 4, 1, dtype=torch.float64)],
                            *_case([0], [0], E=6)[:1], _case([0], [0], E=6)[1],
                            torch.zeros(6, dtype=torch.float64), [0], [0], b)
    assert torch.isfinite(gr0).all()


def test_empty_edges():
    x, T, r, b = _case([0, 1], [0, 1, 2], E=0)
    assert BD.forward(x, T, r, [0, 1], [0, 1, 2], b).shape == (0, 4, 9)


def test_linear_extrapolation_unclamped():
    b = BD.Binning.linear(10, 0.0, 10.0)
    r = torch.tensor([12.5, -0.5, 10.0], dtype=torch.float64)
    lo, t, dtdr = BD.bin_state(r, b)
    assert lo.tolist() == [9, 0, 9]
    assert torch.allclose(t, torch.tensor([3.5, -0.5, 1.0], dtype=torch.float64))
    assert (dtdr == 1.0).all()


def test_c_binning_matches_python_binning():
    for b in (BD.Binning.linear(100, 0.0, 10.0), BD.Binning.log(50, 0.5, 10.0)):
        r = torch.cat([torch.rand(5000, dtype=torch.float64) * 14 - 1, torch.linspace(0, 10, 101,
                                                                                    dtype=torch.float64)])
        lo, t, _ = BD.bin_state(r, b)
        lo_c, t_c = cref.binning(r, b)
        assert torch.equal(lo.to(torch.int32), lo_c)
        assert (t - t_c).abs().max() < 1e-12
