"""Block-diagonal radial mix, forward and backward (oracle, torch on CPU).

Restates the semantics of ``flash_eq/cuda/csrc/block_diagonal.cu``:

* binning            -- ``compute_binning`` / ``binning_derivative`` (``.cu:82-138``);
* solid-harmonic scale ``s = r/(r+sigma)``, weight scaled by ``s^(l_in+l_out)``
                        (``.cu:202-232, 307-372``);
* forward            -- ``forward_m0_kernel`` / ``forward_mpos_kernel`` (``.cu:558-733``);
* backward           -- ``backward_features_*`` and ``backward_table_*`` (``.cu:747-1161``),
                        including the distance-gradient quirks (log bins use
                        ``1/(edge_hi-edge_lo)`` even where t is clamped; NaN at r=0
                        whenever an l>0 pair exists).

Form: *bin-grouped dense per-m blocks*.  For every m-block the radial table
row of bin b is expanded into the dense real matrix ``L_m[b]`` that acts on the
block's (channel, slot) vector (the inverse of ``_extract_block_diagonal_weights``,
``patch/_conversion.py:99-140``: re/re = a, re/im = b, im/re = -b, im/im = a).
Edges are grouped by their lower bin and every group is two GEMMs.  This is
the timed CPU baseline; it runs in the dtype of its inputs.

Pinned by ``tests/test_oracle_blockdiag.py``: agreement with the C per-edge
restatement (``oracle/blockdiag_ref.c``) and with a per-edge dense brute force;
``torch.autograd.gradcheck`` of the features/table gradients; finite
differences of the distance gradient; t=0 at bin edges reproducing T[b]; r=0
zeroing every l>0 output; a hand-built dense Lambda extracted with the
reference's layout rules.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Sequence

import numpy as np
import torch

from .layout import block_l, block_params, dim_of, weight_dim


@dataclass
class Binning:
    """Kernel binning parameters; p1/p2/sigma are float32 on the kernel side (``.cu:72-76``)."""
    p1: float
    p2: float
    num_bins: int
    log_bins: bool = False
    sigma: float = 0.1

    @staticmethod
    def linear(num_bins: int, min_val: float = 0.0, max_val: float = 10.0, sigma: float = 0.1) -> "Binning":
        return Binning(min_val, num_bins / (max_val - min_val), num_bins, False, sigma)

    @staticmethod
    def log(num_bins: int, min_val: float, max_val: float, sigma: float = 0.1) -> "Binning":
        """``SeparableRadialNet.binning_params`` for log spacing (``radial.py:230-232, 277-281``)."""
        log_min = float(torch.tensor(min_val).log())
        inv = 1.0 / float(torch.tensor(max_val / min_val).log())
        return Binning(log_min, inv, num_bins, True, sigma)


def _f32(x: float) -> np.float32:
    return np.float32(x)


def bin_state(r: torch.Tensor, b: Binning):
    """(lo, t, dt/dr) per edge, with the float32 index path of ``compute_binning``.

    ``normalized`` is float32; ``lo = min(floor(clamp(normalized,0,nb)), nb-1)``;
    ``t`` is computed in the dtype of ``r`` and, for linear bins, is not clamped.
    """
    dt = r.dtype
    rf = r.detach().cpu().numpy().astype(np.float32)
    p1, p2, nb = _f32(b.p1), _f32(b.p2), b.num_bins
    with np.errstate(all="ignore"):
        if b.log_bins:
            # float32 log/exp rounded from float64 (correctly rounded), as the
            # kernels form them; CUDA's logf/expf (<= 1 ulp) can differ from
            # these in the last bit, moving r within one float32 ulp of a bin
            # edge to the neighbouring bin
            lo_edge = np.float32(np.exp(np.float64(p1)))
            lg = np.log(np.maximum(rf, lo_edge).astype(np.float64)).astype(np.float32)
            norm = ((lg - p1) * p2) * np.float32(nb)
        else:
            norm = (rf - p1) * p2
        norm = np.minimum(np.maximum(norm, np.float32(0.0)), np.float32(nb))
        lo = np.minimum(np.floor(norm).astype(np.int64), nb - 1)
    lo_t = torch.from_numpy(lo)
    rr = r.detach()
    if b.log_bins:
        inv_lbw = torch.tensor(float(p2 * np.float32(nb)), dtype=dt)
        log_lo = torch.tensor(float(p1), dtype=dt) + lo_t.to(dt) / inv_lbw
        e_lo = torch.exp(log_lo.double()).to(dt)
        e_hi = torch.exp((log_lo + 1.0 / inv_lbw).double()).to(dt)
        t = (torch.maximum(rr, e_lo) - e_lo) / (e_hi - e_lo)
        t = torch.minimum(t, torch.ones_like(t))
        dtdr = 1.0 / (e_hi - e_lo)
    else:
        width = 1.0 / torch.tensor(float(p2), dtype=dt)
        e_lo = torch.tensor(float(p1), dtype=dt) + lo_t.to(dt) * width
        t = (rr - e_lo) / width
        dtdr = torch.full_like(t, float(p2))
    return lo_t, t, dtdr


def _sigma(b: Binning, dtype) -> torch.Tensor:
    return torch.tensor(float(_f32(b.sigma)), dtype=dtype)


def lambda_blocks(table: torch.Tensor, lvals_in, lvals_out):
    """Dense per-m matrices ``L[m]`` of shape (nb+1, Cout*k*n_out, Cin*k*n_in), k = 1|2.

    Row index (co, o, c_out), column index (ci, i, c_in); c = 0 for the +m
    (re) component and 1 for -m (im).
    """
    nbp1, cout, cin, wd = table.shape
    out = []
    for (m, n_in, n_out, in_off, out_off, w_off) in block_params(lvals_in, lvals_out):
        if m == 0:
            idx = w_off + (torch.arange(n_out)[:, None] * n_in + torch.arange(n_in)[None, :])
            blk = table[..., idx]                           # (b, co, ci, o, i)
            blk = blk.permute(0, 1, 3, 2, 4)                 # (b, co, o, ci, i)
            out.append(blk.reshape(nbp1, cout * n_out, cin * n_in))
        else:
            base = w_off + 2 * (torch.arange(n_out)[:, None] * n_in + torch.arange(n_in)[None, :])
            a = table[..., base]                             # (b, co, ci, o, i)
            bb = table[..., base + 1]
            z = torch.zeros(nbp1, cout, cin, n_out, n_in, 2, 2, dtype=table.dtype)
            z[..., 0, 0] = a
            z[..., 0, 1] = bb
            z[..., 1, 0] = -bb
            z[..., 1, 1] = a
            z = z.permute(0, 1, 3, 5, 2, 4, 6)               # (b, co, o, c_out, ci, i, c_in)
            out.append(z.reshape(nbp1, cout * n_out * 2, cin * n_in * 2))
    return out


def _slot_powers(s: torch.Tensor, ls: List[int], k: int) -> torch.Tensor:
    """(E, len(ls)*k) matrix of s^l for every slot of a block (c fastest)."""
    cols = []
    for l in ls:
        cols += [s ** l] * k
    return torch.stack(cols, -1)


class _Prep:
    def __init__(self, x, table, r, lvals_in, lvals_out, b: Binning):
        self.E, self.cin, self.din = x.shape
        _, self.cout, cin2, self.wdim = table.shape
        assert cin2 == self.cin and self.din == dim_of(lvals_in)
        assert self.wdim == weight_dim(lvals_in, lvals_out)
        self.dout = dim_of(lvals_out)
        self.blocks = block_params(lvals_in, lvals_out)
        self.lo, self.t, self.dtdr = bin_state(r, b)
        sig = _sigma(b, r.dtype)
        self.s = r / (r + sig)
        self.deriv = sig / (r * (r + sig))
        self.lam = lambda_blocks(table, lvals_in, lvals_out)
        self.lin = [block_l(lvals_in, m) for (m, *_r) in self.blocks]
        self.lout = [block_l(lvals_out, m) for (m, *_r) in self.blocks]
        self.has_lpos = max(int(l) for l in lvals_in) + max(int(l) for l in lvals_out) > 0

    def block_in(self, x, j):
        m, n_in, n_out, in_off, out_off, w_off = self.blocks[j]
        k = 1 if m == 0 else 2
        f = x[:, :, in_off:in_off + k * n_in]               # (E, Cin, k n_in)
        return f, k, n_in, n_out, in_off, out_off

    def groups(self):
        order = torch.argsort(self.lo, stable=True)
        lo_sorted = self.lo[order]
        uniq, counts = torch.unique_consecutive(lo_sorted, return_counts=True)
        start = 0
        for b, c in zip(uniq.tolist(), counts.tolist()):
            yield b, order[start:start + c]
            start += c


def forward(x, table, r, lvals_in, lvals_out, b: Binning) -> torch.Tensor:
    """``out[e] = Lambda(r_e) x[e]`` in the m-first basis; returns (E, Cout, Dout)."""
    p = _Prep(x, table, r, lvals_in, lvals_out, b)
    y = torch.zeros(p.E, p.cout, p.dout, dtype=x.dtype)
    if p.E == 0:
        return y
    for j in range(len(p.blocks)):
        f, k, n_in, n_out, in_off, out_off = p.block_in(x, j)
        fs = (f * _slot_powers(p.s, p.lin[j], k)[:, None, :]).reshape(p.E, -1)
        yb = torch.zeros(p.E, p.cout * n_out * k, dtype=x.dtype)
        for bin_lo, idx in p.groups():
            t = p.t[idx][:, None]
            lo_m, hi_m = p.lam[j][bin_lo], p.lam[j][bin_lo + 1]
            fe = fs[idx]
            yb[idx] = (1 - t) * (fe @ lo_m.T) + t * (fe @ hi_m.T)
        yb = yb.reshape(p.E, p.cout, n_out * k) * _slot_powers(p.s, p.lout[j], k)[:, None, :]
        y[:, :, out_off:out_off + k * n_out] = yb
    return y


def backward(gy, x, table, r, lvals_in, lvals_out, b: Binning, need_dr: bool = True):
    """(grad_features, grad_table, grad_distances) with the reference's formulas."""
    p = _Prep(x, table, r, lvals_in, lvals_out, b)
    gx = torch.zeros_like(x)
    gt = torch.zeros_like(table)
    gr = torch.zeros_like(r)
    if p.E == 0:
        return gx, gt, gr
    term_t = torch.zeros_like(r)
    term_s = torch.zeros_like(r)
    for j, (m, n_in, n_out, in_off, out_off, w_off) in enumerate(p.blocks):
        f, k, *_ = p.block_in(x, j)
        pin = _slot_powers(p.s, p.lin[j], k)
        pout = _slot_powers(p.s, p.lout[j], k)
        lin_w = torch.tensor([l for l in p.lin[j] for _ in range(k)], dtype=x.dtype)
        lout_w = torch.tensor([l for l in p.lout[j] for _ in range(k)], dtype=x.dtype)
        fs3 = f * pin[:, None, :]
        fs = fs3.reshape(p.E, -1)
        g3 = gy[:, :, out_off:out_off + k * n_out] * pout[:, None, :]
        gs = g3.reshape(p.E, -1)
        dlam = torch.zeros_like(p.lam[j])
        gfb = torch.zeros(p.E, p.cin * n_in * k, dtype=x.dtype)
        yu = torch.zeros(p.E, p.cout * n_out * k, dtype=x.dtype)
        for bin_lo, idx in p.groups():
            t = p.t[idx][:, None]
            lo_m, hi_m = p.lam[j][bin_lo], p.lam[j][bin_lo + 1]
            ge, fe = gs[idx], fs[idx]
            glo, ghi = ge @ lo_m, ge @ hi_m
            gfb[idx] = (1 - t) * glo + t * ghi
            dlam[bin_lo] += ((1 - t) * ge).T @ fe
            dlam[bin_lo + 1] += (t * ge).T @ fe
            ylo, yhi = fe @ lo_m.T, fe @ hi_m.T
            yu[idx] = (1 - t) * ylo + t * yhi
            term_t[idx] += (ge * (yhi - ylo)).sum(-1)
        # scale-derivative term: sum over (row, col) of (l_row + l_col) gs W fs
        term_s += (gs.reshape(p.E, p.cout, -1) * yu.reshape(p.E, p.cout, -1) * lout_w).sum((1, 2))
        term_s += (fs3 * gfb.reshape(p.E, p.cin, -1) * lin_w).sum((1, 2))
        gx[:, :, in_off:in_off + k * n_in] = gfb.reshape(p.E, p.cin, -1) * pin[:, None, :]
        _scatter_dlam(gt, dlam, m, n_in, n_out, w_off)
    if need_dr:
        gr = term_t * p.dtdr
        if p.has_lpos:
            gr = gr + term_s * p.deriv
    return gx, gt, gr


def _scatter_dlam(gt, dlam, m, n_in, n_out, w_off):
    nbp1, cout, cin, _ = gt.shape
    if m == 0:
        d = dlam.reshape(nbp1, cout, n_out, cin, n_in).permute(0, 1, 3, 2, 4)
        idx = w_off + (torch.arange(n_out)[:, None] * n_in + torch.arange(n_in)[None, :])
        gt[..., idx] += d
    else:
        d = dlam.reshape(nbp1, cout, n_out, 2, cin, n_in, 2).permute(0, 1, 4, 2, 5, 3, 6)
        base = w_off + 2 * (torch.arange(n_out)[:, None] * n_in + torch.arange(n_in)[None, :])
        gt[..., base] += d[..., 0, 0] + d[..., 1, 1]
        gt[..., base + 1] += d[..., 0, 1] - d[..., 1, 0]


def dense_lambda(table, r, lvals_in, lvals_out, b: Binning) -> torch.Tensor:
    """Per-edge dense Lambda_e of shape (E, Cout*Dout, Cin*Din), scaling included.

    Brute-force statement used to cross-check the grouped form on tiny inputs.
    """
    E = r.shape[0]
    _, cout, cin, _ = table.shape
    din, dout = dim_of(lvals_in), dim_of(lvals_out)
    lo, t, _ = bin_state(r, b)
    s = r / (r + _sigma(b, r.dtype))
    lam = torch.zeros(E, cout, dout, cin, din, dtype=table.dtype)
    for (m, n_in, n_out, in_off, out_off, w_off) in block_params(lvals_in, lvals_out):
        li, lo_l = block_l(lvals_in, m), block_l(lvals_out, m)
        for e in range(E):
            w = (1 - t[e]) * table[lo[e]] + t[e] * table[lo[e] + 1]      # (co, ci, W)
            for o in range(n_out):
                for i in range(n_in):
                    sc = s[e] ** (li[i] + lo_l[o])
                    if m == 0:
                        lam[e, :, out_off + o, :, in_off + i] = sc * w[:, :, w_off + o * n_in + i]
                    else:
                        a = sc * w[:, :, w_off + 2 * (o * n_in + i)]
                        bb = sc * w[:, :, w_off + 2 * (o * n_in + i) + 1]
                        ro, io = out_off + 2 * o, out_off + 2 * o + 1
                        ri, ii = in_off + 2 * i, in_off + 2 * i + 1
                        lam[e, :, ro, :, ri] = a
                        lam[e, :, ro, :, ii] = bb
                        lam[e, :, io, :, ri] = -bb
                        lam[e, :, io, :, ii] = a
    return lam.reshape(E, cout * dout, cin * din)
