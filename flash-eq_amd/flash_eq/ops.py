"""Autograd wrappers around the HIP library (``libflasheq.so``).

Every function here runs the GPU kernels through the C ABI on the current
stream of the tensors' device; PyTorch only allocates outputs and workspaces.
Inputs must be GPU tensors; float16/bfloat16/float32 inputs are computed in
float32 (fp32 accumulation) and returned in the input dtype.  float64 runs the
generic block-diagonal op's own float64 kernels and is rejected elsewhere
(the fused kernels are float32).
"""
from __future__ import annotations

import os
from functools import lru_cache
from typing import Optional, Sequence, Tuple

import torch

from . import _native as N

_SUPPORTED = (torch.float32, torch.float16, torch.bfloat16)


def _f32(t: torch.Tensor, name: str) -> torch.Tensor:
    N.require_cuda_tensor(t, name)
    if t.dtype == torch.float64:
        raise TypeError(f"{name}: float64 is not supported by the MI355X kernels (use float32)")
    if t.dtype not in _SUPPORTED:
        raise TypeError(f"{name}: unsupported dtype {t.dtype}")
    return t.detach().to(torch.float32).contiguous()


def _f64(t: torch.Tensor, name: str) -> torch.Tensor:
    N.require_cuda_tensor(t, name)
    if t.dtype not in _SUPPORTED + (torch.float64,):
        raise TypeError(f"{name}: unsupported dtype {t.dtype}")
    return t.detach().to(torch.float64).contiguous()


def _same_device(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


# ---------------------------------------------------------------------------
# fused EquivariantEdgewiseLinear
# ---------------------------------------------------------------------------
class EdgewiseLinearFn(torch.autograd.Function):
    """y = (Lambda(r) (x P)) Q^T with Lambda from (C, F); see ``csrc/edgewise.hip``."""

    @staticmethod
    def forward(ctx, x, P, Q, dist, C, F, layout: N.FeqLayout, binning: N.FeqBinning, rank: int):
        dev = _same_device(x, P, Q, dist, C, F)
        E = x.shape[0]
        xs, Ps, Qs = _f32(x, "edge_features"), _f32(P, "P"), _f32(Q, "Q")
        rs, Cs, Fs = _f32(dist, "distances"), _f32(C, "channel_patterns"), _f32(F, "radial")
        _check_edgewise_shapes(layout, binning, rank, xs, Ps, Qs, rs, Cs, Fs)
        y = torch.empty(E, layout.cout, layout.dout, dtype=torch.float32, device=dev)
        # gradients for the bases on the split kernels: keep the rows before
        # the Q rotation (feq_edgewise_fwd_ym / _bwd_pq)
        keep = E > 0 and (ctx.needs_input_grad[1] or ctx.needs_input_grad[2]) and \
            edgewise_pq_supported(layout, binning, rank)
        ym = torch.empty_like(y) if keep else None
        if E:
            lib = N.lib()
            ws = N.workspace(lib.feq_edgewise_fwd_workspace(N.ctypes.byref(layout),
                                                            N.ctypes.byref(binning), rank, E), dev)
            with torch.cuda.device(dev):
                if keep:
                    rc = lib.feq_edgewise_fwd_ym(N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E,
                                                 N.ptr(xs), 0, None, N.ptr(Ps), N.ptr(Qs), N.ptr(rs),
                                                 N.ptr(Cs), N.ptr(Fs), N.ptr(y), N.ptr(ym), 0, N.ptr(ws),
                                                 ws.numel(), N.stream_ptr(dev))
                else:
                    rc = lib.feq_edgewise_fwd(N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E,
                                              N.ptr(xs), N.ptr(Ps), N.ptr(Qs), N.ptr(rs), N.ptr(Cs),
                                              N.ptr(Fs), N.ptr(y), N.ptr(ws), ws.numel(),
                                              N.stream_ptr(dev))
            N.check(rc, "feq_edgewise_fwd_ym" if keep else "feq_edgewise_fwd")
        ctx.save_for_backward(xs, Ps, Qs, rs, Cs, Fs, ym)
        ctx.meta = (layout, binning, rank, x.dtype, P.dtype, Q.dtype, dist.dtype, C.dtype, F.dtype)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, gy):
        xs, Ps, Qs, rs, Cs, Fs, ym = ctx.saved_tensors
        layout, binning, rank, xdt, pdt, qdt, rdt, cdt, fdt = ctx.meta
        dev = xs.device
        E = xs.shape[0]
        need = ctx.needs_input_grad
        g = gy.detach().to(torch.float32).contiguous()
        gx = torch.empty_like(xs) if (need[0] or ym is not None) else None
        gP = torch.empty_like(Ps) if need[1] else None
        gQ = torch.empty_like(Qs) if need[2] else None
        gr = torch.empty_like(rs) if need[3] else None
        gC = torch.empty_like(Cs)
        gF = torch.empty_like(Fs)
        lib = N.lib()
        ws = N.workspace(lib.feq_edgewise_workspace(N.ctypes.byref(layout), N.ctypes.byref(binning),
                                                    rank, E), dev)
        with torch.cuda.device(dev):
            if ym is not None:
                rc = lib.feq_edgewise_bwd_pq(N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E,
                                             N.ptr(g), N.ptr(xs), 0, None, None, None, N.ptr(Ps), N.ptr(Qs),
                                             N.ptr(rs), N.ptr(Cs), N.ptr(Fs), N.ptr(ym), N.ptr(gx),
                                             N.ptr(gC), N.ptr(gF), N.ptr(gr), N.ptr(gP), N.ptr(gQ), 0,
                                             N.ptr(ws), ws.numel(), N.stream_ptr(dev))
            else:
                rc = lib.feq_edgewise_bwd(N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E,
                                          N.ptr(g), N.ptr(xs), N.ptr(Ps), N.ptr(Qs), N.ptr(rs),
                                          N.ptr(Cs), N.ptr(Fs), N.ptr(gx), N.ptr(gC), N.ptr(gF),
                                          N.ptr(gr), N.ptr(gP), N.ptr(gQ), N.ptr(ws), ws.numel(),
                                          N.stream_ptr(dev))
        N.check(rc, "feq_edgewise_bwd_pq" if ym is not None else "feq_edgewise_bwd")
        if not need[0]:
            gx = None
        cast = lambda t, dt: None if t is None else t.to(dt)
        return (cast(gx, xdt), cast(gP, pdt), cast(gQ, qdt), cast(gr, rdt),
                gC.to(cdt) if need[4] else None, gF.to(fdt) if need[5] else None,
                None, None, None)


class EdgewiseLinearSrcFn(torch.autograd.Function):
    """The message-passing form: y = layer(x[src]) with the gather inside the
    kernels (``feq_edgewise_fwd_src``); the backward sums the input gradient
    over every source node's edges inside the input-gradient kernel
    (``feq_edgewise_bwd_src_nodes``, walking ``perm``, ``offsets``: the CSR by
    source), so neither x[src] nor its gradient is ever materialised.
    ``half_accuracy``: one fp16 product per operand pair (FEQ_EW_HALF_ACCURACY),
    for callers held to the half-precision bar."""

    @staticmethod
    def forward(ctx, x, src, perm, offsets, P, Q, dist, C, F, layout: N.FeqLayout,
                binning: N.FeqBinning, rank: int, half_accuracy: bool = False):
        dev = _same_device(x, src, perm, offsets, P, Q, dist, C, F)
        E = src.shape[0]
        xs, Ps, Qs = _f32(x, "node_features"), _f32(P, "P"), _f32(Q, "Q")
        rs, Cs, Fs = _f32(dist, "distances"), _f32(C, "channel_patterns"), _f32(F, "radial")
        if xs.dim() != 3 or xs.shape[1:] != (layout.cin, layout.din):
            raise ValueError(f"node_features must be (N, {layout.cin}, {layout.din}), got {tuple(xs.shape)}")
        if perm.shape != (E,) or offsets.shape != (xs.shape[0] + 1,):
            raise ValueError(f"the CSR by source must cover {E} edges and {xs.shape[0]} nodes; got "
                             f"perm {tuple(perm.shape)}, offsets {tuple(offsets.shape)}")
        _check_edgewise_shapes(layout, binning, rank, torch.empty(E, layout.cin, layout.din, device="meta"),
                               Ps, Qs, rs, Cs, Fs)
        si = src.to(torch.int64).contiguous()
        flags = N.FEQ_EW_HALF_ACCURACY if half_accuracy else 0
        y = torch.empty(E, layout.cout, layout.dout, dtype=torch.float32, device=dev)
        keep = E > 0 and (ctx.needs_input_grad[4] or ctx.needs_input_grad[5])
        if keep and not edgewise_pq_supported(layout, binning, rank):
            raise ValueError("no message-passing kernels forming gradients for P and Q for this layout; "
                             "gather the rows and call edgewise_linear")
        ym = torch.empty_like(y) if keep else None
        if E:
            lib = N.lib()
            ws = N.workspace(lib.feq_edgewise_fwd_workspace(N.ctypes.byref(layout),
                                                            N.ctypes.byref(binning), rank, E), dev)
            with torch.cuda.device(dev):
                if keep:
                    rc = lib.feq_edgewise_fwd_ym(N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E,
                                                 N.ptr(xs), xs.shape[0], N.ptr(si), N.ptr(Ps), N.ptr(Qs),
                                                 N.ptr(rs), N.ptr(Cs), N.ptr(Fs), N.ptr(y), N.ptr(ym), flags,
                                                 N.ptr(ws), ws.numel(), N.stream_ptr(dev))
                else:
                    rc = lib.feq_edgewise_fwd_src_ex(N.ctypes.byref(layout), N.ctypes.byref(binning), rank,
                                                     E, N.ptr(xs), xs.shape[0], N.ptr(si), N.ptr(Ps),
                                                     N.ptr(Qs), N.ptr(rs), N.ptr(Cs), N.ptr(Fs), N.ptr(y),
                                                     flags, N.ptr(ws), ws.numel(), N.stream_ptr(dev))
            N.check(rc, "feq_edgewise_fwd_ym" if keep else "feq_edgewise_fwd_src_ex")
        ctx.save_for_backward(xs, si, perm, offsets, Ps, Qs, rs, Cs, Fs, ym)
        ctx.meta = (layout, binning, rank, x.dtype, P.dtype, Q.dtype, dist.dtype, C.dtype, F.dtype, flags)
        return y.to(x.dtype)

    @staticmethod
    def backward(ctx, gy):
        xs, si, perm, offsets, Ps, Qs, rs, Cs, Fs, ym = ctx.saved_tensors
        layout, binning, rank, xdt, pdt, qdt, rdt, cdt, fdt, flags = ctx.meta
        dev = xs.device
        E = si.shape[0]
        need = ctx.needs_input_grad
        g = gy.detach().to(torch.float32).contiguous()
        gx = torch.empty_like(xs)
        gP = torch.empty_like(Ps) if need[4] else None
        gQ = torch.empty_like(Qs) if need[5] else None
        gr = torch.empty_like(rs) if need[6] else None
        gC = torch.empty_like(Cs)
        gF = torch.empty_like(Fs)
        lib = N.lib()
        ws = N.workspace(lib.feq_edgewise_bwd_src_nodes_workspace(
            N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E), dev)
        with torch.cuda.device(dev):
            if ym is not None:
                rc = lib.feq_edgewise_bwd_pq(
                    N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E, N.ptr(g), N.ptr(xs),
                    xs.shape[0], N.ptr(si), N.ptr(perm), N.ptr(offsets), N.ptr(Ps), N.ptr(Qs), N.ptr(rs),
                    N.ptr(Cs), N.ptr(Fs), N.ptr(ym), N.ptr(gx), N.ptr(gC), N.ptr(gF), N.ptr(gr),
                    N.ptr(gP), N.ptr(gQ), flags, N.ptr(ws), ws.numel(), N.stream_ptr(dev))
            else:
                rc = lib.feq_edgewise_bwd_src_nodes_ex(
                    N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E, N.ptr(g) if E else None,
                    N.ptr(xs), xs.shape[0], N.ptr(si), N.ptr(perm) if E else None, N.ptr(offsets),
                    N.ptr(Ps), N.ptr(Qs), N.ptr(rs), N.ptr(Cs), N.ptr(Fs), N.ptr(gx), N.ptr(gC),
                    N.ptr(gF), N.ptr(gr), flags, N.ptr(ws), ws.numel(), N.stream_ptr(dev))
        N.check(rc, "feq_edgewise_bwd_pq" if ym is not None else "feq_edgewise_bwd_src_nodes_ex")
        if gP is None and need[4]:
            gP = torch.zeros_like(Ps)
        if gQ is None and need[5]:
            gQ = torch.zeros_like(Qs)
        gx = gx.to(xdt) if need[0] else None
        cast = lambda t, dt: None if t is None else t.to(dt)
        return (gx, None, None, None, cast(gP, pdt), cast(gQ, qdt), None if gr is None else gr.to(rdt),
                gC.to(cdt) if need[7] else None, gF.to(fdt) if need[8] else None, None, None, None,
                None)


def edgewise_src_supported(layout: N.FeqLayout, binning: N.FeqBinning, rank: int) -> bool:
    """Whether ``feq_edgewise_fwd_src``/``_bwd_src`` have kernels for this layout."""
    return bool(N.lib().feq_edgewise_src_supported(N.ctypes.byref(layout), N.ctypes.byref(binning), rank))


def edgewise_pq_supported(layout: N.FeqLayout, binning: N.FeqBinning, rank: int) -> bool:
    """Whether the split kernels form the bases' gradients for this layout
    (``feq_edgewise_fwd_ym``/``_bwd_pq``)."""
    return bool(N.lib().feq_edgewise_pq_supported(N.ctypes.byref(layout), N.ctypes.byref(binning), rank))


def edgewise_linear_src(x, src, perm, offsets, P, Q, dist, C, F, layout, binning, rank,
                        half_accuracy: bool = False) -> torch.Tensor:
    return EdgewiseLinearSrcFn.apply(x, src, perm, offsets, P, Q, dist, C, F, layout, binning, rank,
                                     half_accuracy)


def edgewise_pool_supported(layout: N.FeqLayout, binning: N.FeqBinning, rank: int) -> bool:
    """Whether ``feq_edgewise_fwd_src_pool``/``_bwd_src_pool`` have kernels for this layout."""
    return bool(N.lib().feq_edgewise_pool_supported(N.ctypes.byref(layout), N.ctypes.byref(binning), rank))


class EdgewiseAttnPoolFn(torch.autograd.Function):
    """The V projection of ``EquivariantAttention`` (the layer over x[src])
    fused with the attention's head weighting and sum pooling by destination
    (``attention.py:307-314``, ``pooling.py:21-30``):
    out[n, c, :] = sum over the edges e into n of attn[e, c // chan_per_head] * V[e, c, :]
    (``feq_edgewise_fwd_src_pool``).  Neither attn * V nor its gradient is ever
    formed; V itself is kept, in destination order, only when the attention
    weights need a gradient (``feq_attn_pool_grad_attn``).  The backward reads
    attn * grad_out[dst] inside the layer's backward kernels
    (``feq_edgewise_bwd_src_pool``), the input gradient summed per source node."""

    @staticmethod
    def forward(ctx, x, attn, src, dst, perm_s, offsets_s, perm_d, offsets_d, num_dst: int, P, Q, dist,
                C, F, layout: N.FeqLayout, binning: N.FeqBinning, rank: int, heads: int,
                chan_per_head: int, half_accuracy: bool = False):
        dev = _same_device(x, attn, src, dst, perm_s, offsets_s, perm_d, offsets_d, P, Q, dist, C, F)
        E = src.shape[0]
        xs, As, Ps, Qs = _f32(x, "node_features"), _f32(attn, "attention"), _f32(P, "P"), _f32(Q, "Q")
        rs, Cs, Fs = _f32(dist, "distances"), _f32(C, "channel_patterns"), _f32(F, "radial")
        if xs.dim() != 3 or xs.shape[1:] != (layout.cin, layout.din):
            raise ValueError(f"node_features must be (N, {layout.cin}, {layout.din}), got {tuple(xs.shape)}")
        if As.shape != (E, heads):
            raise ValueError(f"attention must be ({E}, {heads}), got {tuple(As.shape)}")
        if dst.shape != (E,) or perm_d.shape != (E,) or offsets_d.shape != (num_dst + 1,):
            raise ValueError(f"the CSR by destination must cover {E} edges and {num_dst} nodes")
        if perm_s.shape != (E,) or offsets_s.shape != (xs.shape[0] + 1,):
            raise ValueError(f"the CSR by source must cover {E} edges and {xs.shape[0]} nodes")
        _check_edgewise_shapes(layout, binning, rank, torch.empty(E, layout.cin, layout.din, device="meta"),
                               Ps, Qs, rs, Cs, Fs)
        si = src.to(torch.int64).contiguous()
        di = dst.to(torch.int64).contiguous()
        flags = N.FEQ_EW_HALF_ACCURACY if half_accuracy else 0
        out = torch.empty(num_dst, layout.cout, layout.dout, dtype=torch.float32, device=dev)
        keep = ctx.needs_input_grad[1] and E > 0
        y_pos = torch.empty(E, layout.cout, layout.dout, dtype=torch.float32, device=dev) if keep else None
        # gradients for the bases: the rows before the Q rotation, in edge order
        pq = E > 0 and (ctx.needs_input_grad[9] or ctx.needs_input_grad[10])
        if pq and not edgewise_pq_supported(layout, binning, rank):
            raise ValueError("no pooled kernels forming gradients for P and Q for this layout")
        ym = torch.empty(E, layout.cout, layout.dout, dtype=torch.float32, device=dev) if pq else None
        lib = N.lib()
        ws = N.workspace(lib.feq_edgewise_fwd_src_pool_workspace(N.ctypes.byref(layout),
                                                                 N.ctypes.byref(binning), rank, E), dev)
        with torch.cuda.device(dev):
            args = (N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E, N.ptr(xs), xs.shape[0],
                    N.ptr(si), N.ptr(Ps), N.ptr(Qs), N.ptr(rs), N.ptr(Cs), N.ptr(Fs), N.ptr(As), heads,
                    chan_per_head, N.ptr(di), N.ptr(perm_d) if E else None, N.ptr(offsets_d), num_dst,
                    N.ptr(out) if num_dst else None, N.ptr(y_pos))
            tail = (flags, N.ptr(ws), ws.numel(), N.stream_ptr(dev))
            if pq:
                rc = lib.feq_edgewise_fwd_src_pool_ym(*args, N.ptr(ym), *tail)
            else:
                rc = lib.feq_edgewise_fwd_src_pool(*args, *tail)
        N.check(rc, "feq_edgewise_fwd_src_pool_ym" if pq else "feq_edgewise_fwd_src_pool")
        ctx.save_for_backward(xs, As, si, di, perm_s, offsets_s, perm_d, offsets_d, Ps, Qs, rs, Cs, Fs,
                              y_pos, ym)
        ctx.meta = (layout, binning, rank, heads, chan_per_head, num_dst, flags,
                    x.dtype, attn.dtype, dist.dtype, C.dtype, F.dtype, P.dtype, Q.dtype)
        return out.to(x.dtype)

    @staticmethod
    def backward(ctx, gout):
        xs, As, si, di, perm_s, offsets_s, perm_d, offsets_d, Ps, Qs, rs, Cs, Fs, y_pos, ym = ctx.saved_tensors
        layout, binning, rank, heads, cph, num_dst, flags, xdt, adt, rdt, cdt, fdt, pdt, qdt = ctx.meta
        dev = xs.device
        E = si.shape[0]
        need = ctx.needs_input_grad
        g = gout.detach().to(torch.float32).contiguous()
        lib = N.lib()
        gA = None
        if need[1]:
            gA = torch.empty_like(As)
            if E:
                with torch.cuda.device(dev):
                    rc = lib.feq_attn_pool_grad_attn(N.ptr(y_pos), N.ptr(g), N.ptr(perm_d), N.ptr(offsets_d),
                                                     E, num_dst, layout.cout, layout.dout, heads, N.ptr(gA),
                                                     N.stream_ptr(dev))
                N.check(rc, "feq_attn_pool_grad_attn")
        gx = torch.empty_like(xs)
        gP = torch.empty_like(Ps) if need[9] else None
        gQ = torch.empty_like(Qs) if need[10] else None
        gr = torch.empty_like(rs) if need[11] else None
        gC = torch.empty_like(Cs)
        gF = torch.empty_like(Fs)
        ws = N.workspace(lib.feq_edgewise_bwd_src_nodes_workspace(
            N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E), dev)
        with torch.cuda.device(dev):
            head = (N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E, N.ptr(g) if num_dst else None,
                    N.ptr(As), heads, cph, N.ptr(di), num_dst, N.ptr(xs), xs.shape[0], N.ptr(si),
                    N.ptr(perm_s) if E else None, N.ptr(offsets_s), N.ptr(Ps), N.ptr(Qs), N.ptr(rs),
                    N.ptr(Cs), N.ptr(Fs))
            tail = (flags, N.ptr(ws), ws.numel(), N.stream_ptr(dev))
            if ym is not None:
                rc = lib.feq_edgewise_bwd_src_pool_pq(*head, N.ptr(ym), N.ptr(gx), N.ptr(gC), N.ptr(gF),
                                                      N.ptr(gr), N.ptr(gP), N.ptr(gQ), *tail)
            else:
                rc = lib.feq_edgewise_bwd_src_pool(*head, N.ptr(gx), N.ptr(gC), N.ptr(gF), N.ptr(gr), *tail)
        N.check(rc, "feq_edgewise_bwd_src_pool_pq" if ym is not None else "feq_edgewise_bwd_src_pool")
        cast = lambda t, dt: None if t is None else t.to(dt)
        return (gx.to(xdt) if need[0] else None, None if gA is None else gA.to(adt),
                None, None, None, None, None, None, None, cast(gP, pdt), cast(gQ, qdt),
                None if gr is None else gr.to(rdt), gC.to(cdt) if need[12] else None,
                gF.to(fdt) if need[13] else None, None, None, None, None, None, None)


def edgewise_attention_pool(x, attn, src, dst, perm_s, offsets_s, perm_d, offsets_d, num_dst, P, Q,
                            dist, C, F, layout, binning, rank, heads: int, chan_per_head: int,
                            half_accuracy: bool = False) -> torch.Tensor:
    return EdgewiseAttnPoolFn.apply(x, attn, src, dst, perm_s, offsets_s, perm_d, offsets_d, num_dst, P,
                                    Q, dist, C, F, layout, binning, rank, heads, chan_per_head,
                                    half_accuracy)


# ---------------------------------------------------------------------------
# embedding of small canonical layouts into the config-2 shape
# ---------------------------------------------------------------------------
_EMB_L, _EMB_C = 2, 64


def _mfirst_positions(L: int) -> dict:
    """(l, m, c) -> slot of the m-first order of lvals 0..L (m = 0 one slot per
    l; then for m = 1..L and l >= m the (+m, -m) pair, c = 0 / 1)."""
    pos, k = {}, 0
    for l in range(L + 1):
        pos[(l, 0, 0)] = k
        k += 1
    for m in range(1, L + 1):
        for l in range(m, L + 1):
            pos[(l, m, 0)], pos[(l, m, 1)] = k, k + 1
            k += 2
    return pos


def _weight_positions(lin: int, lout: int) -> dict:
    """(m, o, i, c) -> radial weight index of the m-block layout of the canonical
    pair 0..lin -> 0..lout (block_diagonal.cu:1220-1258): in block m the i-th
    input degree is m + i and the o-th output degree m + o."""
    pos, off = {}, 0
    for m in range(min(lin, lout) + 1):
        ni, no = lin - m + 1, lout - m + 1
        for o in range(no):
            for i in range(ni):
                if m == 0:
                    pos[(m, o, i, 0)] = off + o * ni + i
                else:
                    pos[(m, o, i, 0)] = off + 2 * (o * ni + i)
                    pos[(m, o, i, 1)] = off + 2 * (o * ni + i) + 1
        off += (1 if m == 0 else 2) * ni * no
    return pos


class _Embedding:
    """Runs a layer of canonical lvals 0..lin -> 0..lout and at most 64 channels
    with the kernels of a larger canonical layout, lvals 0..tin -> 0..tout with
    64 channels (tin >= lin, tout >= lout): features, channel patterns and bases
    are zero-padded, the radial functions placed at their weights' positions in
    the larger layout (zeros elsewhere), and the output cut back.  Padded inputs
    are zero, so they add exact zeros; the power-of-two block scales of the
    split kernels come from block maxima and do not change.  All steps are
    torch ops, so autograd carries the gradients."""

    def __init__(self, lin: int, lout: int, cin: int, cout: int, device, tin: int = _EMB_L,
                 tout: int = _EMB_L):
        self.lin, self.lout, self.cin, self.cout = lin, lout, cin, cout
        self.din, self.dout = (lin + 1) ** 2, (lout + 1) ** 2
        self.Din, self.Dout = (tin + 1) ** 2, (tout + 1) ** 2

        def cols(lmax, L):
            """Slots of the larger m-first order that the small order's slots take
            (None when the small order is the larger one)."""
            if lmax == L:
                return None
            big, small = _mfirst_positions(L), _mfirst_positions(lmax)
            at = [0] * len(small)
            for key, js in small.items():
                at[js] = big[key]
            return torch.tensor(at, device=device)

        self.pcols, self.qcols = cols(lin, tin), cols(lout, tout)
        ws, wb = _weight_positions(lin, lout), _weight_positions(tin, tout)
        self.wdim = len(ws)
        wsrc = [self.wdim] * len(wb)          # index wdim: an appended zero column
        for key, w in ws.items():
            wsrc[wb[key]] = w
        self.wsrc = torch.tensor(wsrc, device=device)
        self.layout = N.make_layout(list(range(tin + 1)), list(range(tout + 1)), _EMB_C, _EMB_C)

    def features(self, x):
        return torch.nn.functional.pad(x, (0, self.Din - x.shape[-1], 0, _EMB_C - x.shape[-2]))

    @staticmethod
    def _place(R, cols, D):
        """R (E, d, d) placed in a zero (E, D, D): rows d in the standard order
        keep their index, column j goes to cols[j]."""
        if cols is None:
            return R
        Rp = R.new_zeros(R.shape[0], D, D)
        Rp[:, :R.shape[-1], cols] = R
        return Rp

    def basis_in(self, P):
        return self._place(P, self.pcols, self.Din)

    def basis_out(self, Q):
        return self._place(Q, self.qcols, self.Dout)

    def channels(self, C):
        return torch.nn.functional.pad(C, (0, _EMB_C - self.cin, 0, _EMB_C - self.cout))

    def radial(self, F):
        return torch.index_select(torch.nn.functional.pad(F, (0, 1)), 2, self.wsrc)

    def output(self, y):
        return y[:, :self.cout, :self.dout]


_EMB_CACHE: dict = {}


# Canonical (lin, lout) layouts with 64 channels in and out whose split kernels
# (forward and backward) exist, smallest first: the embedding targets.
_EMB_TARGETS = ((1, 2), (2, 2))


def embedding_for(lvals_in, lvals_out, cin: int, cout: int, rank: int, device) -> Optional[_Embedding]:
    """The embedding of a layout into the smallest target layout with split
    kernels that holds it, or None when the layout is not a canonical prefix of
    [0, 1, 2] with at most 64 channels."""
    lin, lout = tuple(lvals_in), tuple(lvals_out)
    if rank != 4 or cin > _EMB_C or cout > _EMB_C:
        return None
    if lin != tuple(range(len(lin))) or lout != tuple(range(len(lout))):
        return None
    li, lo = len(lin) - 1, len(lout) - 1
    target = next(((ti, to) for ti, to in _EMB_TARGETS if li <= ti and lo <= to), None)
    if target is None:
        return None
    key = (lin, lout, cin, cout, str(device))
    if key not in _EMB_CACHE:
        _EMB_CACHE[key] = _Embedding(li, lo, cin, cout, device, *target)
    return _EMB_CACHE[key]


def _check_edgewise_shapes(L, b, rank, x, P, Q, r, C, F) -> None:
    E = x.shape[0]
    if x.shape != (E, L.cin, L.din):
        raise ValueError(f"edge_features must be (E, {L.cin}, {L.din}), got {tuple(x.shape)}")
    if P.shape != (E, L.din, L.din):
        raise ValueError(f"P must be (E, {L.din}, {L.din}), got {tuple(P.shape)}")
    if Q.shape != (E, L.dout, L.dout):
        raise ValueError(f"Q must be (E, {L.dout}, {L.dout}), got {tuple(Q.shape)}")
    if r.shape != (E,):
        raise ValueError(f"distances must be (E,), got {tuple(r.shape)}")
    if C.shape != (rank, L.cout, L.cin):
        raise ValueError(f"channel_patterns must be ({rank}, {L.cout}, {L.cin}), got {tuple(C.shape)}")
    if F.shape != (b.num_bins + 1, rank, L.wdim):
        raise ValueError(f"radial functions must be ({b.num_bins + 1}, {rank}, {L.wdim}), "
                         f"got {tuple(F.shape)}")


class EdgewiseLinearHLFn(torch.autograd.Function):
    """The high-degree form for bfloat16 features (``csrc/edgewise_hl.hip``):
    x, P, Q and y stay bf16 (no float32 copies), the GEMMs run on the bf16
    matrix cores with float32 accumulation; the radial parameters and
    distances are float32."""

    @staticmethod
    def forward(ctx, x, P, Q, dist, C, F, layout: N.FeqLayout, binning: N.FeqBinning, rank: int):
        dev = _same_device(x, P, Q, dist, C, F)
        E = x.shape[0]
        xs, Ps, Qs = (t.detach().contiguous() for t in (x, P, Q))
        rs, Cs, Fs = _f32(dist, "distances"), _f32(C, "channel_patterns"), _f32(F, "radial")
        _check_edgewise_shapes(layout, binning, rank, xs, Ps, Qs, rs, Cs, Fs)
        y = torch.empty(E, layout.cout, layout.dout, dtype=torch.bfloat16, device=dev)
        # the rotated input s^l (x P), kept for the backward (one bf16 copy of x)
        fs = torch.empty(E, layout.din, layout.cin, dtype=torch.bfloat16, device=dev)
        if E:
            lib = N.lib()
            ws = N.workspace(lib.feq_edgewise_hl_workspace(N.ctypes.byref(layout),
                                                           N.ctypes.byref(binning), rank, E, 0), dev)
            with torch.cuda.device(dev):
                rc = lib.feq_edgewise_hl_fwd(N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E,
                                             N.ptr(xs), N.ptr(Ps), N.ptr(Qs), N.ptr(rs), N.ptr(Cs),
                                             N.ptr(Fs), N.ptr(y), N.ptr(fs), N.ptr(ws), ws.numel(),
                                             N.stream_ptr(dev))
            N.check(rc, "feq_edgewise_hl_fwd")
        ctx.save_for_backward(xs, Ps, Qs, rs, Cs, Fs, fs)
        ctx.meta = (layout, binning, rank, dist.dtype, C.dtype, F.dtype)
        return y

    @staticmethod
    def backward(ctx, gy):
        xs, Ps, Qs, rs, Cs, Fs, fs = ctx.saved_tensors
        layout, binning, rank, rdt, cdt, fdt = ctx.meta
        dev = xs.device
        E = xs.shape[0]
        need = ctx.needs_input_grad
        g = gy.detach().to(torch.bfloat16).contiguous()
        gx = torch.empty_like(xs) if need[0] else None
        gr = torch.empty_like(rs) if need[3] else None
        gC = torch.empty_like(Cs)
        gF = torch.empty_like(Fs)
        lib = N.lib()
        ws = N.workspace(lib.feq_edgewise_hl_workspace(N.ctypes.byref(layout), N.ctypes.byref(binning),
                                                       rank, E, 1), dev)
        with torch.cuda.device(dev):
            rc = lib.feq_edgewise_hl_bwd(N.ctypes.byref(layout), N.ctypes.byref(binning), rank, E,
                                         N.ptr(g), N.ptr(xs), N.ptr(Ps), N.ptr(Qs), N.ptr(rs),
                                         N.ptr(Cs), N.ptr(Fs), N.ptr(gx), N.ptr(gC), N.ptr(gF),
                                         N.ptr(gr), N.ptr(fs) if E else None, N.ptr(ws), ws.numel(),
                                         N.stream_ptr(dev))
        N.check(rc, "feq_edgewise_hl_bwd")
        return (gx, None, None, None if gr is None else gr.to(rdt),
                gC.to(cdt) if need[4] else None, gF.to(fdt) if need[5] else None,
                None, None, None)


def _use_hl(x, P, Q, layout, binning, rank) -> bool:
    """bf16 features, bases and a layout with high-degree kernels; P and Q
    without gradients (the high-degree backward does not form them)."""
    if not (x.dtype == P.dtype == Q.dtype == torch.bfloat16):
        return False
    if P.requires_grad or Q.requires_grad:
        return False
    return bool(N.lib().feq_edgewise_hl_supported(N.ctypes.byref(layout), N.ctypes.byref(binning),
                                                  rank))


def edgewise_linear(x, P, Q, dist, C, F, layout, binning, rank) -> torch.Tensor:
    if _use_hl(x, P, Q, layout, binning, rank):
        return EdgewiseLinearHLFn.apply(x, P, Q, dist, C, F, layout, binning, rank)
    return EdgewiseLinearFn.apply(x, P, Q, dist, C, F, layout, binning, rank)


# ---------------------------------------------------------------------------
# generic block-diagonal op (reference table layout)
# ---------------------------------------------------------------------------
class BlockDiagonalFn(torch.autograd.Function):
    """The reference's block-diagonal op on a (num_bins+1, Cout, Cin, Wdim) table
    (``_BlockDiagonalFunction``, block_diagonal.py:77-174): float32 and float64
    run their own kernels, float16/bfloat16 compute in float32 and return the
    input dtype.  Gradients for features, table and distances; the table
    gradient is summed per bin in a fixed order (deterministic)."""

    @staticmethod
    def forward(ctx, features, table, dist, layout: N.FeqLayout, binning: N.FeqBinning):
        dev = _same_device(features, table, dist)
        f64 = features.dtype == torch.float64
        cast = (lambda t, n: _f64(t, n)) if f64 else _f32
        xs, ts, rs = cast(features, "features"), cast(table, "radial_table"), cast(dist, "distances")
        E = xs.shape[0]
        if xs.shape[1:] != (layout.cin, layout.din):
            raise ValueError(f"features must be (E, {layout.cin}, {layout.din}), got {tuple(xs.shape)}")
        if ts.shape != (binning.num_bins + 1, layout.cout, layout.cin, layout.wdim):
            raise ValueError(f"radial_table must be ({binning.num_bins + 1}, {layout.cout}, "
                             f"{layout.cin}, {layout.wdim}), got {tuple(ts.shape)}")
        y = torch.empty(E, layout.cout, layout.dout, dtype=xs.dtype, device=dev)
        if E:
            lib = N.lib()
            with torch.cuda.device(dev):
                if f64:
                    rc = lib.feq_blockdiag_fwd_f64(N.ctypes.byref(layout), N.ctypes.byref(binning), E,
                                                   N.ptr(xs), N.ptr(ts), N.ptr(rs), N.ptr(y),
                                                   N.stream_ptr(dev))
                else:
                    rc = lib.feq_blockdiag_fwd(N.ctypes.byref(layout), N.ctypes.byref(binning), E,
                                               N.ptr(xs), N.ptr(ts), N.ptr(rs), N.ptr(y), None, 0,
                                               N.stream_ptr(dev))
            N.check(rc, "feq_blockdiag_fwd")
        ctx.save_for_backward(xs, ts, rs)
        ctx.meta = (layout, binning, features.dtype, table.dtype, dist.dtype)
        return y.to(features.dtype)

    @staticmethod
    def backward(ctx, gy):
        xs, ts, rs = ctx.saved_tensors
        layout, binning, xdt, tdt, rdt = ctx.meta
        dev = xs.device
        E = xs.shape[0]
        g = gy.detach().to(xs.dtype).contiguous()
        gx = torch.empty_like(xs)
        gt = torch.empty_like(ts)
        gr = torch.empty_like(rs) if ctx.needs_input_grad[2] else None
        lib = N.lib()
        ws = N.workspace(lib.feq_blockdiag_workspace(N.ctypes.byref(layout), N.ctypes.byref(binning),
                                                     E), dev)
        fn = lib.feq_blockdiag_bwd_f64 if xs.dtype == torch.float64 else lib.feq_blockdiag_bwd
        with torch.cuda.device(dev):
            rc = fn(N.ctypes.byref(layout), N.ctypes.byref(binning), E, N.ptr(g) if E else None,
                    N.ptr(xs), N.ptr(ts), N.ptr(rs), N.ptr(gx), N.ptr(gt), N.ptr(gr), N.ptr(ws),
                    ws.numel(), N.stream_ptr(dev))
        N.check(rc, "feq_blockdiag_bwd")
        return gx.to(xdt), gt.to(tdt), (None if gr is None else gr.to(rdt)), None, None


# ---------------------------------------------------------------------------
# graph reductions
# ---------------------------------------------------------------------------
class SegmentSumFn(torch.autograd.Function):
    """out[n] = sum_{e: dst[e]=n} x[e] over the cached CSR (GraphPooling 'sum')."""

    @staticmethod
    def forward(ctx, x, dst, perm, offsets, num_nodes: int):
        dev = _same_device(x, dst, perm, offsets)
        xs = _f32(x, "edge_features")
        E = xs.shape[0]
        row = int(xs[0].numel()) if E else int(torch.tensor(xs.shape[1:]).prod())
        out = torch.empty((num_nodes,) + tuple(xs.shape[1:]), dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            rc = N.lib().feq_segment_sum(N.ptr(xs) if E else None, row, N.ptr(perm) if E else None,
                                         N.ptr(offsets), num_nodes, N.ptr(out), N.stream_ptr(dev))
        N.check(rc, "feq_segment_sum")
        ctx.save_for_backward(dst)
        ctx.meta = (x.dtype, E, row, num_nodes, tuple(xs.shape))
        return out.to(x.dtype)

    @staticmethod
    def backward(ctx, gout):
        (dst,) = ctx.saved_tensors
        xdt, E, row, num_nodes, shape = ctx.meta
        dev = dst.device
        g = gout.detach().to(torch.float32).contiguous()
        gx = torch.empty(shape, dtype=torch.float32, device=dev)
        if E:
            d64 = dst.to(torch.int64).contiguous()
            with torch.cuda.device(dev):
                rc = N.lib().feq_gather_rows(N.ptr(g), num_nodes, row, N.ptr(d64), E, N.ptr(gx),
                                             N.stream_ptr(dev))
            N.check(rc, "feq_gather_rows")
        return gx.to(xdt), None, None, None, None


class GatherRowsFn(torch.autograd.Function):
    """out[e] = x[idx[e]]; the backward sums the rows of every node's edges over
    the CSR grouping of ``idx`` (``perm``, ``offsets``), deterministically."""

    @staticmethod
    def forward(ctx, x, idx, perm, offsets):
        dev = _same_device(x, idx, perm, offsets)
        xs = _f32(x, "node_features")
        num_src = xs.shape[0]
        E = idx.shape[0]
        row = int(torch.tensor(xs.shape[1:]).prod()) if xs.dim() > 1 else 1
        out = torch.empty((E,) + tuple(xs.shape[1:]), dtype=torch.float32, device=dev)
        i64 = idx.to(torch.int64).contiguous()
        if E:
            with torch.cuda.device(dev):
                rc = N.lib().feq_gather_rows(N.ptr(xs), num_src, row, N.ptr(i64), E, N.ptr(out),
                                             N.stream_ptr(dev))
            N.check(rc, "feq_gather_rows")
        ctx.save_for_backward(perm, offsets)
        ctx.meta = (x.dtype, num_src, row, E, tuple(xs.shape))
        return out.to(x.dtype)

    @staticmethod
    def backward(ctx, gout):
        perm, offsets = ctx.saved_tensors
        xdt, num_src, row, E, shape = ctx.meta
        dev = perm.device
        g = gout.detach().to(torch.float32).contiguous()
        gx = torch.empty(shape, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            rc = N.lib().feq_segment_sum(N.ptr(g) if E else None, row, N.ptr(perm) if E else None,
                                         N.ptr(offsets), num_src, N.ptr(gx), N.stream_ptr(dev))
        N.check(rc, "feq_segment_sum")
        return gx.to(xdt), None, None, None


def gather_rows(x, idx, perm, offsets) -> torch.Tensor:
    return GatherRowsFn.apply(x, idx, perm, offsets)


class EdgeSoftmaxFn(torch.autograd.Function):
    """Per-destination softmax of scale*<Q,K> (- r/decay) with +1e-8 (``attention.py:92-141``),
    for edge-level Q, K (E, H, Dh) (the edge form of ``feq_attn_softmax_fwd``)."""

    @staticmethod
    def forward(ctx, Q, K, dist, log_scale, decay: float, perm, offsets, num_nodes: int):
        dev = _same_device(Q, K, log_scale, perm, offsets)
        Qs, Ks = _f32(Q, "Q"), _f32(K, "K")
        E, H, Dh = Qs.shape
        if Ks.shape != Qs.shape:
            raise ValueError(f"Q and K shapes differ: {tuple(Qs.shape)} and {tuple(Ks.shape)}")
        scale_t = log_scale.detach().float().exp().reshape(1).contiguous()   # read by the kernels
        rs = _f32(dist, "distances") if (dist is not None and decay > 0) else None
        attn = torch.empty(E, H, dtype=torch.float32, device=dev)
        qk = torch.empty(E, H, dtype=torch.float32, device=dev)
        if E:
            with torch.cuda.device(dev):
                rc = N.lib().feq_attn_softmax_fwd(N.ptr(Qs), H * Dh, N.ptr(Ks), H * Dh, None, None,
                                                  E, N.ptr(rs), E, H, Dh, N.ptr(scale_t),
                                                  float(decay), N.ptr(perm), N.ptr(offsets),
                                                  num_nodes, N.ptr(attn), N.ptr(qk),
                                                  N.stream_ptr(dev))
            N.check(rc, "feq_attn_softmax_fwd")
        ctx.save_for_backward(Qs, Ks, attn, qk, perm, offsets, scale_t)
        ctx.meta = (decay, num_nodes, Q.dtype, K.dtype, None if dist is None else dist.dtype,
                    log_scale.dtype)
        return attn.to(Q.dtype)

    @staticmethod
    def backward(ctx, gattn):
        Qs, Ks, attn, qk, perm, offsets, scale_t = ctx.saved_tensors
        decay, num_nodes, qdt, kdt, rdt, ldt = ctx.meta
        dev = Qs.device
        E, H, Dh = Qs.shape
        need = ctx.needs_input_grad
        ga = gattn.detach().to(torch.float32).contiguous()
        gQ = torch.empty_like(Qs)
        gK = torch.empty_like(Ks)
        glog = torch.empty(E, H, dtype=torch.float32, device=dev)
        if E:
            with torch.cuda.device(dev):
                rc = N.lib().feq_attn_softmax_bwd(N.ptr(Qs), H * Dh, N.ptr(Ks), H * Dh, None, None,
                                                  E, N.ptr(attn), N.ptr(ga), E, H, Dh,
                                                  N.ptr(scale_t), N.ptr(perm),
                                                  N.ptr(offsets), num_nodes, None, None,
                                                  N.ptr(gQ), H * Dh, N.ptr(gK), H * Dh,
                                                  N.ptr(glog), N.stream_ptr(dev))
            N.check(rc, "feq_attn_softmax_bwd")
        return (gQ.to(qdt), gK.to(kdt), *_softmax_scalar_grads(glog, qk, need[2], need[3], decay,
                                                                 rdt, ldt),
                None, None, None, None)


def _softmax_scalar_grads(glog, qk, need_dist: bool, need_scale: bool, decay: float, rdt, ldt):
    """Distance and log-scale gradients from the logit gradient (E, H):
    d logit / d r = -1/decay, d logit / d log_scale = scale <Q,K> = qk."""
    g_dist = (glog.sum(1) * (-1.0 / decay)).to(rdt) if (need_dist and decay > 0) else None
    # one scalar from E*H products that largely cancel: accumulated in float64
    g_log = dot_f64(glog, qk).to(ldt) if need_scale else None
    return g_dist, g_log


class NodeSoftmaxFn(torch.autograd.Function):
    """The same softmax with Q and K read from the node table of the fused QK
    projection (``attention.py:298-304``): qk (N, 2 mult, dim), Q = channels
    [0, mult) read at dst[e], K = channels [mult, 2 mult) read at src[e], H
    heads of (mult / H) * dim values.  The gathers run inside the kernels (node
    form of ``feq_attn_softmax_fwd``), so the (E, H, Dh) Q and K are never
    formed; the backward sums the Q gradient per destination and the K
    gradient per source (CSR by source), writing the (N, 2 mult, dim) gradient.
    ``cm``: qk (and its gradient) component-major (dim, N, 2 mult), the layout
    the projection writes (feq_attn_softmax_fwd_cm / _bwd_cm)."""

    @staticmethod
    def forward(ctx, qk, dist, log_scale, decay: float, heads: int, src, dst, perm, offsets,
                perm_s, offsets_s, num_nodes: int, cm: bool = False):
        dev = _same_device(qk, log_scale, src, dst, perm, offsets, perm_s, offsets_s)
        qs = _f32(qk, "qk")
        src = src.to(torch.int64).contiguous()
        dst = dst.to(torch.int64).contiguous()
        if cm:
            dim, Nn, two_mult = qs.shape
        else:
            Nn, two_mult, dim = qs.shape
        mult = two_mult // 2
        if two_mult != 2 * mult or mult % heads:
            raise ValueError(f"qk must be (N, 2*mult, dim) with heads | mult, got {tuple(qs.shape)}")
        if Nn != num_nodes:
            # the backward writes one Q-gradient row per destination segment and
            # one K-gradient row per source segment of the graph's CSRs
            raise ValueError(f"qk has {Nn} rows but the graph has {num_nodes} nodes")
        E = src.shape[0]
        Dh, ld = mult // heads * dim, two_mult * dim
        scale_t = log_scale.detach().float().exp().reshape(1).contiguous()   # read by the kernels
        rs = _f32(dist, "distances") if (dist is not None and decay > 0) else None
        attn = torch.empty(E, heads, dtype=torch.float32, device=dev)
        qkv = torch.empty(E, heads, dtype=torch.float32, device=dev)
        if E:
            with torch.cuda.device(dev):
                if cm:
                    rc = N.lib().feq_attn_softmax_fwd_cm(N.ptr(qs), N.ptr(qs) + 4 * mult, two_mult,
                                                         Nn * two_mult, dim, N.ptr(dst), N.ptr(src), Nn,
                                                         N.ptr(rs), E, heads, mult // heads, N.ptr(scale_t),
                                                         float(decay), N.ptr(perm), N.ptr(offsets),
                                                         num_nodes, N.ptr(attn), N.ptr(qkv),
                                                         N.stream_ptr(dev))
                else:
                    rc = N.lib().feq_attn_softmax_fwd(N.ptr(qs), ld, N.ptr(qs) + 4 * mult * dim, ld,
                                                      N.ptr(dst), N.ptr(src), Nn, N.ptr(rs), E, heads,
                                                      Dh, N.ptr(scale_t), float(decay),
                                                      N.ptr(perm), N.ptr(offsets), num_nodes,
                                                      N.ptr(attn), N.ptr(qkv), N.stream_ptr(dev))
            N.check(rc, "feq_attn_softmax_fwd")
        ctx.save_for_backward(qs, attn, qkv, src, dst, perm, offsets, perm_s, offsets_s, scale_t)
        ctx.meta = (decay, num_nodes, heads, qk.dtype, None if dist is None else dist.dtype,
                    log_scale.dtype, cm)
        return attn.to(qk.dtype)

    @staticmethod
    def backward(ctx, gattn):
        qs, attn, qkv, src, dst, perm, offsets, perm_s, offsets_s, scale_t = ctx.saved_tensors
        decay, num_nodes, heads, qdt, rdt, ldt, cm = ctx.meta
        dev = qs.device
        if cm:
            dim, Nn, two_mult = qs.shape
        else:
            Nn, two_mult, dim = qs.shape
        mult = two_mult // 2
        E = src.shape[0]
        Dh, ld = mult // heads * dim, two_mult * dim
        need = ctx.needs_input_grad
        ga = gattn.detach().to(torch.float32).contiguous()
        glog = torch.empty(E, heads, dtype=torch.float32, device=dev)
        if E == 0:
            g_dist, g_log = _softmax_scalar_grads(glog, qkv, need[1], need[2], decay, rdt, ldt)
            return (torch.zeros_like(qs).to(qdt), g_dist, g_log, None, None, None, None, None, None,
                    None, None, None, None)
        gqk = torch.empty_like(qs)
        with torch.cuda.device(dev):
            if cm:
                rc = N.lib().feq_attn_softmax_bwd_cm(N.ptr(qs), N.ptr(qs) + 4 * mult, two_mult, Nn * two_mult,
                                                     dim, N.ptr(dst), N.ptr(src), Nn, N.ptr(attn), N.ptr(ga),
                                                     E, heads, mult // heads, N.ptr(scale_t), N.ptr(perm),
                                                     N.ptr(offsets), num_nodes, N.ptr(perm_s),
                                                     N.ptr(offsets_s), N.ptr(gqk), N.ptr(gqk) + 4 * mult,
                                                     N.ptr(glog), N.stream_ptr(dev))
            else:
                rc = N.lib().feq_attn_softmax_bwd(N.ptr(qs), ld, N.ptr(qs) + 4 * mult * dim, ld,
                                                  N.ptr(dst), N.ptr(src), Nn, N.ptr(attn), N.ptr(ga),
                                                  E, heads, Dh, N.ptr(scale_t), N.ptr(perm),
                                                  N.ptr(offsets), num_nodes, N.ptr(perm_s),
                                                  N.ptr(offsets_s), N.ptr(gqk), ld,
                                                  N.ptr(gqk) + 4 * mult * dim, ld, N.ptr(glog),
                                                  N.stream_ptr(dev))
        N.check(rc, "feq_attn_softmax_bwd")
        g_dist, g_log = _softmax_scalar_grads(glog, qkv, need[1], need[2], decay, rdt, ldt)
        return (gqk.to(qdt), g_dist, g_log, None, None, None, None, None, None, None, None, None, None)


class AttnPoolFn(torch.autograd.Function):
    """out[n,c,:] = sum_{e->n} attn[e, head(c)] V[e,c,:] (``attention.py:143-167`` + sum pooling)."""

    @staticmethod
    def forward(ctx, V, attn, dst, perm, offsets, num_nodes: int, heads: int):
        dev = _same_device(V, attn, dst, perm, offsets)
        Vs, As = _f32(V, "V"), _f32(attn, "attention")
        E, mult, dim = Vs.shape
        out = torch.empty(num_nodes, mult, dim, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            rc = N.lib().feq_attn_pool_fwd(N.ptr(Vs) if E else None, N.ptr(As) if E else None, E,
                                           mult, dim, heads, N.ptr(perm) if E else None,
                                           N.ptr(offsets), num_nodes, N.ptr(out), N.stream_ptr(dev))
        N.check(rc, "feq_attn_pool_fwd")
        ctx.save_for_backward(Vs, As, perm, offsets)
        ctx.meta = (num_nodes, heads, V.dtype, attn.dtype)
        return out.to(V.dtype)

    @staticmethod
    def backward(ctx, gout):
        Vs, As, perm, offsets = ctx.saved_tensors
        num_nodes, heads, vdt, adt = ctx.meta
        dev = Vs.device
        E, mult, dim = Vs.shape
        g = gout.detach().to(torch.float32).contiguous()
        gV = torch.empty_like(Vs)
        gA = torch.empty_like(As)
        if E:
            with torch.cuda.device(dev):
                rc = N.lib().feq_attn_pool_bwd(N.ptr(Vs), N.ptr(As), N.ptr(g), N.ptr(perm),
                                               N.ptr(offsets), E, num_nodes, mult, dim, heads,
                                               N.ptr(gV), N.ptr(gA), N.stream_ptr(dev))
            N.check(rc, "feq_attn_pool_bwd")
        return gV.to(vdt), gA.to(adt), None, None, None, None, None


def bin_edges(dist: torch.Tensor, binning: N.FeqBinning) -> Tuple[torch.Tensor, torch.Tensor]:
    """(lo int32, t float32) per edge from the kernels' binning (for checks and tools)."""
    dev = dist.device
    rs = _f32(dist, "distances")
    E = rs.shape[0]
    lo = torch.empty(E, dtype=torch.int32, device=dev)
    t = torch.empty(E, dtype=torch.float32, device=dev)
    if E:
        with torch.cuda.device(dev):
            rc = N.lib().feq_bin_edges(N.ctypes.byref(binning), E, N.ptr(rs), N.ptr(lo), N.ptr(t),
                                       N.stream_ptr(dev))
        N.check(rc, "feq_bin_edges")
    return lo, t


# ---- node-side norms and gating (csrc/nodeside.hip) ---------------------------------

NODE_MAX_MULT = 256
NODE_MAX_SCALARS = 8


@lru_cache(maxsize=256)
def _lvals_i32(lvals: Tuple[int, ...]):
    return (N.ctypes.c_int32 * len(lvals))(*lvals)


def node_kernels_ok(x: torch.Tensor, lvals: Tuple[int, ...], mult: int,
                    *params: Optional[torch.Tensor]) -> bool:
    """The node-side kernels take float32 GPU tables of at most NODE_MAX_MULT
    channels whose float32 parameters live on the same device; other inputs run
    the modules' PyTorch formulation."""
    if not (x.is_cuda and x.dtype == torch.float32 and 1 <= mult <= NODE_MAX_MULT):
        return False
    if not 1 <= len(lvals) <= 32:
        return False
    return all(p is None or (p.dtype == torch.float32 and p.device == x.device) for p in params)


def _node_rows(x: torch.Tensor, mult: int, dim: int) -> int:
    if x.dim() < 2 or x.shape[-2] != mult or x.shape[-1] != dim:
        raise RuntimeError(f"node features must be (..., {mult}, {dim}); got {tuple(x.shape)}")
    return x.numel() // (mult * dim) if x.numel() else 0


def _c(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.detach().contiguous()


class SepNormFn(torch.autograd.Function):
    """SeparableEquivariantLayerNorm (norm.py:177-246) on feq_sepnorm_fwd/bwd.
    ``cm``: the output (and its gradient) component-major (dim, N, mult),
    feq_sepnorm_fwd_cm / _bwd_cm (the input stays node-major).  ``alias``: also
    returns the input (as a view) for a second branch; that branch's gradient
    is added inside the backward kernel (feq_sepnorm_bwd_add) instead of by
    autograd in a separate pass."""

    @staticmethod
    def forward(ctx, x, w_s, b_s, w_h, lvals, mult, eps, cm=False, alias=False):
        dim = sum(2 * l + 1 for l in lvals)
        xs = x.contiguous()
        n = _node_rows(xs, mult, dim)
        w_s, b_s, w_h = _c(w_s), _c(b_s), _c(w_h)
        y = torch.empty(dim, n, mult, dtype=xs.dtype, device=xs.device) if cm else torch.empty_like(xs)
        if n:
            fn = N.lib().feq_sepnorm_fwd_cm if cm else N.lib().feq_sepnorm_fwd
            with torch.cuda.device(xs.device):
                rc = fn(_lvals_i32(lvals), len(lvals), mult, n, N.ptr(xs), N.ptr(w_s), N.ptr(b_s),
                        N.ptr(w_h), eps, N.ptr(y), N.stream_ptr(xs.device))
            N.check(rc, "feq_sepnorm_fwd")
        ctx.save_for_backward(xs, w_s, b_s, w_h)
        ctx.meta = (lvals, mult, eps, n, cm)
        if alias:
            ctx.set_materialize_grads(False)
            return y, xs.view_as(xs)
        return y

    @staticmethod
    def backward(ctx, gy, ga=None):
        xs, w_s, b_s, w_h = ctx.saved_tensors
        lvals, mult, eps, n, cm = ctx.meta
        if gy is None:
            return ga, None, None, None, None, None, None, None, None
        gy = gy.contiguous()
        dev = xs.device
        gx = torch.empty_like(xs)
        gws = torch.empty_like(w_s) if w_s is not None else None
        gbs = torch.empty_like(b_s) if b_s is not None else None
        gwh = torch.empty_like(w_h) if w_h is not None else None
        lib = N.lib()
        arr = _lvals_i32(lvals)
        ws = N.workspace(lib.feq_sepnorm_workspace(arr, len(lvals), mult, n), dev)
        with torch.cuda.device(dev):
            if ga is not None:
                ga = ga.contiguous()
                rc = lib.feq_sepnorm_bwd_add(arr, len(lvals), mult, n, N.ptr(gy), N.ptr(xs), N.ptr(w_s),
                                             N.ptr(w_h), eps, N.ptr(ga), N.ptr(gx), N.ptr(gws), N.ptr(gbs),
                                             N.ptr(gwh), N.ptr(ws), ws.numel(), int(cm), N.stream_ptr(dev))
            else:
                fn = lib.feq_sepnorm_bwd_cm if cm else lib.feq_sepnorm_bwd
                rc = fn(arr, len(lvals), mult, n, N.ptr(gy), N.ptr(xs), N.ptr(w_s), N.ptr(w_h), eps, N.ptr(gx),
                        N.ptr(gws), N.ptr(gbs), N.ptr(gwh), N.ptr(ws), ws.numel(), N.stream_ptr(dev))
        N.check(rc, "feq_sepnorm_bwd")
        return gx, gws, gbs, gwh, None, None, None, None, None


class EqNormFn(torch.autograd.Function):
    """EquivariantLayerNorm (norm.py:148-174) on feq_eqnorm_fwd/bwd.  ``cm``:
    the output (and its gradient) component-major (dim, N, mult),
    feq_eqnorm_fwd_cm / _bwd_cm (the input stays node-major).  ``alias``: as
    SepNormFn's (feq_eqnorm_bwd_add)."""

    @staticmethod
    def forward(ctx, x, w_ln, b_ln, lvals, mult, eps, ln_eps, cm=False, alias=False):
        dim = sum(2 * l + 1 for l in lvals)
        xs = x.contiguous()
        n = _node_rows(xs, mult, dim)
        w_ln, b_ln = _c(w_ln), _c(b_ln)
        y = torch.empty(dim, n, mult, dtype=xs.dtype, device=xs.device) if cm else torch.empty_like(xs)
        if n:
            fn = N.lib().feq_eqnorm_fwd_cm if cm else N.lib().feq_eqnorm_fwd
            with torch.cuda.device(xs.device):
                rc = fn(_lvals_i32(lvals), len(lvals), mult, n, N.ptr(xs),
                                            N.ptr(w_ln), N.ptr(b_ln), eps, ln_eps, N.ptr(y),
                                            N.stream_ptr(xs.device))
            N.check(rc, "feq_eqnorm_fwd")
        ctx.save_for_backward(xs, w_ln, b_ln)
        ctx.meta = (lvals, mult, eps, ln_eps, n, cm)
        if alias:
            ctx.set_materialize_grads(False)
            return y, xs.view_as(xs)
        return y

    @staticmethod
    def backward(ctx, gy, ga=None):
        xs, w_ln, b_ln = ctx.saved_tensors
        lvals, mult, eps, ln_eps, n, cm = ctx.meta
        if gy is None:
            return ga, None, None, None, None, None, None, None, None
        gy = gy.contiguous()
        dev = xs.device
        gx = torch.empty_like(xs)
        gw = torch.empty_like(w_ln) if w_ln is not None else None
        gb = torch.empty_like(b_ln) if b_ln is not None else None
        lib = N.lib()
        arr = _lvals_i32(lvals)
        ws = N.workspace(lib.feq_eqnorm_workspace(arr, len(lvals), mult, n), dev)
        with torch.cuda.device(dev):
            if ga is not None:
                ga = ga.contiguous()
                rc = lib.feq_eqnorm_bwd_add(arr, len(lvals), mult, n, N.ptr(gy), N.ptr(xs), N.ptr(w_ln),
                                            N.ptr(b_ln), eps, ln_eps, N.ptr(ga), N.ptr(gx), N.ptr(gw), N.ptr(gb),
                                            N.ptr(ws), ws.numel(), int(cm), N.stream_ptr(dev))
            else:
                fn = lib.feq_eqnorm_bwd_cm if cm else lib.feq_eqnorm_bwd
                rc = fn(arr, len(lvals), mult, n, N.ptr(gy), N.ptr(xs), N.ptr(w_ln), N.ptr(b_ln), eps, ln_eps,
                        N.ptr(gx), N.ptr(gw), N.ptr(gb), N.ptr(ws), ws.numel(), N.stream_ptr(dev))
        N.check(rc, "feq_eqnorm_bwd")
        return gx, gw, gb, None, None, None, None, None, None


def transpose_last2(t: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """A contiguous tensor read as (batch, rows, cols) -> a new (batch, cols, rows)
    tensor (feq_transpose: LDS-tiled, reads and writes in consecutive addresses).
    The caller reshapes the result.  CPU tensors (host-side tests of the
    layers' index logic) are transposed by PyTorch."""
    if not t.is_contiguous():
        raise RuntimeError("transpose_last2: the input must be contiguous")
    n = t.numel()
    if rows * cols == 0 or n % (rows * cols):
        if n == 0:
            return torch.empty_like(t)
        raise RuntimeError(f"transpose_last2: {n} elements are not a batch of {rows} x {cols}")
    if not t.is_cuda:
        return t.view(-1, rows, cols).transpose(1, 2).contiguous().view(t.shape)
    out = torch.empty_like(t)
    with torch.cuda.device(t.device):
        rc = N.lib().feq_transpose(N.ptr(t), n // (rows * cols), rows, cols, t.element_size(),
                                   N.ptr(out), N.stream_ptr(t.device))
    N.check(rc, "feq_transpose")
    return out


def column_sums(t: torch.Tensor) -> torch.Tensor:
    """Sum over the rows of a 2-D tensor (feq_column_sums: one pass at memory
    speed, partial sums per row chunk combined in a fixed order, so the result
    is the same on every run).  Half precision, and CPU tensors (host-side
    tests), go through PyTorch's sum."""
    if t.dtype not in (torch.float32, torch.float64) or not t.is_cuda:
        return t.sum(0)
    ts = t.contiguous()
    rows, cols = ts.shape
    out = torch.empty(cols, dtype=ts.dtype, device=ts.device)
    lib = N.lib()
    es = ts.element_size()
    ws = N.workspace(lib.feq_column_sums_workspace(rows, cols, es), ts.device)
    with torch.cuda.device(ts.device):
        rc = lib.feq_column_sums(N.ptr(ts), rows, cols, es, N.ptr(out), N.ptr(ws), ws.numel(),
                                 N.stream_ptr(ts.device))
    N.check(rc, "feq_column_sums")
    return out


def dot_f64(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """sum(a * b) over all elements, the products and their sum in float64
    (one scalar from many products that largely cancel; a float32 sum of a
    million of them loses several digits).  float32 GPU inputs: feq_dot_f64 (no
    float64 copies); others (float64, CPU tensors): PyTorch in float64.  Returns a float32 0-d tensor
    for float32 inputs, else float64."""
    if a.dtype == torch.float32 and b.dtype == torch.float32 and a.is_cuda:
        a_, b_ = a.detach().contiguous(), b.detach().contiguous()
        if a_.numel() != b_.numel():
            raise RuntimeError(f"dot_f64: {a_.numel()} and {b_.numel()} elements")
        out = torch.empty((), dtype=torch.float32, device=a_.device)
        lib = N.lib()
        ws = N.workspace(lib.feq_dot_f64_workspace(), a_.device)
        with torch.cuda.device(a_.device):
            rc = lib.feq_dot_f64(N.ptr(a_), N.ptr(b_), a_.numel(), N.ptr(out), N.ptr(ws),
                                 ws.numel(), N.stream_ptr(a_.device))
        N.check(rc, "feq_dot_f64")
        return out
    return torch.dot(a.reshape(-1).double(), b.reshape(-1).double())


class BiasRowsFn(torch.autograd.Function):
    """y + b for y (rows, n) and b (n,); the bias gradient by column_sums."""

    @staticmethod
    def forward(ctx, y, b):
        return y + b

    @staticmethod
    def backward(ctx, gy):
        gb = column_sums(gy.reshape(-1, gy.shape[-1])) if ctx.needs_input_grad[1] else None
        return gy, gb


class ScaleFn(torch.autograd.Function):
    """x * g for a scalar parameter g; its gradient is one dot product (float64
    accumulation: the products cancel, and a float32 sum of a million of them
    loses several digits)."""

    @staticmethod
    def forward(ctx, x, g):
        ctx.save_for_backward(x, g)
        return x * g

    @staticmethod
    def backward(ctx, gy):
        x, g = ctx.saved_tensors
        gx = gy * g if ctx.needs_input_grad[0] else None
        gg = None
        if ctx.needs_input_grad[1]:
            # one scalar from many products that largely cancel: accumulated in float64
            gg = dot_f64(gy, x).reshape(g.shape).to(g.dtype)
        return gx, gg


class ResidualScaleFn(torch.autograd.Function):
    """x + gamma * y for a scalar parameter gamma: the transformer block's
    residual connection with LayerScale (transformer.py:245, :252 and
    LayerScale :23-38 of the reference) in one pass (feq_scale_add).  The
    backward forms grad_y = gamma g and grad_gamma = sum g y (float64 products
    and sum, fixed order) in one pass (feq_scale_add_bwd); grad_x is g itself."""

    @staticmethod
    def forward(ctx, x, y, gamma):
        xs, ys = x.contiguous(), y.contiguous()
        if xs.shape != ys.shape:
            raise RuntimeError(f"residual: shapes {tuple(xs.shape)} and {tuple(ys.shape)}")
        out = torch.empty_like(xs)
        with torch.cuda.device(xs.device):
            rc = N.lib().feq_scale_add(N.ptr(xs), N.ptr(ys), N.ptr(gamma), xs.numel(), N.ptr(out),
                                       N.stream_ptr(xs.device))
        N.check(rc, "feq_scale_add")
        ctx.save_for_backward(ys, gamma)
        return out

    @staticmethod
    def backward(ctx, g):
        ys, gamma = ctx.saved_tensors
        g = g.contiguous()
        gy = torch.empty_like(g) if ctx.needs_input_grad[1] else None
        gg = torch.empty((), dtype=torch.float32, device=g.device) if ctx.needs_input_grad[2] else None
        if gy is not None or gg is not None:
            lib = N.lib()
            ws = N.workspace(lib.feq_dot_f64_workspace(), g.device)
            with torch.cuda.device(g.device):
                rc = lib.feq_scale_add_bwd(N.ptr(g), N.ptr(ys), N.ptr(gamma), g.numel(),
                                           N.ptr(gy) if gy is not None else None,
                                           N.ptr(gg) if gg is not None else None, N.ptr(ws), ws.numel(),
                                           N.stream_ptr(g.device))
            N.check(rc, "feq_scale_add_bwd")
        return (g if ctx.needs_input_grad[0] else None, gy,
                gg.reshape(gamma.shape) if gg is not None else None)


class ResidualScaleCmFn(torch.autograd.Function):
    """x + gamma * y with x node-major (N, mult, dim) and y component-major
    (dim, N, mult), returned node-major (feq_scale_add_cm): the block's MLP
    output joins the residual stream without a separate transpose.  The
    backward forms grad_y (component-major) and grad_gamma (float64 products
    and sum, fixed order) in one pass (feq_scale_add_cm_bwd); grad_x is g."""

    @staticmethod
    def forward(ctx, x, y, gamma):
        xs, ys = x.contiguous(), y.contiguous()
        n, mult, dim = xs.shape[0], xs.shape[1], xs.shape[2]
        if ys.shape != (dim, n, mult):
            raise RuntimeError(f"residual: component-major branch {tuple(ys.shape)} for rows {tuple(xs.shape)}")
        out = torch.empty_like(xs)
        with torch.cuda.device(xs.device):
            rc = N.lib().feq_scale_add_cm(N.ptr(xs), N.ptr(ys), N.ptr(gamma), n, mult, dim, N.ptr(out),
                                          N.stream_ptr(xs.device))
        N.check(rc, "feq_scale_add_cm")
        ctx.save_for_backward(ys, gamma)
        ctx.meta = (n, mult, dim)
        return out

    @staticmethod
    def backward(ctx, g):
        ys, gamma = ctx.saved_tensors
        n, mult, dim = ctx.meta
        g = g.contiguous()
        gy = torch.empty_like(ys) if ctx.needs_input_grad[1] else None
        gg = torch.empty((), dtype=torch.float32, device=g.device) if ctx.needs_input_grad[2] else None
        if gy is not None or gg is not None:
            lib = N.lib()
            ws = N.workspace(lib.feq_scale_add_cm_workspace(), g.device)
            with torch.cuda.device(g.device):
                rc = lib.feq_scale_add_cm_bwd(N.ptr(g), N.ptr(ys), N.ptr(gamma), n, mult, dim,
                                              N.ptr(gy) if gy is not None else None,
                                              N.ptr(gg) if gg is not None else None, N.ptr(ws), ws.numel(),
                                              N.stream_ptr(g.device))
            N.check(rc, "feq_scale_add_cm_bwd")
        return (g if ctx.needs_input_grad[0] else None, gy,
                gg.reshape(gamma.shape) if gg is not None else None)


def rows_weight_grad(gy: torch.Tensor, x: torch.Tensor, dtype: torch.dtype,
                     chunks: int = 64) -> torch.Tensor:
    """gy^T x over many rows, as a batched GEMM over row chunks whose partial
    products are summed in float32 (or the inputs' wider type).  As one GEMM
    (M = out, N = in, K = rows) the library runs it on a few output tiles (about
    5 TFLOP/s at 100k rows on MI355X)."""
    rows = x.shape[0]
    s = chunks if rows >= 64 * chunks else 1
    per = rows // s
    head = s * per
    if gy.dtype in (torch.float32, torch.float64):
        # the chunks of gy as transposed views: the library reads the transposed
        # operand in place
        gyc = gy[:head].contiguous().view(s, per, gy.shape[1]).transpose(1, 2)
    else:
        # 16-bit batched products take no transposed views here (copied instead)
        gyc = transpose_last2(gy[:head].contiguous(), per, gy.shape[1]).view(s, gy.shape[1], per)
    xc = x[:head].reshape(s, per, x.shape[1])
    acc = torch.promote_types(dtype, torch.float32)
    gw = column_sums(torch.bmm(gyc, xc).to(acc).reshape(s, -1)).view(gy.shape[1], x.shape[1])
    if head < rows:
        gw = gw + torch.mm(gy[head:].t().to(acc), x[head:].to(acc))
    return gw.to(dtype)


class FanOutFn(torch.autograd.Function):
    """k views of one tensor for k consumers; the backward sums their
    gradients in one pass (feq_sum_tables, in consumer order) where autograd
    would add them pairwise (k - 1 passes over three tables each)."""

    @staticmethod
    def forward(ctx, x, k: int):
        ctx.set_materialize_grads(False)
        return tuple(x.view_as(x) for _ in range(k))

    @staticmethod
    def backward(ctx, *grads):
        gs = [g for g in grads if g is not None]
        if not gs:
            return None, None
        if len(gs) == 1:
            return gs[0], None
        if (all(g.is_cuda and g.dtype == torch.float32 and g.shape == gs[0].shape for g in gs)
                and len(gs) <= 16):
            gc = [g.contiguous() for g in gs]
            out = torch.empty_like(gc[0])
            ptrs = (N.ctypes.c_void_p * len(gc))(*[g.data_ptr() for g in gc])
            with torch.cuda.device(out.device):
                rc = N.lib().feq_sum_tables(ptrs, len(gc), out.numel(), N.ptr(out), N.stream_ptr(out.device))
            N.check(rc, "feq_sum_tables")
            return out, None
        out = gs[0].clone()
        for g in gs[1:]:
            out += g
        return out, None


class GatingFn(torch.autograd.Function):
    """EquivariantGating (gating.py:54-76): irrep norms and the sigmoid gate
    in kernels (feq_gate_*), the Linear over the flattened norms as a GEMM."""

    @staticmethod
    def forward(ctx, x, weight, bias, lvals, mult, eps, cm=False):
        """x: (..., mult, dim), or (dim, N, mult) with cm (component-major)."""
        dim = sum(2 * l + 1 for l in lvals)
        nreps = len(lvals)
        xs = x.contiguous()
        if cm:
            if xs.dim() != 3 or xs.shape[0] != dim or xs.shape[2] != mult:
                raise RuntimeError(f"component-major features must be ({dim}, N, {mult}); "
                                   f"got {tuple(xs.shape)}")
            n = xs.shape[1]
        else:
            n = _node_rows(xs, mult, dim)
        dev = xs.device
        lib = N.lib()
        arr = _lvals_i32(lvals)
        norms = torch.empty(n, mult * nreps, dtype=torch.float32, device=dev)
        with torch.cuda.device(dev):
            rc = lib.feq_gate_norms(arr, nreps, mult, n, int(cm), N.ptr(xs), eps, N.ptr(norms),
                                    N.stream_ptr(dev))
        N.check(rc, "feq_gate_norms")
        lin = torch.addmm(bias.detach(), norms, weight.detach().t())
        y = torch.empty_like(xs)
        with torch.cuda.device(dev):
            rc = lib.feq_gate_apply(arr, nreps, mult, n, int(cm), N.ptr(xs), N.ptr(lin), N.ptr(y),
                                    N.stream_ptr(dev))
        N.check(rc, "feq_gate_apply")
        ctx.save_for_backward(xs, weight, norms, lin)
        ctx.meta = (lvals, mult, n, cm)
        return y

    @staticmethod
    def backward(ctx, gy):
        xs, weight, norms, lin = ctx.saved_tensors
        lvals, mult, n, cm = ctx.meta
        gy = gy.contiguous()
        dev = xs.device
        lib = N.lib()
        arr = _lvals_i32(lvals)
        nreps = len(lvals)
        dlin = torch.empty_like(lin)
        with torch.cuda.device(dev):
            rc = lib.feq_gate_bwd_lin(arr, nreps, mult, n, int(cm), N.ptr(gy), N.ptr(xs),
                                      N.ptr(lin), N.ptr(dlin), N.stream_ptr(dev))
        N.check(rc, "feq_gate_bwd_lin")
        dnorms = torch.mm(dlin, weight.detach())
        gw = rows_weight_grad(dlin, norms, weight.dtype) if ctx.needs_input_grad[1] else None
        gb = column_sums(dlin) if ctx.needs_input_grad[2] else None
        gx = torch.empty_like(xs)
        with torch.cuda.device(dev):
            rc = lib.feq_gate_bwd_x(arr, nreps, mult, n, int(cm), N.ptr(gy), N.ptr(xs),
                                    N.ptr(lin), N.ptr(norms), N.ptr(dnorms), N.ptr(gx),
                                    N.stream_ptr(dev))
        N.check(rc, "feq_gate_bwd_x")
        return gx, gw, gb, None, None, None, None


def _slice_lvals(slices) -> Tuple[int, ...]:
    return tuple((b - a - 1) // 2 for a, b in slices)


def eqlinear_kernels_ok(fd: torch.Tensor, weight: torch.Tensor, slices, cin: int, cout: int) -> bool:
    """One ``feq_eqlinear_*`` launch per map: float32 GPU tables, channel
    counts the kernels have (32, 64 or 128 each), at most 16 irreps and
    64 components.  ``FEQ_EQLINEAR=lib`` keeps the per-irrep library GEMMs."""
    return (fd.is_cuda and fd.dtype == torch.float32 and weight.dtype == torch.float32
            and os.environ.get("FEQ_EQLINEAR") != "lib" and len(slices) <= 16
            and slices[-1][1] <= 64 and bool(N.lib().feq_eqlinear_supported(cin, cout)))


class EqLinearFn(torch.autograd.Function):
    """EquivariantLinear (linear.py:242-268) in component-major form: one
    feq_eqlinear_* launch per direction over every irrep (split-fp16 matrix-core
    products, float32 accuracy), or, where those kernels lack the channel
    counts, one library GEMM per irrep, (rows * (2l+1), cin) x (cin, cout),
    written straight into its slice of a (dim, rows, cout) table; the bias of
    the j-th scalar irrep is the GEMM's bias column.  Input and output are node-major
    (rows, c, dim) or, with in_cm / out_cm, component-major (dim, rows, c), so
    consecutive linear maps and the gating can skip the transposes."""

    @staticmethod
    def forward(ctx, f, weight, bias, slices, bias_cols, cin, cout, in_cm, out_cm):
        if in_cm:
            fd = f.contiguous()
        else:
            D = f.shape[-1]
            fc = f.contiguous()
            fd = transpose_last2(fc, fc.numel() // D, D).view(D, -1, cin)
        D, rows = fd.shape[0], fd.shape[1]
        w = weight.detach().view(-1, cout, cin)
        out = torch.empty(D, rows, cout, dtype=fd.dtype, device=fd.device)
        if eqlinear_kernels_ok(fd, weight, slices, cin, cout):
            lib = N.lib()
            nreps = len(slices)
            wc = weight.detach().contiguous()
            bc = bias.detach().contiguous() if bias is not None else None
            ws = N.workspace(lib.feq_eqlinear_workspace(nreps, cin, cout), fd.device)
            with torch.cuda.device(fd.device):
                rc = lib.feq_eqlinear_fwd(_lvals_i32(_slice_lvals(slices)), nreps, rows, cin, cout,
                                          N.ptr(fd), N.ptr(wc), N.ptr(bc) if bc is not None else None,
                                          bc.shape[1] if bc is not None else 0,
                                          _lvals_i32(bias_cols) if bc is not None else None, N.ptr(out),
                                          N.ptr(ws), ws.numel(), N.stream_ptr(fd.device))
            N.check(rc, "feq_eqlinear_fwd")
        else:
            for k, (a, b) in enumerate(slices):
                xk = fd[a:b].view(-1, cin)
                ok = out[a:b].view(-1, cout)
                j = bias_cols[k]
                if bias is not None and j >= 0:
                    torch.addmm(bias.detach()[:, j], xk, w[k].t(), out=ok)
                else:
                    torch.mm(xk, w[k].t(), out=ok)
        ctx.save_for_backward(fd, weight, bias)
        ctx.meta = (slices, bias_cols, cin, cout, in_cm, out_cm, tuple(f.shape))
        return out if out_cm else transpose_last2(out, D, rows * cout).view(rows, cout, D)

    @staticmethod
    def backward(ctx, gy):
        fd, weight, bias = ctx.saved_tensors
        slices, bias_cols, cin, cout, in_cm, out_cm, fshape = ctx.meta
        D = fd.shape[0]
        gyd = gy.contiguous()
        if not out_cm:
            gyd = transpose_last2(gyd, gyd.numel() // D, D).view(D, -1, cout)
        w = weight.detach().view(-1, cout, cin)
        gfd = torch.empty_like(fd) if ctx.needs_input_grad[0] else None
        gw = torch.empty_like(w) if ctx.needs_input_grad[1] else None
        gb = torch.zeros_like(bias) if bias is not None and ctx.needs_input_grad[2] else None
        fused_x = gfd is not None and eqlinear_kernels_ok(gyd, weight, slices, cin, cout)
        if fused_x:
            lib = N.lib()
            nreps = len(slices)
            wc = weight.detach().contiguous()
            ws = N.workspace(lib.feq_eqlinear_workspace(nreps, cin, cout), gyd.device)
            with torch.cuda.device(gyd.device):
                rc = lib.feq_eqlinear_bwd_x(_lvals_i32(_slice_lvals(slices)), nreps, gyd.shape[1], cin,
                                            cout, N.ptr(gyd), N.ptr(wc), N.ptr(gfd), N.ptr(ws), ws.numel(),
                                            N.stream_ptr(gyd.device))
            N.check(rc, "feq_eqlinear_bwd_x")
        fused_w = (gw is not None or gb is not None) and eqlinear_kernels_ok(gyd, weight, slices, cin, cout)
        if fused_w:
            lib = N.lib()
            nreps = len(slices)
            lv = _lvals_i32(_slice_lvals(slices))
            rows = gyd.shape[1]
            gwk = gw if gw is not None else torch.empty_like(w)
            ws = N.workspace(lib.feq_eqlinear_bwd_w_workspace(lv, nreps, rows, cin, cout), gyd.device)
            with torch.cuda.device(gyd.device):
                rc = lib.feq_eqlinear_bwd_w(lv, nreps, rows, cin, cout, N.ptr(gyd), N.ptr(fd),
                                            gb.shape[1] if gb is not None else 0,
                                            _lvals_i32(bias_cols) if gb is not None else None, N.ptr(gwk),
                                            N.ptr(gb) if gb is not None else None, N.ptr(ws), ws.numel(),
                                            N.stream_ptr(gyd.device))
            N.check(rc, "feq_eqlinear_bwd_w")
        for k, (a, b) in enumerate(slices):
            gk = gyd[a:b].view(-1, cout)
            if gfd is not None and not fused_x:
                torch.mm(gk, w[k], out=gfd[a:b].view(-1, cin))
            if gw is not None and not fused_w:
                gw[k] = rows_weight_grad(gk, fd[a:b].view(-1, cin), weight.dtype)
            if gb is not None and bias_cols[k] >= 0 and not fused_w:
                gb[:, bias_cols[k]] = column_sums(gk)
        gx = None
        if gfd is not None:
            gx = gfd if in_cm else transpose_last2(gfd, D, gfd.numel() // D).view(fshape)
        return (gx, gw.view_as(weight) if gw is not None else None, gb,
                None, None, None, None, None, None)


class RadialMLPFn(torch.autograd.Function):
    """The radial network of ``SeparableRadialNet`` at the bin edges
    (``radial.py:200-275``): F = head(silu(W2 silu(W1 basis + b1) + b2)) + b3 as
    ``feq_radial_fwd`` (a workgroup per row) and the parameter gradients as
    ``feq_radial_bwd`` (per-row gradients, then one thread per weight summing
    the rows in order: deterministic).  basis needs no gradient (it is formed
    from buffers)."""

    @staticmethod
    def forward(ctx, basis, W1, b1, W2, b2, W3, b3):
        B, I = basis.shape
        H, O = W1.shape[0], W3.shape[0]
        dev = basis.device
        F = torch.empty(B, O, dtype=torch.float32, device=dev)
        acts = torch.empty(B, 4 * H, dtype=torch.float32, device=dev)
        ts = [t.detach().contiguous() for t in (basis, W1, b1, W2, b2, W3, b3)]
        with torch.cuda.device(dev):
            rc = N.lib().feq_radial_fwd(N.ptr(ts[0]), B, I, H, O, *[N.ptr(t) for t in ts[1:]], N.ptr(F),
                                        N.ptr(acts), N.stream_ptr(dev))
        N.check(rc, "feq_radial_fwd")
        ctx.save_for_backward(ts[0], ts[3], ts[5], acts)
        ctx.meta = (I, H, O, W1.shape, b1.shape)
        return F

    @staticmethod
    def backward(ctx, gF):
        basis, W2, W3, acts = ctx.saved_tensors
        I, H, O, w1s, b1s = ctx.meta
        B = basis.shape[0]
        dev = basis.device
        g = gF.detach().to(torch.float32).contiguous()
        grads = [torch.empty(w1s, device=dev), torch.empty(b1s, device=dev), torch.empty_like(W2),
                 torch.empty(H, device=dev), torch.empty_like(W3), torch.empty(O, device=dev)]
        lib = N.lib()
        ws = N.workspace(lib.feq_radial_workspace(B, H), dev)
        with torch.cuda.device(dev):
            rc = lib.feq_radial_bwd(N.ptr(basis), B, I, H, O, N.ptr(W2), N.ptr(W3), N.ptr(acts), N.ptr(g),
                                    *[N.ptr(t) for t in grads], N.ptr(ws), ws.numel(), N.stream_ptr(dev))
        N.check(rc, "feq_radial_bwd")
        return (None, *grads)


def radial_mlp_supported(rows: int, in_dim: int, hidden: int, out_dim: int) -> bool:
    return bool(N.lib().feq_radial_supported(rows, in_dim, hidden, out_dim))


class SumSquaresFn(torch.autograd.Function):
    """sum(y ** 2) of a float32 or bfloat16 GPU tensor (feq_sum_squares /
    feq_sum_squares_bf16: float32 sums, deterministic, graph capturable), a
    float32 scalar; the gradient 2 y g in one elementwise pass, in y's dtype."""

    @staticmethod
    def forward(ctx, y):
        N.require_cuda_tensor(y, "sum-of-squares input")
        if y.dtype not in (torch.float32, torch.bfloat16):
            raise TypeError(f"SumSquaresFn: float32 or bfloat16 expected, got {y.dtype}")
        ys = y.contiguous()
        out = torch.empty((), dtype=torch.float32, device=ys.device)
        lib = N.lib()
        fn = lib.feq_sum_squares if ys.dtype == torch.float32 else lib.feq_sum_squares_bf16
        ws = N.workspace(lib.feq_sum_squares_workspace(), ys.device)
        with torch.cuda.device(ys.device):
            rc = fn(N.ptr(ys), ys.numel(), N.ptr(out), N.ptr(ws), ws.numel(), N.stream_ptr(ys.device))
        N.check(rc, "feq_sum_squares")
        ctx.save_for_backward(ys)
        return out

    @staticmethod
    def backward(ctx, g):
        (ys,) = ctx.saved_tensors
        # the scalar in y's dtype: a same-dtype product needs no per-element casts
        return ys * (2.0 * g).to(ys.dtype)
