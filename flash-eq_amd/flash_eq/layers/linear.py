"""SO(3)-equivariant linear layers (drop-in for ``flash_eq/layers/linear.py``).

``EquivariantEdgewiseLinear`` computes ``out = Q Lambda(r) P^T f`` per edge
(``linear.py:100-160``) in ONE fused HIP pass per direction
(``csrc/edgewise.hip``): rotate into the m-first frame with P, apply the
binned, interpolated, solid-harmonic-scaled radial weights in their separable
form ``sum_k C_k (x) F_k`` (the ``SeparableRadialNet`` factors), rotate back
with Q.  Neither the rotated features nor the (num_bins+1, Cout, Cin, Wdim)
table are written to memory.

``EquivariantLinear`` is the node-side per-degree channel mix
(``linear.py:172-268``); it is O(N) work and stays a PyTorch matmul.
"""
from __future__ import annotations

import os
from functools import lru_cache
from typing import Tuple

import torch
import torch.nn as nn

from .. import _native as N
from ..ops import (_use_hl, edgewise_attention_pool, edgewise_linear, edgewise_linear_src,
                   edgewise_pool_supported, edgewise_pq_supported, edgewise_src_supported,
                   embedding_for, rows_weight_grad, BiasRowsFn, EqLinearFn)
from ..representations import ProductRepr, Repr
from .radial import SeparableRadialNet
from ..utils import half_precision_active


class RowsLinearFn(torch.autograd.Function):
    """y = x W^T for x (rows, in) with many rows.  The weight gradient
    dy^T x reduces over every row; as one GEMM (M = out, N = in, K = rows) the
    library runs it on a few output tiles (about 5 TFLOP/s at 100k rows on
    MI355X), so it is formed as a batched GEMM over row chunks whose partial
    products are summed in float32 (or the inputs' wider type)."""

    CHUNKS = 64

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return torch.mm(x, w.t())

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        gx = torch.mm(gy, w) if ctx.needs_input_grad[0] else None
        gw = rows_weight_grad(gy, x, w.dtype, RowsLinearFn.CHUNKS) if ctx.needs_input_grad[1] else None
        return gx, gw


def rows_linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return RowsLinearFn.apply(x, w)


@lru_cache(maxsize=256)
def _layout(lvals_in: Tuple[int, ...], lvals_out: Tuple[int, ...], cin: int, cout: int):
    return N.make_layout(lvals_in, lvals_out, cin, cout)


class EquivariantEdgewiseLinear(nn.Module):
    """Edge-to-edge equivariant linear map with distance-dependent binned weights."""

    radial_weights: SeparableRadialNet

    def __init__(self, in_repr: Repr, out_repr: Repr, num_bins: int = 100, rank: int = 4,
                 hidden_dim: int = 64, min_dist: float = 0.0, max_dist: float = 10.0,
                 log_bins: bool = False, solid_harmonic_scale: float = 0.1) -> None:
        super().__init__()
        self.in_repr = in_repr
        self.out_repr = out_repr
        self.rank = rank
        self.solid_harmonic_scale = solid_harmonic_scale
        self.product_repr = ProductRepr(in_repr, out_repr)
        self.weight_dim = self.product_repr.nreps()
        self.channels_in = in_repr.mult
        self.channels_out = out_repr.mult
        self.radial_weights = SeparableRadialNet(
            num_bins=num_bins, out_mult=self.channels_out, in_mult=self.channels_in,
            weight_dim=self.weight_dim, rank=rank, hidden_dim=hidden_dim,
            min_val=min_dist, max_val=max_dist, log=log_bins)
        self._lin = tuple(int(l) for l in in_repr.lvals.tolist())
        self._lout = tuple(int(l) for l in out_repr.lvals.tolist())

    def layout(self) -> N.FeqLayout:
        return _layout(self._lin, self._lout, self.channels_in, self.channels_out)

    # below this many edges the shape-generic kernels beat the padded fast ones
    EMBED_MIN_EDGES = 4096

    def _embedding(self, x, num_edges, layout, binning, pq: bool = False):
        """The zero-embedding into the [0,1,2]x64 kernels when this layout has no
        split-fp16 backward of its own (with ``pq``: none that forms the bases'
        gradients), else None (only canonical prefixes of [0, 1, 2] with at
        most 64 channels embed).  ``FEQ_EW_PATH`` other than the default keeps
        the layout's own kernels."""
        if os.environ.get("FEQ_EW_PATH") or os.environ.get("FEQ_FORCE_GENERIC") == "1":
            return None
        if num_edges < self.EMBED_MIN_EDGES:
            return None
        rank = self.radial_weights.rank
        own = (edgewise_pq_supported(layout, binning, rank) if pq
               else edgewise_src_supported(layout, binning, rank))
        if own:
            return None
        emb = embedding_for(self._lin, self._lout, self.channels_in, self.channels_out, rank, x.device)
        if emb is not None and pq and not edgewise_pq_supported(emb.layout, binning, rank):
            return None
        return emb

    def binning(self) -> N.FeqBinning:
        rw = self.radial_weights
        p1, p2 = rw.binning_params()
        return N.make_binning(p1, p2, rw.num_bins, rw.log, self.solid_harmonic_scale)

    def forward(self, P: torch.Tensor, Q: torch.Tensor, edge_features: torch.Tensor,
                distances: torch.Tensor, *, graph=None) -> torch.Tensor:
        """P (E, Din, Din), Q (E, Dout, Dout), edge_features (E, Cin, Din), distances (E,)
        -> (E, Cout, Dout), all in the standard SH basis.

        ``graph`` (keyword, not in the reference): ``edge_features`` then holds node
        features (N, Cin, Din) and edge e reads row ``graph.src[e]``, i.e. the layer
        of ``graph.gather_src(edge_features)``.  Where the fused kernels have the
        layout, the gather happens inside them and its backward is a segmented sum
        over the graph's CSR by source; otherwise the rows are gathered first."""
        N.require_cuda_tensor(edge_features, "edge_features")
        rw = self.radial_weights
        if edge_features.dtype == torch.float64:
            return self._forward_composed(P, Q, edge_features, distances, graph, torch.float64)
        layout, binning = self.layout(), self.binning()
        if not (_use_hl(edge_features, P, Q, layout, binning, rw.rank)
                or N.lib().feq_edgewise_fused_supported(N.ctypes.byref(layout), N.ctypes.byref(binning),
                                                        rw.rank)):
            # wider than the fused kernels' LDS (e.g. lvals 0..6 at 64+ channels
            # in float32): the reference's own composition, in float32
            out = self._forward_composed(P, Q, edge_features, distances, graph, torch.float32)
            return out.to(edge_features.dtype)
        pq = torch.is_grad_enabled() and (P.requires_grad or Q.requires_grad)
        emb = self._embedding(edge_features, distances.shape[0], layout, binning, pq)
        if pq and not edgewise_pq_supported(emb.layout if emb is not None else layout, binning, rw.rank):
            # gradients for the bases without split kernels that form them: the
            # shape-generic kernels do, on edge rows, so the gather (if any)
            # happens first
            if graph is not None:
                if graph.num_edges != distances.shape[0]:
                    raise ValueError(f"graph has {graph.num_edges} edges, distances {distances.shape[0]}")
                edge_features = graph.gather_src(edge_features)
            return edgewise_linear(edge_features, P, Q, distances, rw.channel_patterns,
                                   rw.radial_functions(), layout, binning, rw.rank)
        if emb is not None:
            # a small layout without split-fp16 backward kernels: run it
            # zero-embedded in the [0,1,2]x64 kernels (ops._Embedding)
            x = emb.features(edge_features)
            Pp, Qp = emb.basis_in(P), emb.basis_out(Q)
            C, F = emb.channels(rw.channel_patterns), emb.radial(rw.radial_functions())
            if graph is not None:
                if graph.num_edges != distances.shape[0]:
                    raise ValueError(f"graph has {graph.num_edges} edges, distances {distances.shape[0]}")
                perm, offsets = graph.csr_src()
                y = edgewise_linear_src(x, graph.src, perm, offsets, Pp, Qp, distances, C, F,
                                        emb.layout, binning, rw.rank,
                                        half_precision_active(edge_features))
            else:
                y = edgewise_linear(x, Pp, Qp, distances, C, F, emb.layout, binning, rw.rank)
            return emb.output(y)
        if graph is not None:
            if graph.num_edges != distances.shape[0]:
                raise ValueError(f"graph has {graph.num_edges} edges, distances {distances.shape[0]}")
            if edgewise_src_supported(layout, binning, rw.rank):
                perm, offsets = graph.csr_src()
                return edgewise_linear_src(edge_features, graph.src, perm, offsets, P, Q, distances,
                                           rw.channel_patterns, rw.radial_functions(), layout,
                                           binning, rw.rank, half_precision_active(edge_features))
            edge_features = graph.gather_src(edge_features)
        return edgewise_linear(edge_features, P, Q, distances, rw.channel_patterns,
                               rw.radial_functions(), layout, binning, rw.rank)

    def _forward_composed(self, P, Q, edge_features, distances, graph, dtype):
        """The reference's own composition (linear.py:131-160) in ``dtype``: x P by
        library bmm, the block-diagonal op on the full radial table
        (``block_diagonal_cuda``: blockdiag.hip's kernels, float32 and float64 as
        block_diagonal.cu:1332 dispatches), then by Q^T, every gradient
        (features, bases, radial network, distances) by autograd through it.
        float64 layers take it, and float32 layouts too wide for the fused
        kernels (their table, (num_bins+1) Cout Cin Wdim floats, is formed)."""
        from ..cuda.block_diagonal import block_diagonal_cuda
        if graph is not None:
            if graph.num_edges != distances.shape[0]:
                raise ValueError(f"graph has {graph.num_edges} edges, distances {distances.shape[0]}")
            edge_features = edge_features.index_select(0, graph.src)
        rw = self.radial_weights
        p1, p2 = rw.binning_params()
        f = torch.bmm(edge_features.to(dtype), P.to(dtype))
        out = block_diagonal_cuda(f, rw().to(dtype), distances.to(dtype), self.product_repr,
                                  bin_param1=p1, bin_param2=p2, num_bins=rw.num_bins, log_bins=rw.log,
                                  sh_scale=self.solid_harmonic_scale)
        return torch.bmm(out, Q.to(dtype).mT.contiguous())

    def attention_pool(self, P: torch.Tensor, Q: torch.Tensor, node_features: torch.Tensor,
                       distances: torch.Tensor, graph, attn: torch.Tensor, num_heads: int):
        """sum over the edges e into n of attn[e, head(c)] * layer(x[src])[e, c, :]:
        the layer in message-passing form fused with an attention's head
        weighting and sum pooling by destination (``attention.py:307-314``,
        ``pooling.py:21-30``), channel c in head c // (Cout / num_heads).  Returns
        (num_nodes, Cout, Dout), or None where the fused kernels do not cover the
        call (the caller then forms V and pools it)."""
        if not node_features.is_cuda or graph is None or graph.num_edges != distances.shape[0]:
            return None
        pq = torch.is_grad_enabled() and (P.requires_grad or Q.requires_grad)
        cout = self.channels_out
        if (num_heads < 1 or num_heads > N.POOL_MAX_HEADS or cout % num_heads
                or (cout // num_heads) % 4 or attn.shape != (graph.num_edges, num_heads)
                or graph.num_nodes < 1):
            return None
        rw = self.radial_weights
        layout, binning = self.layout(), self.binning()
        x, Pp, Qp, C, F, emb = node_features, P, Q, rw.channel_patterns, rw.radial_functions(), None
        if not edgewise_pool_supported(layout, binning, rw.rank):
            emb = self._embedding(node_features, distances.shape[0], layout, binning)
            if emb is None or emb.layout.cout != cout or not edgewise_pool_supported(emb.layout, binning,
                                                                                    rw.rank):
                return None
            x, Pp, Qp = emb.features(node_features), emb.basis_in(P), emb.basis_out(Q)
            C, F, layout = emb.channels(C), emb.radial(F), emb.layout
        if pq and not edgewise_pq_supported(layout, binning, rw.rank):
            return None   # the caller forms V (whose layer forms the bases' gradients) and pools it
        perm_s, offsets_s = graph.csr_src()
        perm_d, offsets_d = graph.csr()
        out = edgewise_attention_pool(x.contiguous(), attn, graph.src, graph.dst, perm_s, offsets_s,
                                      perm_d, offsets_d, graph.num_nodes, Pp, Qp, distances, C, F,
                                      layout, binning, rw.rank, num_heads, cout // num_heads,
                                      half_precision_active(node_features))
        return out if emb is None else emb.output(out)

    def extra_repr(self) -> str:
        rw = self.radial_weights
        spacing = "log" if rw.log else "linear"
        return (f"in_repr={self.in_repr}, out_repr={self.out_repr}, num_bins={rw.num_bins}, "
                f"dist=[{rw.min_val}, {rw.max_val}], spacing={spacing}, rank={self.rank}")


class EquivariantLinear(nn.Module):
    """Per-degree channel mixing of node features; bias/activation on scalars only."""

    def __init__(self, in_repr: Repr, out_repr: Repr, bias: bool = True,
                 activation: nn.Module | None = None) -> None:
        super().__init__()
        if not torch.equal(in_repr.lvals, out_repr.lvals):
            raise ValueError(
                "EquivariantLinear cannot modify the degrees of a representation. "
                f"Got input lvals={in_repr.lvals.tolist()}, output lvals={out_repr.lvals.tolist()}")
        self.in_repr = in_repr
        self.out_repr = out_repr
        self.weight = nn.Parameter(torch.empty(in_repr.nreps() * out_repr.mult, in_repr.mult))
        nn.init.xavier_uniform_(self.weight)
        self.register_buffer("indices", torch.tensor(in_repr.indices(), dtype=torch.long))
        offs = in_repr.cumdims().tolist()
        self._slices = [(offs[k], offs[k + 1]) for k in range(in_repr.nreps())]
        nscalar, locs = in_repr.find_scalar()
        self.scalar_locs = locs
        self.bias: nn.Parameter | None
        if nscalar > 0 and bias:
            self.bias = nn.Parameter(torch.zeros(out_repr.mult, nscalar), requires_grad=True)
        else:
            self.bias = None
        self.activation = activation if activation is not None else nn.Identity()
        # per irrep: the bias column of a scalar irrep, -1 otherwise
        self._bias_cols = tuple(locs.index(a) if (self.bias is not None and a in locs) else -1
                                for a, _ in self._slices)

    def fused_ok(self, f: torch.Tensor) -> bool:
        """Float32 GPU features without an activation take EqLinearFn."""
        return (f.is_cuda and f.dtype == torch.float32 and self.weight.dtype == torch.float32
                and isinstance(self.activation, nn.Identity))

    def forward_layout(self, f: torch.Tensor, in_cm: bool, out_cm: bool) -> torch.Tensor:
        """The map on node-major (rows, cin, dim) or component-major (dim, rows,
        cin) features (in_cm), returning either layout (out_cm); fused_ok(f)."""
        return EqLinearFn.apply(f, self.weight, self.bias, self._slices, self._bias_cols,
                                self.in_repr.mult, self.out_repr.mult, in_cm, out_cm)

    def forward(self, f: torch.Tensor) -> torch.Tensor:
        """(..., in_mult, dim) -> (..., out_mult, dim).

        Computed component-major: f is copied once to (dim, rows, in_mult), each
        irrep's components are one plain (components * rows, in_mult) x
        (in_mult, out_mult) GEMM, and the result is copied back.  (A matmul of
        the weight with the (rows, in_mult, 2l+1) slices broadcasts into one
        tiny GEMM per row, and its backward forms a weight gradient per row
        before summing them.)"""
        cin, cout = self.in_repr.mult, self.out_repr.mult
        lead = f.shape[:-2]
        if self.fused_ok(f):
            return self.forward_layout(f, False, False).view(*lead, cout, f.shape[-1])
        w = self.weight.view(self.in_repr.nreps(), cout, cin)
        fd = f.reshape(-1, cin, f.shape[-1]).permute(2, 0, 1).contiguous()   # (dim, rows, cin)
        rows = fd.shape[1]
        parts, j = [], 0
        for k, (a, b) in enumerate(self._slices):
            y = rows_linear(fd[a:b].reshape(-1, cin), w[k]).view(b - a, rows, cout)
            if self.bias is not None and a in self.scalar_locs:
                # bias column j belongs to the j-th scalar irrep (out[..., scalar_locs] + bias)
                y = self.activation(BiasRowsFn.apply(y, self.bias[:, j])).to(y.dtype)
                j += 1
            parts.append(y)
        out = torch.cat(parts, dim=0) if len(parts) > 1 else parts[0]     # (dim, rows, cout)
        return out.permute(1, 2, 0).reshape(*lead, cout, out.shape[0])
