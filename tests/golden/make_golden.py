"""Writes ``tests/golden/reference_vectors.npz`` from the reference's own pure-torch modules.

Run once, in the build container, where the reference checkout is mounted:

    python tests/golden/make_golden.py /root/reference [--composed-only]

It writes two files: ``reference_vectors.npz`` (below) and
``composed_vectors.npz`` (``composed()``: outputs and gradients of the
reference's edgewise linear, attention layer, transformer block and
transformer, run in float64 with the reference's block-diagonal CUDA op
replaced by the oracle's CPU op, which is pinned without the reference).

It covers what no closed form or reference test pins exactly:

* ``WignerDBasis`` / ``WignerD.rot`` values (flash_eq/representations/wigner.py:144-370):
  the frame twist and the (+m, -m) sign convention of P and Q;
* the seeded parameter initialisation (RNG consumption order) of
  ``EquivariantEdgewiseLinear`` + ``SeparableRadialNet`` (layers/linear.py:62-98,
  layers/radial.py:172-240) and ``EquivariantAttention`` (layers/attention.py:214-269),
  and the radial table ``SeparableRadialNet.forward`` (radial.py:259-275);
* forwards of the node-side modules the attention layer calls
  (EquivariantLinear, EquivariantLayerNorm, SeparableEquivariantLayerNorm,
  EquivariantGating, RepNorm), ``_neighbor_softmax`` (attention.py:108-141) and
  ``GraphPooling`` (pooling.py:21-106).

Only the reference's ``representations``, ``utils``, ``graph`` and the layer
modules above are loaded: their parent packages are registered as bare
namespaces so the reference's package ``__init__`` files, which import optional
dependencies that are not installed (sphericart), are not executed.  Nothing
here runs on the GPU box; the tests read only the ``.npz``.
"""
from __future__ import annotations

import importlib
import os
import sys
import types

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.npz")

WIGNER_LVALS = [(0, 1, 2), (0, 1), (0,), (1, 2, 2), (0, 1, 2, 3, 4, 5, 6), (2, 0, 1)]


def load_reference(root: str):
    pkg = os.path.join(root, "flash_eq")
    for name, sub in (("feq_ref", ""), ("feq_ref.layers", "layers"), ("feq_ref.cuda", "cuda")):
        mod = types.ModuleType(name)
        mod.__path__ = [os.path.join(pkg, sub) if sub else pkg]
        sys.modules[name] = mod
    # transformer.py imports the S2 activation (-> spherical -> sphericart, not
    # installed); the blocks built here use gating (use_s2_activation=False), so
    # the import only has to resolve: a placeholder module that refuses use
    s2 = types.ModuleType("feq_ref.layers.s2_activation")

    class _Unavailable:
        def __init__(self, *a, **k):
            raise RuntimeError("S2 activation is not available in the golden generator")

    s2.S2Activation = s2.SeparableS2Activation = _Unavailable
    sys.modules["feq_ref.layers.s2_activation"] = s2
    ns = types.SimpleNamespace()
    ns.rep = importlib.import_module("feq_ref.representations")
    ns.graph = importlib.import_module("feq_ref.graph")
    ns.radial = importlib.import_module("feq_ref.layers.radial")
    ns.linear = importlib.import_module("feq_ref.layers.linear")
    ns.norm = importlib.import_module("feq_ref.layers.norm")
    ns.gating = importlib.import_module("feq_ref.layers.gating")
    ns.pooling = importlib.import_module("feq_ref.layers.pooling")
    ns.attention = importlib.import_module("feq_ref.layers.attention")
    ns.transformer = importlib.import_module("feq_ref.layers.transformer")
    return ns


def key(lv) -> str:
    return "_".join(str(int(l)) for l in lv)


def directions() -> torch.Tensor:
    g = torch.Generator().manual_seed(7)
    rnd = torch.randn(24, 3, generator=g)
    special = torch.tensor([[0.0, 0.0, 0.0], [0.0, 0.0, 1.0], [0.0, 0.0, -1.0], [1.0, 0.0, 0.0],
                            [0.0, -2.0, 0.0], [1e-7, 0.0, 1.0], [1e-7, 1e-7, -1.0], [3.0, 4.0, 0.0]])
    return torch.cat([rnd, special]).float()


def state(prefix: str, module: torch.nn.Module, out: dict) -> None:
    for k, v in module.state_dict().items():
        out[f"{prefix}__sd__{k}"] = v.detach().cpu().numpy().copy()


def main(root: str) -> None:
    R = load_reference(root)
    Repr = R.rep.Repr
    out: dict[str, np.ndarray] = {}

    # ---- Wigner-D bases -------------------------------------------------------------
    d = directions()
    out["wigner__dirs"] = d.numpy()
    for lv in WIGNER_LVALS:
        (M,) = R.rep.WignerDBasis([Repr(list(lv), 1)])(d)
        out[f"wigner__{key(lv)}"] = M.detach().numpy()
    multi = [Repr([0, 1], 2), Repr([0, 1, 2], 3), Repr([0, 1], 5), Repr([0], 1)]
    for i, M in enumerate(R.rep.WignerDBasis(multi)(d)):
        out[f"wigner_multi__{i}"] = M.detach().numpy()
    g = torch.Generator().manual_seed(11)
    axis = torch.randn(8, 3, generator=g)
    axis = axis / axis.norm(dim=-1, keepdim=True)
    angle = torch.rand(8, generator=g) * 6.0 - 3.0
    out["rot__axis"], out["rot__angle"] = axis.numpy(), angle.numpy()
    w = R.rep.WignerD(Repr([0, 1, 2]))
    out["rot__cart"] = w.rot(axis, angle, cartesian=True).detach().numpy()
    out["rot__sph"] = w.rot(axis, angle, cartesian=False).detach().numpy()

    # ---- seeded construction + radial tables -----------------------------------------
    torch.manual_seed(0)
    a = R.linear.EquivariantEdgewiseLinear(Repr([0, 1], 4), Repr([0, 1, 2], 3), num_bins=10)
    state("ewlA", a, out)
    out["ewlA__table"] = a.radial_weights().detach().numpy()
    torch.manual_seed(1)
    b = R.linear.EquivariantEdgewiseLinear(Repr([0, 1, 2], 8), Repr([0, 1, 2], 8), num_bins=20,
                                           log_bins=True, min_dist=0.5, max_dist=8.0)
    state("ewlB", b, out)
    out["ewlB__table"] = b.radial_weights().detach().numpy()
    out["ewlB__binning"] = np.array(b.radial_weights.binning_params(), dtype=np.float64)
    torch.manual_seed(3)
    att = R.attention.EquivariantAttention(Repr([0, 1, 2], 8), Repr([0, 1, 2], 8), num_heads=2,
                                           num_bins=10)
    state("attn", att, out)

    # ---- node-side modules -----------------------------------------------------------
    rp = Repr([0, 1, 2], 6)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(7, 6, 9, generator=g)
    out["node__x"] = x.numpy()
    torch.manual_seed(4)
    lin = R.linear.EquivariantLinear(rp, Repr([0, 1, 2], 5))
    state("elin", lin, out)
    out["elin__y"] = lin(x).detach().numpy()
    torch.manual_seed(4)
    ln = R.norm.EquivariantLayerNorm(rp)
    state("eln", ln, out)
    out["eln__y"] = ln(x).detach().numpy()
    torch.manual_seed(4)
    sln = R.norm.SeparableEquivariantLayerNorm(rp)
    state("sln", sln, out)
    out["sln__y"] = sln(x).detach().numpy()
    torch.manual_seed(4)
    gate = R.gating.EquivariantGating(rp)
    state("gate", gate, out)
    out["gate__y"] = gate(x).detach().numpy()
    out["repnorm__y"] = R.norm.RepNorm(rp)(x).detach().numpy()

    # ---- neighbour softmax and pooling ---------------------------------------------
    g = torch.Generator().manual_seed(9)
    E, Nn, H = 40, 9, 3
    dst = torch.randint(0, Nn - 1, (E,), generator=g)          # node Nn-1 stays isolated
    src = torch.randint(0, Nn, (E,), generator=g)
    logits = torch.randn(E, H, generator=g) * 3.0
    ea = R.attention.EquivariantEdgeAttention(num_heads=H, qk_dim=4)
    out["softmax__dst"], out["softmax__logits"] = dst.numpy(), logits.numpy()
    out["softmax__y"] = ea._neighbor_softmax(logits, dst, Nn).detach().numpy()
    feats = torch.randn(E, 5, 4, generator=g)
    graph = R.graph.Graph(src, dst, Nn)
    out["pool__src"], out["pool__x"] = src.numpy(), feats.numpy()
    for red in ("sum", "mean", "max"):
        out[f"pool__{red}"] = R.pooling.GraphPooling(red)(feats, graph).detach().numpy()

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, {os.path.getsize(OUT)} bytes")


# ---- composed layers: outputs and gradients of the reference's own modules -------------------
COMPOSED_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "composed_vectors.npz")


def oracle_block_op(repo_root: str):
    """The reference signature of ``block_diagonal_cuda`` (cuda/block_diagonal.py:206-216)
    over the oracle's CPU block op (``oracle.layer.BlockDiag``), which is pinned
    independently of the reference (closed forms, brute force, the C restatement)."""
    if repo_root not in sys.path:
        sys.path.insert(0, repo_root)
    from oracle import blockdiag as BD
    from oracle.layer import BlockDiag

    def op(features, radial_table, distances, product_repr, bin_param1, bin_param2, num_bins,
           log_bins=False, sh_scale=0.1):
        lin = [int(l) for l in product_repr.rep1.lvals]
        lout = [int(l) for l in product_repr.rep2.lvals]
        b = BD.Binning(float(bin_param1), float(bin_param2), int(num_bins), bool(log_bins),
                       float(sh_scale))
        return BlockDiag.apply(features, radial_table, distances.to(features.dtype), lin, lout, b)

    return op


def _graph(E: int, N: int, seed: int, isolated: bool = True, no_self_loops: bool = True):
    g = torch.Generator().manual_seed(seed)
    hi = N - 1 if isolated else N                    # node N-1 receives no edge
    dst = torch.randint(0, hi, (E,), generator=g)
    src = torch.randint(0, N, (E,), generator=g)
    if no_self_loops:
        for e in range(E):
            while int(src[e]) == int(dst[e]):
                src[e] = torch.randint(0, N, (1,), generator=g)
    return src, dst


def _grads(prefix: str, module, y, inputs: dict, out: dict, seed: int) -> None:
    """Weights W (fixed, seeded) of the loss sum(y * W); the loss's gradient with
    respect to every named input and every parameter of the module."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(y.shape, generator=g, dtype=torch.float64)
    out[f"{prefix}__y"] = y.detach().numpy()
    out[f"{prefix}__lossw"] = w.numpy()
    (y * w).sum().backward()
    for k, t in inputs.items():
        out[f"{prefix}__in__{k}"] = t.detach().numpy()
        if t.requires_grad:
            out[f"{prefix}__grad__{k}"] = t.grad.detach().numpy()
    for k, p in module.named_parameters():
        out[f"{prefix}__pgrad__{k}"] = p.grad.detach().numpy()


def composed(root: str) -> None:
    """Reference outputs and gradients (float64 modules built from float32 seeded
    init) of EquivariantEdgewiseLinear, EquivariantAttention, EquivariantTransformerBlock
    and EquivariantTransformer on small graphs (E <= 64, mult <= 8)."""
    R = load_reference(root)
    R.linear.block_diagonal_cuda = oracle_block_op(os.path.dirname(os.path.dirname(
        os.path.dirname(os.path.abspath(__file__)))))
    Repr = R.rep.Repr
    out: dict[str, np.ndarray] = {}
    dd = torch.float64
    HID = 16                               # radial-MLP width of the modules below (small fixtures)

    def dirs(E, seed):
        g = torch.Generator().manual_seed(seed)
        return torch.randn(E, 3, generator=g, dtype=dd)

    # ---- EquivariantEdgewiseLinear: P != Q, linear bins with extrapolation; log bins
    for name, seed, rin, rout, kw in (
            ("ewl", 21, Repr([0, 1], 4), Repr([0, 1, 2], 3), dict(num_bins=10, hidden_dim=HID)),
            ("ewlL", 22, Repr([0, 1, 2], 3), Repr([0, 1, 2], 3),
             dict(num_bins=8, log_bins=True, min_dist=0.5, max_dist=8.0, hidden_dim=HID))):
        torch.manual_seed(seed)
        m = R.linear.EquivariantEdgewiseLinear(rin, rout, **kw)
        state(name, m, out)
        m = m.double()
        E = 24
        g = torch.Generator().manual_seed(seed + 100)
        v = dirs(E, seed + 200)
        P, Q = R.rep.WignerDBasis([rin, rout]).double()(v)
        P = P.detach().clone().requires_grad_(True)
        Q = Q.detach().clone().requires_grad_(True)
        x = torch.randn(E, rin.mult, rin.dim(), generator=g, dtype=dd).requires_grad_(True)
        r = (torch.rand(E, generator=g, dtype=dd) * 12.0 + 0.3).requires_grad_(True)
        y = m(P, Q, x, r)
        _grads(name, m, y, dict(x=x, P=P, Q=Q, r=r, dirs=v), out, seed + 300)

    # ---- EquivariantAttention with distance decay; with and without edge features
    for name, seed, with_ef in (("att", 31, False), ("attE", 32, True)):
        rp = Repr([0, 1, 2], 4)
        torch.manual_seed(seed)
        m = R.attention.EquivariantAttention(rp, rp, num_heads=2, num_bins=10, hidden_dim=HID,
                                             distance_decay_scale=3.0)
        state(name, m, out)
        m = m.double()
        E, Nn = 40, 9
        src, dst = _graph(E, Nn, seed + 100)
        graph = R.graph.Graph(src, dst, Nn)
        g = torch.Generator().manual_seed(seed + 200)
        v = torch.randn(E, 3, generator=g, dtype=dd)
        (P,) = R.rep.WignerDBasis([rp]).double()(v)
        x = torch.randn(Nn, 4, 9, generator=g, dtype=dd).requires_grad_(True)
        r = (torch.rand(E, generator=g, dtype=dd) * 9.0 + 0.2).requires_grad_(True)
        inputs = dict(x=x, r=r, src=src, dst=dst, dirs=v)
        ef = None
        if with_ef:
            ef = torch.randn(E, 4, 9, generator=g, dtype=dd).requires_grad_(True)
            inputs["ef"] = ef
        y = m(P, P, x, r, graph, edge_features=ef)
        _grads(name, m, y, inputs, out, seed + 300)

    # ---- EquivariantTransformerBlock: residual (equal reprs) and not
    for name, seed, rin, rout, decay in (("blk", 41, Repr([0, 1, 2], 4), Repr([0, 1, 2], 4), None),
                                         ("blkN", 42, Repr([0, 1], 4), Repr([0, 1, 2], 6), 2.5)):
        torch.manual_seed(seed)
        m = R.transformer.EquivariantTransformerBlock(rin, rout, num_heads=2, num_bins=10,
                                                      hidden_dim=HID, distance_decay_scale=decay)
        state(name, m, out)
        with torch.no_grad():              # sizeable residual branches for the comparison
            for mod in (m.layer_scale_attn, m.layer_scale_mlp):
                if hasattr(mod, "gamma"):
                    mod.gamma.fill_(0.6)
        m = m.double()
        E, Nn = 48, 11
        src, dst = _graph(E, Nn, seed + 100)
        graph = R.graph.Graph(src, dst, Nn)
        g = torch.Generator().manual_seed(seed + 200)
        v = torch.randn(E, 3, generator=g, dtype=dd)
        P, Q = R.rep.WignerDBasis([rin, rout]).double()(v)
        x = torch.randn(Nn, rin.mult, rin.dim(), generator=g, dtype=dd).requires_grad_(True)
        r = (torch.rand(E, generator=g, dtype=dd) * 9.0 + 0.2).requires_grad_(True)
        y = m(P, Q, x, r, graph)
        _grads(name, m, y, dict(x=x, r=r, src=src, dst=dst, dirs=v), out, seed + 300)

    # ---- EquivariantTransformer: coordinates -> bases -> 3 blocks -> final norm
    rin, rh, ro = Repr([0, 1], 4), Repr([0, 1, 2], 4), Repr([0], 4)
    torch.manual_seed(51)
    m = R.transformer.EquivariantTransformer(rin, rh, ro, num_layers=3, num_heads=2, num_bins=10)
    state("tf", m, out)                    # default init (hidden_dim 64): the seeded-init pin
    torch.manual_seed(51)
    m = R.transformer.EquivariantTransformer(rin, rh, ro, num_layers=3, num_heads=2, num_bins=10,
                                             hidden_dim=HID, layer_scale_init=0.6)
    state("tfS", m, out)
    m = m.double()
    E, Nn = 56, 12
    src, dst = _graph(E, Nn, 151, isolated=False)
    graph = R.graph.Graph(src, dst, Nn)
    g = torch.Generator().manual_seed(251)
    coords = (torch.randn(Nn, 3, generator=g, dtype=dd) * 3.0).requires_grad_(True)
    x = torch.randn(Nn, 4, 4, generator=g, dtype=dd).requires_grad_(True)
    y = m(coords, x, graph)
    _grads("tfS", m, y, dict(x=x, coords=coords, src=src, dst=dst), out, 351)

    np.savez_compressed(COMPOSED_OUT, **out)
    print(f"wrote {COMPOSED_OUT}: {len(out)} arrays, {os.path.getsize(COMPOSED_OUT)} bytes")


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    ref_root = args[0] if args else "/root/reference"
    if "--composed-only" not in sys.argv:
        main(ref_root)
    composed(ref_root)
