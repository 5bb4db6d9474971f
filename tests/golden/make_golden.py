"""Writes ``tests/golden/reference_vectors.npz`` from the reference's own pure-torch modules.

Run once, in the build container, where the reference checkout is mounted:

    python tests/golden/make_golden.py /root/reference

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
    ns = types.SimpleNamespace()
    ns.rep = importlib.import_module("feq_ref.representations")
    ns.graph = importlib.import_module("feq_ref.graph")
    ns.radial = importlib.import_module("feq_ref.layers.radial")
    ns.linear = importlib.import_module("feq_ref.layers.linear")
    ns.norm = importlib.import_module("feq_ref.layers.norm")
    ns.gating = importlib.import_module("feq_ref.layers.gating")
    ns.pooling = importlib.import_module("feq_ref.layers.pooling")
    ns.attention = importlib.import_module("feq_ref.layers.attention")
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
        out[f"{prefix}__sd__{k}"] = v.detach().cpu().numpy()


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


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
