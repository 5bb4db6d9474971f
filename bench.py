"""Benchmark of the equivariant edge hot path on one MI355X.

Workload (the metric's config): one
EquivariantEdgewiseLinear with in = out = Repr([0,1,2], mult=64), fp32;
N = 10,000 nodes uniform in a 40^3 cube, k = 16 nearest neighbours
(E = 160,000 edges, src = neighbour -> dst = centre), distances clipped to
max_dist = 10, num_bins = 100.  Node features (N, 64, 9) ~ N(0,1) are gathered
to edges by src inside the fused layer (layer(P, P, feats, r, graph=graph):
the kernels read row src[e] of the node table; the backward sums the per-edge
input gradient over the edges grouped by source).  One step = gather + layer
forward + the sum-of-squares loss sum(out**2) + backward into the node
features and every layer parameter.  P = Q come from
WignerDBasis outside the timed region (as in the reference's benchmark,
benchmarks/compare_all.py:168).

Prints one JSON line (driver contract).  ``roofline`` describes the dominant
library kernel: its launches are bracketed with HIP events on their own
stream during the timed steps (feq_profile_enable), and its achieved rate is
the algorithmic work per launch (per-edge figures below x E) over the mean
launch duration: HBM bytes for the split-fp16 kernels (HBM-bound), fp32 flops
for the fp32-MFMA kernels.  ``cpu_baseline`` times the float32 CPU oracle on
this host.
"""
from __future__ import annotations

import argparse
import copy
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "flash-eq_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np
import torch

PEAK_FP32_TFLOPS = 157.3      # MI355X dense fp32 matrix peak
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
PEAK_F16_TFLOPS = 2500.0      # MI355X dense fp16 matrix peak
METRIC = "edges/s fwd+bwd, edgewise linear L=2 mult=64; % of HBM/MFMA roofline"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "edgewise_c2_hbm_traffic.md")


def knn_graph(n: int, k: int, box: float, seed: int):
    """Uniform points in [0, box)^3 and their k nearest neighbours (ties by index)."""
    from scipy.spatial import cKDTree
    g = torch.Generator().manual_seed(seed)
    coords = torch.rand(n, 3, generator=g, dtype=torch.float32) * box
    tree = cKDTree(coords.double().numpy())
    _, idx = tree.query(coords.double().numpy(), k=k + 1)
    nbr = torch.from_numpy(idx[:, 1:].astype(np.int64))      # drop self
    dst = torch.arange(n).repeat_interleave(k)
    src = nbr.reshape(-1)
    return coords, src, dst


def algorithmic_per_edge(lin, lout, cin, cout, same_pq=True, nodes_per_edge=None):
    """Algorithmic flop and HBM bytes per edge of each fused kernel (fp32).

    The mix of one (co, ci) pair costs M real MACs, M = n0_in n0_out +
    2 sum_{m>=1} 2 n_in(m) n_out(m); a rotation of one channel costs
    S = sum (2l+1)^2 MACs (P and Q are block diagonal over irreps).

    Bytes follow one convention everywhere (the yardstick the 60%-of-HBM
    target for this layer is stated in): every tensor of the reference
    layer's interface once per edge, as the reference's EquivariantEdgewiseLinear
    reads and writes them (linear.py:144-160) -- x, P (= Q), r, y for the
    forward; gy, x, P, r, gx for the input-gradient kernel; gy, x, P, r for
    the channel-pattern-gradient kernel.  The message-passing form moves fewer
    bytes than that (it writes gx as node rows, N / E of them per edge); with
    nodes_per_edge set, the "_node_rows" entries count gx that way.  The
    distance-gradient mix is excluded (the benchmark does not differentiate the
    distances).
    """
    mmax = max(max(lin), max(lout))
    M = 0
    for m in range(mmax + 1):
        ni = sum(1 for l in lin if l >= m)
        no = sum(1 for l in lout if l >= m)
        M += ni * no if m == 0 else 4 * ni * no
    s_in = sum((2 * l + 1) ** 2 for l in lin)
    s_out = sum((2 * l + 1) ** 2 for l in lout)
    din = sum(2 * l + 1 for l in lin)
    dout = sum(2 * l + 1 for l in lout)
    mix = 2 * cout * cin * M
    rot = 2 * cin * s_in + 2 * cout * s_out
    X, Y = 4 * cin * din, 4 * cout * dout
    PQ = 4 * din * din + (0 if same_pq else 4 * dout * dout)
    out = {
        "k_ews_fwd": (mix + rot, X + PQ + 4 + Y),
        "k_ews_bwd_x": (mix + rot, Y + X + PQ + 4 + X),
        "k_ews_bwd_c": (mix, Y + X + PQ + 4),
        "_mix_macs_per_pair": M,
    }
    if nodes_per_edge is not None:
        out["_node_rows"] = {"k_ews_bwd_x": Y + X + PQ + 4 + X * nodes_per_edge}
    return out


def executed_mfma_flop_per_edge(lin, lout, cin, cout, rank=4):
    """fp16 matrix-core flops the split kernels execute per edge: three products
    (hi*hi, hi*lo, lo*hi) per fp32 product of each GEMM; the channel-pattern
    GEMM's reduction over 16 Din (slot, edge) pairs is padded to 32-steps."""
    din = sum(2 * l + 1 for l in lin)
    dout = sum(2 * l + 1 for l in lout)
    g_fwd = 3 * 2 * rank * cout * cin * din                 # G_k = C_k fs
    g_x = 3 * 2 * rank * cin * cout * dout                  # H_k = C_k^T gd
    kpad = -(-16 * din // 32) * 32 / 16                     # padded slots per edge
    g_c = 3 * 2 * rank * cout * cin * kpad                  # dC_k += U_k fs^T
    return {"k_ews_fwd": g_fwd, "k_ews_bwd_x": g_x, "k_ews_bwd_c": g_c}


def highl_mfma_flop_per_edge(C: int = 128, L: int = 6, rank: int = 4) -> dict:
    """bf16 matrix-core flops the high-degree kernels (csrc/edgewise_hl.hip)
    execute per edge, counted from their tile loops (one 16x16x32 MFMA =
    16 384 flop): the input rotation takes (C x D) x (D x D) per edge with D
    padded to 16-column blocks and 32-steps; the mixes (k_hl_mixr) per 16
    channels, with the D slots in NB = 4 blocks of 16 rows, stage 1 NB x rank x
    C/32 products, stage 2 NB x rank/2 and the output rotation ceil(D/16) x NB;
    the per-edge radial-function gradient (k_hl_dfer) per rank and 64
    channels NB x 4 x C/32 stage-1 and NB x 4 stage-2 products; the
    channel-pattern gradient (k_hl_dcc) per 16 output channels, rank and pair
    of blocks one stage-1 product per block and C/16 stage-2 products."""
    D = (L + 1) ** 2
    f32 = 16 * 16 * 32 * 2
    nb, ndb = 4, -(-D // 16)
    rot = (C // 16) * -(-D // 16) * -(-D // 32) * f32
    mixr = (C // 16) * (nb * rank * (C // 32) + nb * rank // 2 + ndb * nb) * f32
    dfe = rank * (C // 64) * (nb * 4 * (C // 32) + nb * 4) * f32
    dc = (C // 16) * (nb // 2) * rank * (2 + C // 16) * f32
    return {"k_hl_rot_in": rot, "k_hl_mix": mixr, "k_hl_mix_t": mixr, "k_hl_dfe": dfe, "k_hl_dc": dc}


# config 5's algorithmic work, 54.7 MFLOP per edge fwd + bwd (the products of
# the layer at [0..6]x128 without padding), bounds the step at 3.479 ms on the
# bf16 matrix cores
C5_BOUND_MS = 3.479


def read_traffic(path: str = TRAFFIC_FILE) -> dict:
    """HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE.

    Parsed from the committed summary: rows ``| kernel | fetch_bytes | write_bytes | ...``.
    """
    out = {}
    if not os.path.exists(path):
        return out
    for line in open(path):
        m = re.match(r"\|\s*(k_\w+)\s*\|\s*([0-9.e+]+)\s*\|\s*([0-9.e+]+)\s*\|", line)
        if m:
            out[m.group(1)] = float(m.group(2)) + float(m.group(3))
    return out


def cpu_baseline(layer, feats, src, dst, coords, sample_edges: int, reps: int):
    """Float32 CPU oracle (bin-grouped BLAS restatement) fwd+bwd on the first edges."""
    from oracle import layer as OL
    from oracle import wigner as OW
    torch.set_num_threads(min(os.cpu_count() or 1, 16))
    e = slice(0, sample_edges)
    vec = (coords[src[e]] - coords[dst[e]])
    r = vec.norm(dim=-1).clamp(max=10.0)
    P = OW.basis([0, 1, 2], vec).float()
    params, cfg = OL.module_cfg(layer)
    params = {k: v.detach().float().requires_grad_(True) for k, v in params.items()}
    cfg["bin_edges"] = cfg["bin_edges"].float()
    x = feats[src[e]].clone().requires_grad_(True)
    times = []
    for it in range(reps + 1):
        t0 = time.perf_counter()
        y = OL.edgewise_linear(x, P, P, r, params, cfg)
        (y ** 2).sum().backward()
        dt = time.perf_counter() - t0
        if it:
            times.append(dt)
    return sample_edges / float(np.median(times)), torch.get_num_threads(), times


def copy_calibration(dev, nbytes: int = 1 << 30, reps: int = 3) -> None:
    """Plain device-to-device copies of a known size (reference for the --pmc byte counters)."""
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=dev).fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"copy calibration: {reps} copies of {nbytes} bytes", file=sys.stderr)


def radius_graph(n: int, box: float, radius: float, kmax: int, seed: int):
    """Uniform points in [0, box)^3; each node's neighbours within ``radius``, the
    ``kmax`` nearest kept (ties by index), src = neighbour -> dst = centre."""
    from scipy.spatial import cKDTree
    g = torch.Generator().manual_seed(seed)
    coords = torch.rand(n, 3, generator=g, dtype=torch.float32) * box
    tree = cKDTree(coords.double().numpy())
    d, idx = tree.query(coords.double().numpy(), k=kmax + 1, distance_upper_bound=radius)
    idx, d = idx[:, 1:], d[:, 1:]
    keep = np.isfinite(d)
    dst = np.repeat(np.arange(n), kmax).reshape(n, kmax)[keep]
    src = idx[keep]
    return coords, torch.from_numpy(src.astype(np.int64)), torch.from_numpy(dst.astype(np.int64))


def timed_steps(step, steps: int, warmup: int):
    """Runs warmup + timed steps; returns (wall ms/step, event ms/step, library kernel summary)."""
    from flash_eq import _native as NAT
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    NAT.profile_summary()
    NAT.profile_enable(True)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        step()
    stop.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    NAT.profile_enable(False)
    return wall * 1e3 / steps, start.elapsed_time(stop) / steps, NAT.profile_summary()


def cpu_info() -> dict:
    """The host's logical CPU count and model (the CPU baselines' hardware)."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"os_cpu_count": os.cpu_count(), "torch_threads": torch.get_num_threads(), "model": model}


def _median_time(fn, reps: int):
    times = []
    for it in range(reps + 1):
        t0 = time.perf_counter()
        fn()
        dt = time.perf_counter() - t0
        if it:
            times.append(dt)
    return float(np.median(times)), times


def _rotation(dev, seed: int):
    import flash_eq as fe
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(4, generator=g, dtype=torch.float64)
    q = q / q.norm()
    angle = 2 * torch.acos(q[0].abs().clamp(max=1.0))
    axis = (q[1:] * torch.sign(q[0] if q[0] != 0 else torch.tensor(1.0)))
    axis = axis / axis.norm()
    return axis.float().to(dev), angle.float().to(dev)


def equivariance_error(out1: torch.Tensor, out2: torch.Tensor) -> float:
    """max|a-b| / (max|a| + 1e-8): the reference's metric (tests/helpers.py:54-69)."""
    return float(((out1 - out2).abs().max() / (out1.abs().max() + 1e-8)).item())


def build_workload(name: str):
    """Full-size secondary configurations (3, 4, 5).

    Returns a dict: step (one fwd + loss + bwd), E, N, config text, the
    algorithmic table of the fused kernels, a bounded CPU-oracle timing
    (edges/s on a stated sample; None to skip) and an equivariance check."""
    import flash_eq as fe
    from flash_eq.ops import SumSquaresFn
    dev = torch.device("cuda", 0)
    wl = {"name": name}
    if name.startswith("c3"):
        dtype = torch.bfloat16 if name == "c3bf16" else torch.float32
        coords, src, dst = radius_graph(20000, 60.0, 10.0, 32, seed=1003)
        E, N = src.numel(), 20000
        g = torch.Generator().manual_seed(2003)
        feats_cpu = torch.randn(N, 64, 9, generator=g)
        feats = feats_cpu.to(dev, dtype).requires_grad_(True)
        torch.manual_seed(3)
        rep = fe.Repr([0, 1, 2], 64)
        block = fe.EquivariantTransformerBlock(rep, rep, num_heads=8, max_dist=10.0)
        block_cpu = {k: v.clone() for k, v in block.state_dict().items()}
        block = block.to(dev, dtype)
        basis = fe.WignerDBasis([rep]).to(dev)
        graph = fe.Graph(src.to(dev), dst.to(dev), N)
        xyz = coords.to(dev)

        def step():
            vec = xyz[graph.src] - xyz[graph.dst]
            dist = vec.norm(dim=-1)
            (P,) = basis(vec)
            Pd = P.to(dtype)
            out = block(Pd, Pd, feats, dist.to(dtype), graph)
            loss = SumSquaresFn.apply(out)
            loss.backward()
            return loss

        def equiv():
            axis, angle = _rotation(dev, 77)
            D = fe.WignerD(rep).to(dev).rot(axis, angle)
            R = fe.WignerD(fe.Repr([1])).to(dev).rot(axis, angle, cartesian=True)
            with torch.no_grad():
                vec = xyz[graph.src] - xyz[graph.dst]
                dist = vec.norm(dim=-1).to(dtype)
                (P1,) = basis(vec)
                (P2,) = basis(vec @ R.T)
                x = feats.detach()
                o1 = torch.einsum("ij,ncj->nci", D, block(P1.to(dtype), P1.to(dtype), x, dist, graph).float())
                x2 = torch.einsum("ij,ncj->nci", D, x.float()).to(dtype)
                o2 = block(P2.to(dtype), P2.to(dtype), x2, dist, graph).float()
            return equivariance_error(o1, o2)

        def cpu():
            # the oracle's block (float32) on its own graph: 500 nodes at config
            # 3's density (box scaled by (500/20000)^(1/3)), radius 10, k <= 32,
            # fed the values the GPU run sees (bf16-rounded for the bf16 variant)
            from oracle import model as OM
            from oracle import wigner as OW
            n = 500
            c, s, d = radius_graph(n, 60.0 * (n / 20000) ** (1.0 / 3.0), 10.0, 32, seed=1103)
            vec = c[s] - c[d]
            P = OW.basis([0, 1, 2], vec).to(dtype).float()
            r = vec.norm(dim=-1).to(dtype).float()
            params = {k: (v.to(dtype).float().requires_grad_(True) if v.is_floating_point()
                          and not k.endswith(("bin_edges", "frequencies")) else v.float()
                          if v.is_floating_point() else v) for k, v in block_cpu.items()}
            cfg = OM.block_cfg([0, 1, 2], [0, 1, 2], 64, 64, heads=8, num_bins=100, max_dist=10.0)
            x = feats_cpu[:n].to(dtype).float().clone().requires_grad_(True)

            def run():
                out = OM.block(params, cfg, P, P, x, r, s, d, n)
                (out ** 2).sum().backward()
            med, times = _median_time(run, 2)
            return {"value": round(s.numel() / med, 1),
                    "sample": f"its own graph of {n} nodes at config 3's density (radius 10, k <= 32, "
                              f"{s.numel()} edges): fwd + (out**2).sum() + bwd of the float32 oracle "
                              f"block (oracle/model.py) on the {str(dtype).replace('torch.', '')} "
                              f"values, median of 2 after 1 warmup ({sum(times):.1f} s)"}

        wl.update(step=step, E=E, N=N, equiv=equiv, cpu=cpu,
                  leaves=[feats] + list(block.parameters()),
                  work=algorithmic_per_edge([0, 1, 2], [0, 1, 2], 64, 64, nodes_per_edge=N / E),
                  config=(f"c3: EquivariantTransformerBlock 8 heads [0,1,2]x64, radius-10 graph "
                          f"capped at k=32 on 20k nodes in 60^3, E={E}, fwd+bwd incl. "
                          f"WignerDBasis, {str(dtype).replace('torch.', '')}"),
                  dtype="bf16" if dtype == torch.bfloat16 else "f32")
    elif name in ("c4", "c4pq"):
        # c4pq: the same step with the coordinates requiring grad (force
        # training): every edgewise layer then also forms grad_P and grad_Q
        g = torch.Generator().manual_seed(1004)
        N = 50000
        u = torch.randn(N, 3, generator=g, dtype=torch.float64)
        u = u / u.norm(dim=1, keepdim=True)
        coords = torch.cumsum(3.8 * u, 0).float()
        coords = coords - coords[0]
        from scipy.spatial import cKDTree
        _, idx = cKDTree(coords.double().numpy()).query(coords.double().numpy(), k=25)
        src = torch.from_numpy(idx[:, 1:].astype(np.int64)).reshape(-1)
        dst = torch.arange(N).repeat_interleave(24)
        E = src.numel()
        feats_cpu = torch.randn(N, 32, 4, generator=g)
        feats = feats_cpu.to(dev).requires_grad_(True)
        torch.manual_seed(4)
        # out Repr([0], mult=1) cannot be split into 8 heads (attention.py:233-234);
        # mult=8 is the nearest constructible output
        model = fe.EquivariantTransformer(fe.Repr([0, 1], 32), fe.Repr([0, 1, 2], 64),
                                          fe.Repr([0], 8), num_layers=6, num_heads=8, max_dist=10.0)
        model_cpu = {k: v.clone() for k, v in model.state_dict().items()}
        model = model.to(dev)
        graph = fe.Graph(src.to(dev), dst.to(dev), N)
        xyz = coords.to(dev).requires_grad_(name == "c4pq")

        def step():
            out = model(xyz, feats, graph)
            loss = SumSquaresFn.apply(out)
            loss.backward()
            return loss

        def cpu():
            # the oracle's 6-layer model (float32) on the first 600 nodes of the chain
            from oracle import model as OM
            n = 600
            c = coords[:n]
            _, ii = cKDTree(c.double().numpy()).query(c.double().numpy(), k=25)
            s = torch.from_numpy(ii[:, 1:].astype(np.int64)).reshape(-1)
            d = torch.arange(n).repeat_interleave(24)
            params = {k: (v.float().requires_grad_(True) if v.is_floating_point()
                          and not k.endswith(("bin_edges", "frequencies")) else v.float()
                          if v.is_floating_point() else v) for k, v in model_cpu.items()}
            cfg = OM.transformer_cfg([0, 1], [0, 1, 2], [0], 32, 64, 8, num_layers=6, heads=8,
                                     num_bins=100, max_dist=10.0)
            x = feats_cpu[:n].clone().requires_grad_(True)

            def run():
                out = OM.transformer(params, cfg, c, x, s, d, n)
                (out ** 2).sum().backward()
            med, times = _median_time(run, 1)
            return {"value": round(s.numel() / med, 1),
                    "sample": f"the first {n} nodes of the chain with their own k=24 graph "
                              f"({s.numel()} edges): fwd + (out**2).sum() + bwd of the float32 "
                              f"oracle transformer (oracle/model.py), median of 1 after 1 warmup "
                              f"({sum(times):.1f} s)"}

        def equiv():
            # the output is Repr([0], 8): invariant under a rotation of the
            # coordinates with the input features Wigner-rotated
            axis, angle = _rotation(dev, 79)
            D = fe.WignerD(fe.Repr([0, 1])).to(dev).rot(axis, angle)
            R = fe.WignerD(fe.Repr([1])).to(dev).rot(axis, angle, cartesian=True)
            with torch.no_grad():
                x = feats.detach()
                o1 = model(xyz, x, graph)
                o2 = model(xyz @ R.T, torch.einsum("ij,ncj->nci", D, x), graph)
            return equivariance_error(o1, o2)

        wl.update(step=step, E=E, N=N, equiv=equiv, cpu=cpu if name == "c4" else None,
                  leaves=[feats] + list(model.parameters()) + ([xyz] if name == "c4pq" else []),
                  work=algorithmic_per_edge([0, 1, 2], [0, 1, 2], 64, 64, nodes_per_edge=N / E),
                  config=(f"{name}: EquivariantTransformer 6 layers, in [0,1]x32, hidden [0,1,2]x64, "
                          f"out [0]x8 (x1 is not divisible into 8 heads), 8 heads, random-walk "
                          f"chain of 50k nodes, kNN k=24, E={E}, fwd+bwd incl. WignerDBasis, fp32"
                          + (", coordinates with grad (gradients through every basis)"
                             if name == "c4pq" else "")),
                  dtype="f32")
    elif name == "c1":
        g = torch.Generator().manual_seed(1001)
        N, E = 100, 500
        coords = torch.randn(N, 3, generator=g) * 3
        src = torch.randint(0, N, (E,), generator=g)
        dst = torch.randint(0, N, (E,), generator=g)
        while (src == dst).any():
            bad = src == dst
            dst[bad] = torch.randint(0, N, (int(bad.sum()),), generator=g)
        feats_cpu = torch.randn(N, 32, 4, generator=g)
        feats = feats_cpu.to(dev).requires_grad_(True)
        torch.manual_seed(1)
        rin, rout = fe.Repr([0, 1], 32), fe.Repr([0, 1, 2], 64)
        layer_cpu = fe.EquivariantEdgewiseLinear(rin, rout, num_bins=100, max_dist=10.0)
        layer = copy.deepcopy(layer_cpu).to(dev)
        graph = fe.Graph(src.to(dev), dst.to(dev), N)
        vec = coords.to(dev)[graph.src] - coords.to(dev)[graph.dst]
        dist = vec.norm(dim=-1)
        P, Q = fe.WignerDBasis([rin, rout]).to(dev)(vec)
        pool = fe.GraphPooling("sum")

        def step():
            y = layer(P, Q, feats, dist, graph=graph)
            loss = SumSquaresFn.apply(pool(y, graph))
            loss.backward()
            return loss

        def cpu():
            from oracle import graphops as OG
            from oracle import layer as OL
            from oracle import wigner as OW
            v = coords[src] - coords[dst]
            Pc, Qc = OW.basis([0, 1], v).float(), OW.basis([0, 1, 2], v).float()
            r = v.norm(dim=-1)
            params, cfg = OL.module_cfg(layer_cpu)
            params = {k: t.detach().float().requires_grad_(True) for k, t in params.items()}
            cfg["bin_edges"] = cfg["bin_edges"].float()
            x = feats_cpu.clone().requires_grad_(True)

            def run():
                y = OG.pool_sum(OL.edgewise_linear(x[src], Pc, Qc, r, params, cfg), dst, N)
                (y ** 2).sum().backward()
            med, times = _median_time(run, 5)
            return {"value": round(E / med, 1),
                    "sample": f"all {E} edges: gather + float32 oracle layer + sum pooling, fwd + "
                              f"bwd, median of 5 after 1 warmup ({sum(times):.2f} s)"}

        def equiv():
            axis, angle = _rotation(dev, 78)
            Din = fe.WignerD(rin).to(dev).rot(axis, angle)
            Dout = fe.WignerD(rout).to(dev).rot(axis, angle)
            R = fe.WignerD(fe.Repr([1])).to(dev).rot(axis, angle, cartesian=True)
            with torch.no_grad():
                x = feats.detach()
                o1 = torch.einsum("ij,ncj->nci", Dout, pool(layer(P, Q, x, dist, graph=graph), graph))
                P2, Q2 = fe.WignerDBasis([rin, rout]).to(dev)(vec @ R.T)
                o2 = pool(layer(P2, Q2, torch.einsum("ij,ncj->nci", Din, x), dist, graph=graph), graph)
            return equivariance_error(o1, o2)

        wl.update(step=step, E=E, N=N, equiv=equiv, cpu=cpu, leaves=[feats] + list(layer.parameters()),
                  work=algorithmic_per_edge([0, 1], [0, 1, 2], 32, 64),
                  config=("c1: EquivariantEdgewiseLinear [0,1]x32 -> [0,1,2]x64, N=100, E=500 "
                          "random edges (self-loops resampled), gather + layer + scatter-sum, fp32"),
                  dtype="f32")
    elif name == "c5":
        lv = list(range(7))
        coords, src, dst = knn_graph(5000, 32, 30.0, seed=1005)
        E, N = src.numel(), 5000
        g = torch.Generator().manual_seed(2005)
        x_cpu = torch.randn(E, 128, 49, generator=g).to(torch.bfloat16)
        x = x_cpu.to(dev).requires_grad_(True)
        torch.manual_seed(5)
        rep = fe.Repr(lv, 128)
        layer_cpu = fe.EquivariantEdgewiseLinear(rep, rep, num_bins=100, max_dist=10.0)
        layer = copy.deepcopy(layer_cpu).to(dev)
        xyz = coords.to(dev)
        vec = xyz[src.to(dev)] - xyz[dst.to(dev)]
        dist = vec.norm(dim=-1).clamp(max=10.0)
        (P,) = fe.WignerDBasis([rep]).to(dev)(vec)
        P = P.to(torch.bfloat16)

        def step():
            y = layer(P, P, x, dist.to(torch.bfloat16))
            loss = SumSquaresFn.apply(y)          # bf16 values, float32 sums
            loss.backward()
            return loss

        def cpu():
            # the oracle forms the (101, 128, 128, 231) radial table once per step
            # whatever the edge count: two sample sizes give the table's time a and
            # the per-edge time b (t = a + b n), and the full step a + b E
            from oracle import layer as OL
            params, cfg = OL.module_cfg(layer_cpu)
            params = {k: t.detach().float().requires_grad_(True) for k, t in params.items()}
            cfg["bin_edges"] = cfg["bin_edges"].float()
            meds, spent = {}, 0.0
            for n in (128, 640):
                Pc = P[:n].float().cpu()
                r = dist[:n].to(torch.bfloat16).float().cpu()
                xs = x_cpu[:n].float().requires_grad_(True)

                def run():
                    y = OL.edgewise_linear(xs, Pc, Pc, r, params, cfg)
                    (y ** 2).sum().backward()
                meds[n], times = _median_time(run, 1)
                spent += sum(times)
            b = (meds[640] - meds[128]) / (640 - 128)
            a = max(meds[128] - b * 128, 0.0)
            step_s = a + b * E
            return {"value": round(E / step_s, 1),
                    "sample": f"fwd + (y**2).sum() + bwd of the float32 oracle layer on the bf16 "
                              f"values at 128 and 640 edges (1 run after 1 warmup each, "
                              f"{spent:.1f} s): {a:.2f} s per step for the (101, 128, 128, 231) "
                              f"radial table and its gradient, {b * 1e3:.2f} ms per edge; edges/s "
                              f"of the full step E / (a + b E), E = {E}",
                    "table_s": round(a, 3), "per_edge_ms": round(b * 1e3, 3)}

        def equiv():
            axis, angle = _rotation(dev, 80)
            D = fe.WignerD(rep).to(dev).rot(axis, angle)
            R = fe.WignerD(fe.Repr([1])).to(dev).rot(axis, angle, cartesian=True)
            with torch.no_grad():
                xf = x.detach()
                db = dist.to(torch.bfloat16)
                o1 = torch.einsum("ij,ecj->eci", D, layer(P, P, xf, db).float())
                (P2,) = fe.WignerDBasis([rep]).to(dev)(vec @ R.T)
                P2 = P2.to(torch.bfloat16)
                x2 = torch.einsum("ij,ecj->eci", D, xf.float()).to(torch.bfloat16)
                o2 = layer(P2, P2, x2, db).float()
            return equivariance_error(o1, o2)

        wl.update(step=step, E=E, N=N, equiv=equiv, cpu=cpu, leaves=[x] + list(layer.parameters()),
                  work=algorithmic_per_edge(lv, lv, 128, 128),
                  mfma=highl_mfma_flop_per_edge(128, 6),
                  config=("c5: EquivariantEdgewiseLinear [0..6]x128 -> [0..6]x128, kNN k=32 on 5k "
                          f"nodes in 30^3, E={E}, bf16 edge features, fwd+bwd"),
                  dtype="bf16")
    else:
        raise SystemExit(f"unknown workload {name}")
    return wl


def run_workload(name: str, steps: int, warmup: int, with_cpu: bool) -> dict:
    """One secondary configuration at full size: eager steps timed (synchronised
    on both sides), a second pass with every library launch bracketed by events
    (per-kernel times, the dominant kernel's algorithmic HBM fraction), the
    CPU oracle on a bounded sample and, where defined, the equivariance error
    under one random rotation."""
    wl = build_workload(name)
    E = wl["E"]
    t0 = time.perf_counter()
    for _ in range(warmup):
        wl["step"]()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(steps):
        wl["step"]()
    torch.cuda.synchronize()
    ms_eager = (time.perf_counter() - t1) * 1e3 / steps
    # the same step recorded once in a HIP graph and replayed (no host work per
    # step); kept only when its loss equals an eager step's
    ms_graph, graph_note = None, None
    try:
        from flash_eq.capture import capture_step
        for t in wl["leaves"]:
            t.grad = None
        ref = float(wl["step"]())
        cg, loss = capture_step(wl["step"], wl["leaves"], warmup=1)
        cg.replay()
        torch.cuda.synchronize()
        if abs(float(loss) - ref) <= 1e-5 * max(abs(ref), 1.0):
            t2 = time.perf_counter()
            for _ in range(steps):
                cg.replay()
            torch.cuda.synchronize()
            ms_graph = (time.perf_counter() - t2) * 1e3 / steps
        else:
            graph_note = f"replayed loss {float(loss)} differs from the eager {ref}"
        del cg
    except Exception as exc:      # a step that cannot be captured reports the eager time
        graph_note = f"{type(exc).__name__}: {exc}"[:200]
    ms = ms_graph if ms_graph is not None else ms_eager
    from flash_eq import _native as NAT
    NAT.profile_summary()
    NAT.profile_enable(True)
    for _ in range(steps):
        wl["step"]()
    torch.cuda.synchronize()
    NAT.profile_enable(False)
    kern = NAT.profile_summary()
    per_kernel, dom = {}, None
    mfma = wl.get("mfma", {})
    for kname, (calls, tot) in sorted(kern.items(), key=lambda kv: -kv[1][1])[:5]:
        avg = tot / calls
        entry = {"launches": calls, "avg_ms": round(avg, 4), "ms_per_step": round(tot / steps, 4)}
        if kname in wl["work"]:
            fl, by = wl["work"][kname]
            entry["hbm_frac_algorithmic"] = round(by * E / (avg * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
        if kname in mfma:
            tf = mfma[kname] * E / (avg * 1e-3) / 1e12
            entry["bf16_mfma_tflops_executed"] = round(tf, 1)
            entry["bf16_mfma_frac"] = round(tf / PEAK_F16_TFLOPS, 4)
        per_kernel[kname] = entry
        dom = dom or kname
    out = {"workload": name, "config": wl["config"], "edges": E, "nodes": wl["N"],
           "dtype": wl["dtype"], "ms_per_step": round(ms, 4),
           "step_form": "hip_graph" if ms_graph is not None else "eager",
           "ms_per_step_eager": round(ms_eager, 4),
           "ms_per_step_graph": None if ms_graph is None else round(ms_graph, 4),
           "graph_note": graph_note,
           "value": round(E / (ms * 1e-3), 1), "unit": "edges/s", "steps": steps,
           "warmup": warmup, "dominant_kernel": dom,
           "dominant_kernel_hbm_frac": per_kernel.get(dom, {}).get("hbm_frac_algorithmic"),
           "per_kernel": per_kernel}
    if mfma:
        # the matrix-core kernels against the bf16 MFMA peak (executed flops) and
        # the whole step against its algorithmic bound (C5_BOUND_MS)
        frac = {}
        for kname, fl in mfma.items():
            if kname in kern:
                calls, tot = kern[kname]
                frac[kname] = round(fl * E / (tot / calls * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4)
        top = max(frac, key=lambda k: kern[k][1]) if frac else None
        out["roofline"] = {"bound": "mfma", "kernel": top,
                           "achieved": None if top is None else
                           round(mfma[top] * E / (kern[top][1] / kern[top][0] * 1e-3) / 1e12, 1),
                           "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                           "frac": None if top is None else frac[top],
                           "frac_per_kernel": frac,
                           "step_vs_algorithmic_bound": round(C5_BOUND_MS / ms, 4)}
    if wl.get("equiv") is not None:
        out["equivariance_err"] = wl["equiv"]()
    if with_cpu and wl.get("cpu") is not None:
        c = wl["cpu"]()
        c.update({"unit": "edges/s", "kind": "port", "cores": torch.get_num_threads()})
        out["cpu_baseline"] = c
    out["wall_s"] = round(time.perf_counter() - t0, 1)
    return out


# The reference's published EquivariantEdgewiseLinear numbers (H100,
# benchmarks/compare_all.py:146-182, README.md:281-305):
# (lmax, edges, ms per fwd + MSE + bwd + Adam step) at C = 32, num_bins = 64
PUBLISHED_FP32 = [(1, 32000, 5.3), (2, 32000, 11.5), (4, 5000, 7.1), (6, 5000, 14.7), (4, 20000, 21.5),
                  (6, 20000, 50.6), (4, 50000, 50.1), (6, 50000, 123.5), (4, 128000, 125.6),
                  (6, 128000, 309.7)]
PUBLISHED_AMP = [(1, 32000, 5.4), (2, 32000, 10.5), (4, 5000, 6.6), (6, 5000, 13.6), (4, 20000, 19.7),
                 (6, 20000, 46.2), (4, 50000, 45.3), (6, 50000, 110.9), (4, 128000, 112.9),
                 (6, 128000, 279.8)]


def run_published(amp: bool, n_warmup: int = 3, n_iter: int = 10, only=None) -> list:
    """The reference's own benchmark step (compare_all.py:146-182) at its
    published configurations: EquivariantEdgewiseLinear(Repr(0..L, 32)) with
    num_bins = 64, features (E, 32, dim) requiring grad, P = Q from WignerDBasis
    of random unit directions (outside the step), distances U[0, 10), one step =
    zero_grad + forward + MSE against a random target + backward + Adam (lr
    1e-4); fp16 autocast with a GradScaler for the AMP rows; mean over 10 steps
    after 3 warmups, timed with events as the reference does (compare_all.py:
    60-81)."""
    import flash_eq as fe
    dev = torch.device("cuda", 0)
    rows = []
    for lmax, E, ref_ms in (PUBLISHED_AMP if amp else PUBLISHED_FP32):
        if only and (lmax, E) not in only:
            continue
        torch.manual_seed(lmax * 1000 + E // 1000)
        rep = fe.Repr(list(range(lmax + 1)), 32)
        dim = rep.dim()
        layer = fe.EquivariantEdgewiseLinear(rep, rep, num_bins=64, min_dist=0.0, max_dist=10.0).to(dev)
        basis = fe.WignerDBasis([rep, rep]).to(dev)
        opt = torch.optim.Adam(layer.parameters(), lr=1e-4)
        scaler = torch.amp.GradScaler("cuda", enabled=amp)
        feats = torch.randn(E, 32, dim, device=dev, requires_grad=True)
        dirs = torch.randn(E, 3, device=dev)
        dirs = dirs / dirs.norm(dim=-1, keepdim=True)
        dist = torch.rand(E, device=dev) * 10.0
        target = torch.randn(E, 32, dim, device=dev)
        P, Q = basis(dirs)

        def step():
            opt.zero_grad()
            with torch.amp.autocast("cuda", enabled=amp):
                out = layer(P, Q, feats, dist)
                loss = ((out - target) ** 2).mean()
            scaler.scale(loss).backward()
            scaler.step(opt)
            scaler.update()
        try:
            for _ in range(n_warmup):
                step()
            torch.cuda.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(n_iter):
                step()
            t1.record()
            torch.cuda.synchronize()
            ms = t0.elapsed_time(t1) / n_iter
            rows.append({"lmax": lmax, "edges": E, "ms_per_step": round(ms, 3),
                         "reference_h100_ms": ref_ms, "speedup_vs_reference": round(ref_ms / ms, 2)})
        except Exception as exc:      # one failing row must not lose the others
            rows.append({"lmax": lmax, "edges": E, "error": f"{type(exc).__name__}: {exc}"[:200]})
        del layer, basis, opt, feats, target, P, Q
        torch.cuda.empty_cache()
    return rows


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-sample", type=int, default=160000, help="edges in the CPU baseline sample")
    ap.add_argument("--cpu-reps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true",
                    help="report the eager step (default: the step captured in one HIP graph and "
                         "replayed; the eager step is timed too and reported beside it)")
    ap.add_argument("--grad-dist", action="store_true", help="also differentiate w.r.t. distances")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run 1 GiB device copies first (for rocprofv3 --pmc byte calibration)")
    ap.add_argument("--rows", default="",
                    help="published workloads: only these L:E rows, comma-separated (e.g. 6:20000)")
    ap.add_argument("--workload", default="c2",
                    choices=["c2", "c1", "c3", "c3bf16", "c4", "c4pq", "c5", "published", "published_amp"],
                    help="c2 (default) is the metric's configuration; the others print a "
                         "secondary line with their full-size throughput and kernel times")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the other BASELINE configurations (by default each runs at full "
                         "size after the metric's step and is reported under 'secondary')")
    ap.add_argument("--secondary-steps", type=int, default=3)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path; run it with --gpus 1.", file=sys.stderr)
        return 2
    if args.workload.startswith("published"):
        only = {tuple(int(v) for v in r.split(":")) for r in args.rows.split(",")} if args.rows else None
        print(json.dumps({"workload": args.workload,
                          "rows": run_published(args.workload == "published_amp", only=only)}))
        return 0
    if args.workload != "c2":
        print(json.dumps(run_workload(args.workload, args.steps, args.warmup, not args.no_cpu)))
        return 0
    import flash_eq as fe
    from flash_eq import _native as NAT

    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        copy_calibration(dev)
    N, K_NN, BOX, MULT = 10000, 16, 40.0, 64
    coords, src, dst = knn_graph(N, K_NN, BOX, seed=1002)
    E = src.numel()
    g = torch.Generator().manual_seed(2002)
    feats_cpu = torch.randn(N, MULT, 9, generator=g)
    torch.manual_seed(2)
    rep = fe.Repr([0, 1, 2], MULT)
    layer = fe.EquivariantEdgewiseLinear(rep, rep, num_bins=100, max_dist=10.0).to(dev)
    src_d, dst_d = src.to(dev), dst.to(dev)
    vec = coords.to(dev)[src_d] - coords.to(dev)[dst_d]
    dist = vec.norm(dim=-1).clamp(max=10.0)
    basis = fe.WignerDBasis([rep]).to(dev)
    (P,) = basis(vec)
    feats = feats_cpu.to(dev).requires_grad_(True)
    if args.grad_dist:
        dist.requires_grad_(True)

    graph = fe.Graph(src_d, dst_d, N)
    graph.csr_src()                            # CSR by source, built once per graph

    from flash_eq.capture import capture_step
    from flash_eq.ops import SumSquaresFn
    leaves = [feats] + list(layer.parameters()) + ([dist] if args.grad_dist else [])

    def step():
        y = layer(P, P, feats, dist, graph=graph)
        loss = SumSquaresFn.apply(y)
        loss.backward()
        return loss

    def clear():
        for t in leaves:
            t.grad = None

    def timed(run, n):
        """(wall ms, event ms) per call of run over n calls, synchronised on both sides."""
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for _ in range(n):
            run()
        stop.record()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / n, start.elapsed_time(stop) / n

    for _ in range(args.warmup):
        clear()
        step()
    # eager step: clean timing, then a pass with every library launch bracketed
    # by events (per-kernel times and the roofline)
    ms_eager, ms_eager_ev = timed(step, args.steps)
    NAT.profile_summary()                      # drop anything recorded so far
    NAT.profile_enable(True)
    timed(step, args.steps)
    NAT.profile_enable(False)
    kern = NAT.profile_summary()
    ms_graph = ms_graph_ev = None
    if not args.eager:
        # the same step (fwd, loss, bwd into features and every parameter)
        # recorded once in a HIP graph and replayed: no host work per step
        cg, _ = capture_step(step, leaves, warmup=args.warmup)
        for _ in range(args.warmup):
            cg.replay()
        ms_graph, ms_graph_ev = timed(cg.replay, args.steps)
    ms_per_step, ms_events = (ms_eager, ms_eager_ev) if args.eager else (ms_graph, ms_graph_ev)

    # WignerDBasis (outside the step, as in the reference benchmark): mean of 10 calls
    wstart = torch.cuda.Event(enable_timing=True)
    wstop = torch.cuda.Event(enable_timing=True)
    wstart.record()
    for _ in range(10):
        basis(vec)
    wstop.record()
    torch.cuda.synchronize()
    wigner_ms = wstart.elapsed_time(wstop) / 10

    work = algorithmic_per_edge([0, 1, 2], [0, 1, 2], MULT, MULT, nodes_per_edge=N / E)
    mfma_exec = executed_mfma_flop_per_edge([0, 1, 2], [0, 1, 2], MULT, MULT)
    traffic = read_traffic()
    per_kernel = {}
    for name, (calls, tot) in kern.items():
        avg = tot / calls
        entry = {"launches": calls, "avg_ms": round(avg, 4), "ms_per_step": round(tot / args.steps, 4)}
        if name in work:
            fl, by = work[name]
            entry["fp32_tflops_algorithmic"] = round(fl * E / (avg * 1e-3) / 1e12, 2)
            entry["hbm_gbs_algorithmic"] = round(by * E / (avg * 1e-3) / 1e9, 1)
            entry["hbm_frac"] = round(by * E / (avg * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
        if name in mfma_exec:
            entry["f16_mfma_util"] = round(mfma_exec[name] * E / (avg * 1e-3) / 1e12 / PEAK_F16_TFLOPS, 4)
        per_kernel[name] = entry
    dom = max((n for n in kern if n in work), key=lambda n: kern[n][1])
    calls, tot = kern[dom]
    avg_ms = tot / calls
    fl, by = work[dom]
    if dom.startswith("k_ews_"):
        # split-fp16 kernels: ~34 fp32 flop per algorithmic byte against a ridge
        # of 2500 / 3 TFLOP/s / 8 TB/s = 104, so HBM bounds them
        achieved = by * E / (avg_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4)}
    else:
        achieved = fl * E / (avg_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4)}
    roofline.update({"traffic": (round(traffic[dom]) if dom in traffic else None),
                     "kernel": dom, "kernel_avg_ms": round(avg_ms, 4),
                     "algorithmic_flop_per_edge": fl, "algorithmic_bytes_per_edge": by,
                     "byte_convention": "the reference layer's tensors once per edge (x, gx, y, gy, "
                                        "P, r)",
                     "edges_per_launch": E,
                     "per_kernel": dict(sorted(per_kernel.items(),
                                               key=lambda kv: -kv[1]["ms_per_step"])[:8])})
    if dom in work["_node_rows"]:
        # the same launch against the bytes the message-passing form must move
        # (gx as node rows)
        roofline["frac_gx_node_rows"] = round(work["_node_rows"][dom] * E / (avg_ms * 1e-3) / 1e9
                                              / PEAK_HBM_GBS, 4)

    cpu = None
    if not args.no_cpu:
        v, cores, times = cpu_baseline(layer.cpu(), feats_cpu, src, dst, coords, args.cpu_sample,
                                       args.cpu_reps)
        layer.to(dev)
        cpu = {"value": round(v, 1), "unit": "edges/s", "cores": cores, "kind": "port",
               "host": cpu_info(),
               "sample": f"first {args.cpu_sample} of the {E} edges: fwd + (y**2).sum() + bwd of the "
                         f"float32 CPU oracle (bin-grouped BLAS), median of {args.cpu_reps} after 1 "
                         f"warmup ({sum(times):.1f} s timed)"}

    # equivariance under one random rotation (inputs and directions rotated)
    axis, angle = _rotation(dev, 1234)
    D = fe.WignerD(rep).to(dev).rot(axis, angle)
    R = fe.WignerD(fe.Repr([1])).to(dev).rot(axis, angle, cartesian=True)
    with torch.no_grad():
        o1 = torch.einsum("ij,ecj->eci", D, layer(P, P, feats.detach(), dist.detach(), graph=graph))
        (P2,) = basis(vec @ R.T)
        o2 = layer(P2, P2, torch.einsum("ij,ncj->nci", D, feats.detach()), dist.detach(), graph=graph)
    equiv = equivariance_error(o1, o2)

    value = E / (ms_per_step * 1e-3)
    # each tensor once per pass: forward (x, P, r, y), backward (gy, x, P, r, gx) and the
    # radial table read and its gradient written once per step (12 573 B per edge;
    # gx counted per edge, as the reference's layer writes it, for a fixed yardstick)
    table_bytes = 4 * (layer.radial_weights.num_bins + 1) * MULT * MULT * layer.weight_dim
    work_ref = algorithmic_per_edge([0, 1, 2], [0, 1, 2], MULT, MULT)
    step_bytes = work_ref["k_ews_fwd"][1] + work_ref["k_ews_bwd_x"][1] + 2 * table_bytes / E
    step_flop = work["k_ews_fwd"][0] + work["k_ews_bwd_x"][0] + work["k_ews_bwd_c"][0]
    secondary = []
    if not args.no_secondary:
        for wname in ("c1", "c3", "c3bf16", "c4", "c5"):
            print(f"secondary {wname} ...", file=sys.stderr, flush=True)
            try:
                secondary.append(run_workload(wname, args.secondary_steps, 2, not args.no_cpu))
            except Exception as exc:     # one failing configuration must not lose the headline
                secondary.append({"workload": wname, "error": f"{type(exc).__name__}: {exc}"})
            torch.cuda.empty_cache()
    line = {"metric": METRIC,
            "value": round(value, 1), "unit": "edges/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
            "ms_per_step_events": round(ms_events, 4),
            "step_form": "eager" if args.eager else "hip_graph",
            "ms_per_step_eager": round(ms_eager, 4),
            "ms_per_step_graph": None if ms_graph is None else round(ms_graph, 4),
            "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "c2: EquivariantEdgewiseLinear [0,1,2]x64 -> [0,1,2]x64, "
                                   "kNN k=16 on 10k uniform nodes in 40^3, E=160000, 100 bins",
                       "edges": E, "nodes": N, "grad_distances": bool(args.grad_dist),
                       "parallelism": "single-gpu"},
            "roofline": roofline, "cpu_baseline": cpu,
            # the whole step against its algorithmic bytes and fp32 flops per edge
            "step_hbm_frac": round(step_bytes * E / (ms_per_step * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "step_algorithmic_bytes_per_edge": round(step_bytes, 1),
            "step_fp32_tflops_algorithmic": round(step_flop * E / (ms_per_step * 1e-3) / 1e12, 2),
            "equivariance_err": equiv,
            "wigner_basis_ms": round(wigner_ms, 4),
            "secondary": secondary}
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
