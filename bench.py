"""Benchmark of the equivariant edge hot path on one MI355X.

Workload (the metric's config): one
EquivariantEdgewiseLinear with in = out = Repr([0,1,2], mult=64), fp32;
N = 10,000 nodes uniform in a 40^3 cube, k = 16 nearest neighbours
(E = 160,000 edges, src = neighbour -> dst = centre), distances clipped to
max_dist = 10, num_bins = 100.  Node features (N, 64, 9) ~ N(0,1) are gathered
to edges by src.  One step = gather + layer forward + (out**2).sum() +
backward into the node features and every layer parameter.  P = Q come from
WignerDBasis outside the timed region.

Prints one JSON line (driver contract) with edges/s, the roofline of the
dominant kernel (timed live with HIP events on the launch stream) and the
CPU-oracle baseline timed on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "flash-eq_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np
import torch

PEAK_FP32_TFLOPS = 157.3      # MI355X dense fp32 (matrix) peak
PEAK_HBM_GBS = 8000.0


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


def edgewise_flops(cin, cout, din, dout, rank, mcount, backward=True):
    """Algorithmic MAC count per edge of the fused separable formulation (x2 = flop)."""
    gemm = rank * cout * cin * dout
    small = rank * cin * mcount
    fwd = cin * din * din + small + gemm + cout * dout * dout
    bwd = cout * dout * dout + gemm + small + gemm + small + small + cin * din * din + cin * din * din
    return 2 * fwd, 2 * bwd


def edgewise_bytes(cin, cout, din, dout):
    """Algorithmic HBM bytes per edge: x, P, Q, r in and y out (fwd); + gy in, gx out (bwd)."""
    fwd = 4 * (cin * din + din * din + dout * dout + 1 + cout * dout)
    bwd = 4 * (cout * dout + cin * din + din * din + dout * dout + 1 + cin * din)
    return fwd, bwd


def time_events(fn, reps: int) -> float:
    """Mean milliseconds of fn() measured with HIP events on the current stream."""
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def cpu_baseline(layer, feats, src, dst, coords, sample_edges: int, reps: int = 3):
    """Oracle (bin-grouped BLAS restatement, float32 on CPU) fwd+bwd on the first edges."""
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
    return sample_edges / float(np.median(times)), torch.get_num_threads()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-sample", type=int, default=40000, help="edges in the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--grad-dist", action="store_true", help="also differentiate w.r.t. distances")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path.", file=sys.stderr)
        return 2
    import flash_eq as fe

    dev = torch.device("cuda", 0)
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
    (P,) = fe.WignerDBasis([rep]).to(dev)(vec)
    feats = feats_cpu.to(dev).requires_grad_(True)
    if args.grad_dist:
        dist.requires_grad_(True)

    def step():
        y = layer(P, P, feats[src_d], dist)
        (y ** 2).sum().backward()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_ev = time_events(step, args.steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    # ---- dominant-kernel timing (forward and backward kernels in isolation) ----
    from flash_eq.ops import EdgewiseLinearFn
    rw = layer.radial_weights
    C, F = rw.channel_patterns.detach(), rw.radial_functions().detach()
    L, B = layer.layout(), layer.binning()
    xe = feats.detach()[src_d].contiguous()
    with torch.no_grad():
        y0 = EdgewiseLinearFn.apply(xe, P, P, dist.detach(), C, F, L, B, rw.rank)
    fwd_ms = time_events(lambda: EdgewiseLinearFn.apply(xe, P, P, dist.detach(), C, F, L, B, rw.rank), 10)
    xr = xe.clone().requires_grad_(True)
    out = EdgewiseLinearFn.apply(xr, P, P, dist.detach(), C, F, L, B, rw.rank)
    gy = torch.randn_like(out)
    bwd_ms = time_events(lambda: torch.autograd.grad(out, xr, gy, retain_graph=True), 5)
    mcount = 9 + 4 * (2 * 2 + 1 * 1)
    f_fwd, f_bwd = edgewise_flops(MULT, MULT, 9, 9, rw.rank, mcount)
    b_fwd, b_bwd = edgewise_bytes(MULT, MULT, 9, 9)
    dom = "bwd" if bwd_ms >= fwd_ms else "fwd"
    dom_ms = max(bwd_ms, fwd_ms)
    dom_flops = (f_bwd if dom == "bwd" else f_fwd) * E
    dom_bytes = (b_bwd if dom == "bwd" else b_fwd) * E
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12
    roofline = {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": None,
                "kernel": f"edgewise_{dom}", "kernel_ms": round(dom_ms, 4),
                "algorithmic_flop_per_edge": (f_bwd if dom == "bwd" else f_fwd),
                "algorithmic_bytes_per_edge": (b_bwd if dom == "bwd" else b_fwd),
                "hbm_frac_at_algorithmic_bytes": round(dom_bytes / (dom_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4)}

    cpu = None
    if not args.no_cpu:
        v, cores = cpu_baseline(layer.cpu(), feats_cpu, src, dst, coords, args.cpu_sample)
        layer.to(dev)
        cpu = {"value": round(v, 1), "unit": "edges/s", "cores": cores, "kind": "port",
               "sample": f"first {args.cpu_sample} of the {E} edges, fwd+bwd of the float32 "
                         "oracle (bin-grouped BLAS), median of 3 after 1 warmup"}

    value = E * args.steps / wall
    line = {"metric": "edges/s fwd+bwd, edgewise linear L=2 mult=64; % of HBM/MFMA roofline",
            "value": round(value, 1), "unit": "edges/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
            "ms_per_step_events": round(ms_ev, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "f32", "data": "synthetic",
            "config": {"workload": "c2: EquivariantEdgewiseLinear [0,1,2]x64 -> [0,1,2]x64, "
                                   "kNN k=16 on 10k uniform nodes in 40^3, E=160000, 100 bins",
                       "edges": E, "nodes": N, "grad_distances": bool(args.grad_dist),
                       "parallelism": "single-gpu"},
            "roofline": roofline, "cpu_baseline": cpu}
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
