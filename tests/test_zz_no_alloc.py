"""The allocation-free message-passing forward (``feq_edgewise_fwd_src_noalloc``).

It must give exactly what ``feq_edgewise_fwd_src`` gives with a caller
workspace (same kernels; only the scratch of the split channel patterns
lives in a static device array), on two calls in a row, the second with fewer
edges, and it must not grow PyTorch's allocation.
"""
import ctypes

import pytest
import torch

import flash_eq as fe
from flash_eq import _native as N
from flash_eq.ops import edgewise_linear_src

pytestmark = pytest.mark.gpu


def _noalloc(layer, x, src, P, dist, y):
    rw = layer.radial_weights
    C = rw.channel_patterns.detach().contiguous()
    F = rw.radial_functions().detach().contiguous()
    lib = N.lib()
    rc = lib.feq_edgewise_fwd_src_noalloc(ctypes.byref(layer.layout()), ctypes.byref(layer.binning()),
                                          rw.rank, src.shape[0], N.ptr(x), x.shape[0], N.ptr(src),
                                          N.ptr(P), N.ptr(P), N.ptr(dist), N.ptr(C), N.ptr(F),
                                          N.ptr(y), N.stream_ptr(x.device))
    N.check(rc, "feq_edgewise_fwd_src_noalloc")


def test_noalloc_forward_equals_workspace_forward(dev):
    torch.manual_seed(0)
    rp = fe.Repr([0, 1, 2], 64)
    layer = fe.EquivariantEdgewiseLinear(rp, rp).to(dev)
    g = torch.Generator().manual_seed(1)
    Nn = 700
    x = torch.randn(Nn, 64, 9, generator=g).to(dev)
    basis = fe.WignerDBasis([rp]).to(dev)
    for E in (6000, 1700):                       # the second call is smaller
        src = torch.randint(0, Nn, (E,), generator=g).to(dev)
        dst = torch.randint(0, Nn, (E,), generator=g).to(dev)
        (P,) = basis(torch.randn(E, 3, generator=g).to(dev))
        dist = (torch.rand(E, generator=g) * 9.5).to(dev)
        graph = fe.Graph(src, dst, Nn)
        with torch.no_grad():
            perm, offsets = graph.csr_src()
            rw = layer.radial_weights
            ref = edgewise_linear_src(x, src, perm, offsets, P, P, dist, rw.channel_patterns,
                                      rw.radial_functions(), layer.layout(), layer.binning(), rw.rank)
            y = torch.full_like(ref, float("nan"))
            torch.cuda.synchronize()
            before = torch.cuda.memory_allocated(dev)
            _noalloc(layer, x, src, P, dist, y)
            torch.cuda.synchronize()
            assert torch.cuda.memory_allocated(dev) == before
        print(f"E={E}: max |noalloc - workspace| = {(y - ref).abs().max().item():.3e}")
        assert torch.equal(y, ref)


def test_noalloc_rejects_layouts_beyond_the_scratch(dev):
    """A layout without message-passing kernels is refused with its reason.
    (Every layout that has them fits the scratch array: the size check is
    covered host-side by test_native_abi.py.)"""
    rp = fe.Repr([0, 1], 8)
    layer = fe.EquivariantEdgewiseLinear(rp, rp).to(dev)
    x = torch.zeros(4, 8, 4, device=dev)
    src = torch.zeros(3, dtype=torch.int64, device=dev)
    P = torch.eye(4, device=dev).expand(3, 4, 4).contiguous()
    y = torch.empty(3, 8, 4, device=dev)
    with pytest.raises(RuntimeError, match="no message-passing kernels"):
        _noalloc(layer, x, src, P, torch.ones(3, device=dev), y)
