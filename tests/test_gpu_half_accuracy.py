"""The single-product mode of the message-passing split kernels
(FEQ_EW_HALF_ACCURACY, feq_edgewise_fwd_src_ex / feq_edgewise_bwd_src_nodes_ex),
used for modules that compute in bfloat16 or float16.

Each operand pair takes one fp16 product instead of the three of the hi/lo
split, so a product carries a relative error up to about 2^-10.  The full-
accuracy path is pinned to the float64 oracle at 1e-5 (test_gpu_edgewise.py,
test_gpu_message_passing.py); these tests hold the half-accuracy results to
the bfloat16 bar against it (2e-2; the differences measure ~3e-4 and are held
below 2e-3, so a lost operand or scale shows), check
that the single-product kernels really ran (the results differ from the full
ones), that flags 0 is the full path bit for bit, and that the bfloat16
transformer block selects the mode."""
import ctypes

import pytest
import torch

import flash_eq as fe
from flash_eq import _native as NAT
from flash_eq import ops
from helpers import rel_err

pytestmark = pytest.mark.gpu

HALF_BAR = 2e-2
SINGLE_PRODUCT_ERR = 2e-3   # ~2^-10 per product; measured ~3e-4 (max-norm, relative)


@pytest.fixture(autouse=True)
def split_kernels(monkeypatch):
    monkeypatch.delenv("FEQ_EW_PATH", raising=False)
    monkeypatch.delenv("FEQ_FORCE_GENERIC", raising=False)


def _setup(dev, cin, lin, E, N, seed):
    g = torch.Generator().manual_seed(seed)
    torch.manual_seed(seed)
    layer = fe.EquivariantEdgewiseLinear(fe.Repr(lin, cin), fe.Repr([0, 1, 2], 64), num_bins=40).to(dev)
    d = torch.randn(E, 3, generator=g).to(dev)
    P, Q = fe.WignerDBasis([fe.Repr(lin, 1), fe.Repr([0, 1, 2], 1)]).to(dev)(d)
    src = torch.randint(0, N - 1, (E,), generator=g).to(dev)
    graph = fe.Graph(src, torch.randint(0, N, (E,), generator=g).to(dev), N)
    x = torch.randn(N, cin, P.shape[-1], generator=g).to(dev)
    r = (torch.rand(E, generator=g) * 11).to(dev)
    gy = torch.randn(E, 64, 9, generator=g).to(dev)
    return layer, graph, P, Q, x, r, gy


def _run(layer, graph, P, Q, x, r, gy, half):
    rw = layer.radial_weights
    perm, offsets = graph.csr_src()
    xg = x.clone().requires_grad_(True)
    rg = r.clone().requires_grad_(True)
    C = rw.channel_patterns.detach().clone().requires_grad_(True)
    F = rw.radial_functions().detach().clone().requires_grad_(True)
    y = ops.edgewise_linear_src(xg, graph.src, perm, offsets, P, Q, rg, C, F, layer.layout(),
                                layer.binning(), rw.rank, half_accuracy=half)
    y.backward(gy)
    return [y.detach(), xg.grad, rg.grad, C.grad, F.grad]


@pytest.mark.parametrize("E", [1000, 1037, 16000])
def test_half_accuracy_within_the_bfloat16_bar(dev, E):
    args = _setup(dev, 64, [0, 1, 2], E, N=max(E // 16, 7), seed=E)
    full = _run(*args, half=False)
    half = _run(*args, half=True)
    for name, a, b in zip(("y", "grad_x", "grad_dist", "grad_C", "grad_F"), half, full):
        err = rel_err(a, b)
        print(f"E={E} {name}: half vs full {err:.2e}", flush=True)
        assert err < SINGLE_PRODUCT_ERR, (name, err)
    # the single-product kernels ran: their rounding differs from the split's
    assert not torch.equal(half[0], full[0]) and not torch.equal(half[3], full[3])


def test_half_accuracy_embedded_layout(dev):
    """[0,1]x32 -> [0,1,2]x64 runs zero-embedded in the [0,1,2]x64 kernels; the
    layer passes the mode on when its input is bfloat16."""
    layer, graph, P, Q, x, r, gy = _setup(dev, 32, [0, 1], 1037, N=70, seed=5)
    xb = x.to(torch.bfloat16)
    ref = layer(P, Q, xb.float(), r, graph=graph)
    out = layer(P, Q, xb, r, graph=graph)
    assert out.dtype == torch.bfloat16
    assert rel_err(out.float(), ref) < HALF_BAR


def _call_fwd_ex(layer, graph, P, Q, x, r, flags):
    rw = layer.radial_weights
    lib = NAT.lib()
    E = r.shape[0]
    L, B = layer.layout(), layer.binning()
    C, F = rw.channel_patterns.detach().contiguous(), rw.radial_functions().detach().contiguous()
    y = torch.empty(E, 64, 9, device=x.device)
    ws = NAT.workspace(lib.feq_edgewise_fwd_workspace(ctypes.byref(L), ctypes.byref(B), rw.rank, E), x.device)
    rc = lib.feq_edgewise_fwd_src_ex(ctypes.byref(L), ctypes.byref(B), rw.rank, E, NAT.ptr(x), x.shape[0],
                                     NAT.ptr(graph.src), NAT.ptr(P), NAT.ptr(Q), NAT.ptr(r), NAT.ptr(C),
                                     NAT.ptr(F), NAT.ptr(y), flags, NAT.ptr(ws), ws.numel(),
                                     NAT.stream_ptr(x.device))
    return rc, y


def test_flags_zero_is_the_full_path_and_unknown_flags_fail(dev):
    layer, graph, P, Q, x, r, gy = _setup(dev, 64, [0, 1, 2], 1000, N=70, seed=9)
    rc, y0 = _call_fwd_ex(layer, graph, P, Q, x, r, 0)
    assert rc == 0
    with torch.no_grad():
        ref = layer(P, Q, x, r, graph=graph)
    assert torch.equal(y0, ref)
    rc, _ = _call_fwd_ex(layer, graph, P, Q, x, r, 2)
    assert rc != 0
    NAT.lib().feq_last_error()


def test_bfloat16_block_selects_half_accuracy(dev, monkeypatch):
    """Inside a bfloat16 transformer block (computed in float32) the edgewise
    layer asks for the single-product kernels (its V projection takes the form
    fused with the attention pooling; half_accuracy is the last argument of
    both message-passing functions)."""
    seen = []
    for fn in (ops.EdgewiseLinearSrcFn, ops.EdgewiseAttnPoolFn):
        def spy(*a, _real=fn.apply):
            seen.append(a[-1])
            return _real(*a)

        monkeypatch.setattr(fn, "apply", spy)
    torch.manual_seed(0)
    rep = fe.Repr([0, 1, 2], 64)
    block = fe.EquivariantTransformerBlock(rep, rep, num_heads=8).to(dev)
    E, N = 800, 60
    g = torch.Generator().manual_seed(1)
    graph = fe.Graph(torch.randint(0, N, (E,), generator=g).to(dev),
                     torch.randint(0, N, (E,), generator=g).to(dev), N)
    d = torch.randn(E, 3, generator=g).to(dev)
    P = fe.WignerDBasis([fe.Repr([0, 1, 2], 1)]).to(dev)(d)[0]
    feats = torch.randn(N, 64, 9, generator=g).to(dev)
    r = d.norm(dim=-1)
    block(P, P, feats, r, graph)
    assert seen and seen[-1] is False
    seen.clear()
    block.to(torch.bfloat16)(P.to(torch.bfloat16), P.to(torch.bfloat16), feats.to(torch.bfloat16),
                             r.to(torch.bfloat16), graph)
    assert seen and seen[-1] is True
