"""Host-side pieces of the node path that are plain PyTorch, checked on the CPU
in float64: the component-major EquivariantLinear (EqLinearFn, node- and
component-major inputs and outputs) against the oracle, and the column
sums, chunked weight gradients, bias and LayerScale functions against direct
formulas, with gradcheck where they carry gradients."""
import pytest
import torch

import flash_eq as fe
from flash_eq import ops
from oracle import layer as OL


@pytest.mark.parametrize("lvals,cin,cout", [([0, 1, 2], 6, 5), ([1, 0, 2], 3, 4), ([2, 1], 4, 2)])
@pytest.mark.parametrize("in_cm,out_cm", [(False, False), (False, True), (True, False), (True, True)])
def test_eq_linear_fn_matches_oracle(lvals, cin, cout, in_cm, out_cm):
    g = torch.Generator().manual_seed(cin * 10 + cout)
    lin = fe.EquivariantLinear(fe.Repr(lvals, cin), fe.Repr(lvals, cout), bias=True).double()
    if lin.bias is not None:
        with torch.no_grad():
            lin.bias.copy_(torch.randn(lin.bias.shape, generator=g, dtype=torch.float64))
    D = fe.Repr(lvals, cin).dim()
    x = torch.randn(7, cin, D, generator=g, dtype=torch.float64)
    xin = (x.permute(2, 0, 1).contiguous() if in_cm else x).requires_grad_(True)
    y = lin.forward_layout(xin, in_cm, out_cm)
    ynm = y.permute(1, 2, 0) if out_cm else y
    ref = OL.equivariant_linear(x, lin.weight, lvals)
    if lin.bias is not None:
        offs = fe.Repr(lvals, cin).cumdims().tolist()
        locs = [offs[k] for k, l in enumerate(lvals) if l == 0]
        ref = ref.clone()
        ref[..., locs] = ref[..., locs] + lin.bias
    assert (ynm - ref).abs().max() < 1e-12
    params = [xin, lin.weight] + ([lin.bias] if lin.bias is not None else [])
    assert torch.autograd.gradcheck(
        lambda *a: lin.forward_layout(a[0], in_cm, out_cm), params[:1], eps=1e-6, atol=1e-8)
    go = torch.randn(y.shape, generator=g, dtype=torch.float64)
    gs = torch.autograd.grad(y, params, go)
    gr = torch.autograd.grad(ref, params[1:], go.permute(1, 2, 0) if out_cm else go)
    for a, b in zip(gs[1:], gr):
        assert (a - b).abs().max() < 1e-10


def test_column_sums_and_weight_grad():
    g = torch.Generator().manual_seed(1)
    for rows in (0, 1, 5, 64 * 64 + 3, 10000):
        t = torch.randn(rows, 7, generator=g, dtype=torch.float64)
        assert torch.allclose(ops.column_sums(t), t.sum(0), atol=1e-10)
        gy = torch.randn(rows, 5, generator=g, dtype=torch.float64)
        assert torch.allclose(ops.rows_weight_grad(gy, t, torch.float64), gy.t() @ t, atol=1e-9)
    t32 = torch.randn(9000, 3, generator=g)
    gy32 = torch.randn(9000, 4, generator=g)
    ref = gy32.double().t() @ t32.double()
    assert (ops.rows_weight_grad(gy32, t32, torch.float32).double() - ref).abs().max() < 1e-3


def test_bias_and_scale_functions_gradcheck():
    g = torch.Generator().manual_seed(2)
    y = torch.randn(11, 4, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(4, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(ops.BiasRowsFn.apply, (y, b))
    x = torch.randn(3, 5, 2, generator=g, dtype=torch.float64, requires_grad=True)
    s = torch.tensor(0.3, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(ops.ScaleFn.apply, (x, s))
