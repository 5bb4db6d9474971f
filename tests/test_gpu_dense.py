"""GPU checks of the dense helpers (csrc/dense.hip) through the C ABI:
feq_transpose (bit-exact against PyTorch's permute for 2-, 4- and 8-byte
elements, narrow and wide shapes, partial tiles, batches), feq_column_sums
(float32 sums within 1e-6 of the float64 sums relative to the sum of absolute
values, float64 within 1e-13; the same bits on every call; zero rows; unaligned
inputs) and feq_dot_f64 (float64 accumulation: within 1e-12 of the float64 dot
of the same float32 values, where float32 accumulation would lose digits)."""
import pytest
import torch

from flash_eq import _native as NAT
from flash_eq import ops

pytestmark = pytest.mark.gpu

# (rows % 4 == 0 with cols <= 32, or the mirror, take the 16-byte form; partial last tiles)
SHAPES = [(1, 1), (7, 3), (1000, 9), (100003, 25), (9, 100003), (49, 4097), (129, 65), (64, 64),
          (3, 5000), (4096, 1), (1, 4096), (333, 777), (100004, 9), (9, 100004), (1000, 32),
          (32, 1000), (36, 5), (5, 36)]


@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
def test_transpose_is_exact(dev, rows, cols, dtype):
    g = torch.Generator(device=dev).manual_seed(rows * 31 + cols)
    x = torch.randn(rows, cols, device=dev, generator=g).to(dtype)
    y = ops.transpose_last2(x, rows, cols)
    assert torch.equal(y.view(cols, rows), x.t().contiguous())


@pytest.mark.parametrize("batch,rows,cols", [(64, 1563, 16), (5, 33, 70), (3, 9, 2000), (7, 1000, 9),
                                             (7, 9, 1004)])
def test_batched_transpose(dev, batch, rows, cols):
    x = torch.randn(batch, rows, cols, device=dev)
    y = ops.transpose_last2(x, rows, cols).view(batch, cols, rows)
    assert torch.equal(y, x.transpose(1, 2).contiguous())


def test_transpose_rejects_bad_shapes(dev):
    x = torch.randn(10, 3, device=dev)
    with pytest.raises(RuntimeError):
        ops.transpose_last2(x, 4, 3)
    with pytest.raises(RuntimeError):
        ops.transpose_last2(x.t(), 3, 10)


def _colsum_ref(x):
    return x.double().sum(0), x.double().abs().sum(0).max().clamp_min(1e-300)


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 3), (1_000_000, 64), (300_000, 7), (64, 16384),
                                       (20000, 129), (257, 1000), (2, 100003), (123457, 4)])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.float64, 1e-13)])
def test_column_sums(dev, rows, cols, dtype, tol):
    g = torch.Generator(device=dev).manual_seed(rows + cols)
    x = torch.randn(rows, cols, device=dev, generator=g, dtype=dtype) + 0.25
    a = ops.column_sums(x)
    ref, scale = _colsum_ref(x)
    assert a.dtype == dtype and a.shape == (cols,)
    assert ((a.double() - ref).abs().max() / scale).item() < tol
    assert torch.equal(a, ops.column_sums(x))


def test_column_sums_unaligned_and_empty(dev):
    base = torch.randn(50001 * 8 + 1, device=dev)
    x = base[1:].view(50001, 8)                  # 4-byte aligned only: scalar loads
    ref, scale = _colsum_ref(x)
    assert ((ops.column_sums(x).double() - ref).abs().max() / scale).item() < 1e-6
    z = ops.column_sums(torch.empty(0, 37, device=dev))
    assert z.shape == (37,) and z.abs().max().item() == 0


@pytest.mark.parametrize("n", [0, 1, 3, 1000, 4_000_001])
def test_dot_f64(dev, n):
    g = torch.Generator(device=dev).manual_seed(n)
    a = torch.randn(n, device=dev, generator=g)
    b = torch.randn(n, device=dev, generator=g)
    d = ops.dot_f64(a, b)
    assert d.dtype == torch.float32 and d.dim() == 0
    ref = torch.dot(a.double(), b.double())
    scale = torch.dot(a.double().abs(), b.double().abs()).clamp_min(1e-300)
    assert (abs(d.double() - ref) <= 1e-7 * abs(ref) + 1e-12 * scale).item()
    assert torch.equal(d, ops.dot_f64(a, b))


def test_dot_f64_unaligned(dev):
    a = torch.randn(100001, device=dev)[1:]
    b = torch.randn(100001, device=dev)[:-1]
    ref = torch.dot(a.double(), b.double())
    assert abs(ops.dot_f64(a, b).double() - ref).item() <= 1e-6 * abs(ref).item() + 1e-9


def test_library_launches_the_helpers(dev):
    """The launch log names the dense kernels: no PyTorch formulation ran."""
    NAT.profile_summary()
    NAT.profile_enable(True)
    try:
        ops.transpose_last2(torch.randn(100, 9, device=dev), 100, 9)
        ops.column_sums(torch.randn(1000, 16, device=dev))
        ops.dot_f64(torch.randn(100, device=dev), torch.randn(100, device=dev))
        names = NAT.profile_summary()
    finally:
        NAT.profile_enable(False)
    for k in ("k_transpose", "k_colsum", "k_dot_f64"):
        assert k in names, names


@pytest.mark.parametrize("n", [1, 5, 1001, 65539])
@pytest.mark.parametrize("k", [2, 3, 10, 16])
@pytest.mark.parametrize("offset", [0, 1])
def test_sum_tables_is_the_ordered_sum(dev, n, k, offset):
    """feq_sum_tables (through ops.FanOutFn's backward) gives the bits of
    adding the tables left to right in float32 (16-byte and 4-byte forms)."""
    g = torch.Generator(device=dev).manual_seed(n + k)
    base = torch.randn(k, n + offset, device=dev, generator=g)
    tabs = [base[j, offset:] for j in range(k)]        # offset 1: not 16-byte aligned
    x = torch.zeros(n, device=dev, requires_grad=True)
    views = ops.FanOutFn.apply(x, k)
    sum((v * t).sum() for v, t in zip(views, tabs)).backward()
    ref = tabs[0].clone()
    for t in tabs[1:]:
        ref += t
    assert torch.equal(x.grad, ref)


def test_fan_out_skips_unused_views(dev):
    """Views without a gradient add nothing; one gradient passes through."""
    x = torch.zeros(7, device=dev, requires_grad=True)
    a, b, c = ops.FanOutFn.apply(x, 3)
    (2.0 * b).sum().backward()
    assert torch.equal(x.grad, torch.full((7,), 2.0, device=dev))
