"""Host-side behaviour of the drop-in API (no GPU needed)."""
import math

import pytest
import torch

import flash_eq as fe
from flash_eq.representations.wigner import _wigner_plan
from oracle import wigner as OW


def test_generators_match_oracle_bitwise():
    for l in range(0, 8):
        assert torch.equal(fe.Irrep(l)._generators(), torch.from_numpy(OW.irrep_generators(l)))


def test_wignerd_rot_matches_oracle():
    g = torch.Generator().manual_seed(0)
    axis, angle = OW.random_rotation((16,), generator=g)
    w = fe.WignerD(fe.Repr([0, 1, 2]))
    assert (w.rot(axis, angle, cartesian=True).double() - OW.rot([0, 1, 2], axis, angle, True)).abs().max() < 2e-6


def test_closed_form_plan_reproduces_matrix_exp():
    """The kernel's constants (V, z, partner) rebuild D = exp(theta rho (cos phi G0 + sin phi G1))."""
    from flash_eq.representations.wigner import _z_matrix
    for l in (1, 2, 4, 6):
        plan = _wigner_plan(fe.Repr([l]))
        n = 2 * l + 1
        V = plan[:n * n].view(n, n)
        z, p = plan[n * n:n * n + n], plan[n * n + n:]
        g = torch.from_numpy(OW.irrep_generators(l)).double()
        for phi, ang in ((0.7, 2.2), (-1.3, 0.5)):
            ref = torch.linalg.matrix_exp(ang * (math.cos(phi) * g[0] + math.sin(phi) * g[1]))
            fac = _z_matrix(z, p, phi) @ V @ _z_matrix(z, p, ang) @ V.T @ _z_matrix(z, p, -phi)
            assert (ref - fac).abs().max() < 1e-6


def test_seeded_construction_is_deterministic_and_named_like_reference():
    torch.manual_seed(0)
    a = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1, 2], 8), fe.Repr([0, 1, 2], 8))
    torch.manual_seed(0)
    b = fe.EquivariantEdgewiseLinear(fe.Repr([0, 1, 2], 8), fe.Repr([0, 1, 2], 8))
    for (ka, va), (kb, vb) in zip(a.state_dict().items(), b.state_dict().items()):
        assert ka == kb and torch.equal(va, vb)
    assert set(a.state_dict()) == {
        "radial_weights.channel_patterns", "radial_weights.frequencies",
        "radial_weights.trunk.0.weight", "radial_weights.trunk.0.bias",
        "radial_weights.trunk.2.weight", "radial_weights.trunk.2.bias",
        "radial_weights.head.weight", "radial_weights.head.bias", "radial_weights.bin_edges"}


def test_transformer_state_dict_structure():
    m = fe.EquivariantTransformer(fe.Repr([0, 1], 8), fe.Repr([0, 1, 2], 8), fe.Repr([0], 8),
                                  num_layers=2, num_heads=2)
    keys = list(m.state_dict())
    assert "basis._perm_1" in keys and "basis._wigner_modules.1.generators" in keys
    assert "layers.0.attn.linear_v.radial_weights.channel_patterns" in keys
    assert "layers.1.layer_scale_mlp.gamma" in keys and "final_norm.scalar_norm.weight" in keys


def test_constructor_errors_match_reference():
    r = fe.Repr([0, 1, 2], 6)
    with pytest.raises(ValueError, match="must divide"):
        fe.EquivariantAttention(r, r, num_heads=4)
    with pytest.raises(ValueError, match="min_val must be > 0"):
        fe.EquivariantEdgewiseLinear(r, r, log_bins=True, min_dist=0.0)
    with pytest.raises(ValueError, match="cannot modify the degrees"):
        fe.EquivariantLinear(fe.Repr([0, 1]), fe.Repr([0, 1, 2]))
    with pytest.raises(ValueError, match="reduce must be one of"):
        fe.GraphPooling(reduce="median")
    with pytest.raises(ValueError, match="src must be 1D"):
        fe.Graph(torch.zeros(2, 2), torch.zeros(2), 3)


def test_hot_path_refuses_cpu_tensors():
    r = fe.Repr([0, 1], 4)
    layer = fe.EquivariantEdgewiseLinear(r, r)
    E = 5
    P = torch.eye(4).expand(E, 4, 4)
    with pytest.raises(fe.CUDANotAvailableError):
        layer(P, P, torch.randn(E, 4, 4), torch.rand(E))
    with pytest.raises(fe.CUDANotAvailableError):
        fe.WignerDBasis([r])(torch.randn(E, 3))
    g = fe.Graph(torch.zeros(E, dtype=torch.long), torch.zeros(E, dtype=torch.long), 2)
    with pytest.raises(fe.CUDANotAvailableError):
        fe.GraphPooling("sum")(torch.randn(E, 4, 4), g)


def test_block_diagonal_empty_returns_zeros_on_cpu():
    from flash_eq.cuda import block_diagonal_cuda
    pr = fe.ProductRepr(fe.Repr([0, 1], 2), fe.Repr([0, 1, 2], 3))
    out = block_diagonal_cuda(torch.zeros(0, 2, 4), torch.zeros(11, 3, 2, 10), torch.zeros(0), pr,
                              0.0, 1.0, 10)
    assert out.shape == (0, 3, 9)


def test_half_precision_active_inside_half_modules():
    """The edgewise layer asks for the single-product kernels when its input is
    16-bit or when it runs inside a half-precision module computed in float32."""
    from flash_eq.utils import epsilon_dtype, half_precision_active
    assert not half_precision_active()
    assert not half_precision_active(torch.zeros(1))
    assert half_precision_active(torch.zeros(1, dtype=torch.bfloat16))
    with epsilon_dtype(torch.bfloat16):
        assert half_precision_active(torch.zeros(1))
    with epsilon_dtype(torch.float32):
        assert not half_precision_active(torch.zeros(1))


def test_radial_basis_cache_inference_then_training():
    """A first call under torch.inference_mode() must not leave an inference
    tensor behind: the training call after it differentiates through the
    basis (the reference recomputes it every call and has no such failure)."""
    import pickle
    net = fe.layers.radial.SeparableRadialNet(num_bins=8, out_mult=4, in_mult=4, weight_dim=3)
    with torch.inference_mode():
        F0 = net.radial_functions()
    F1 = net.radial_functions()
    F1.sum().backward()
    assert torch.equal(F0, F1.detach())
    assert net.trunk[0].weight.grad is not None
    basis = net._edge_basis()
    assert net._edge_basis() is basis                    # kept once formed outside inference mode
    with torch.inference_mode():
        assert net._edge_basis() is basis                # a normal tensor serves inference calls too
    pickle.loads(pickle.dumps(net))                      # the cache is not part of the module's state
    # a float32 copy of the buffers (as a half-precision module run in float32
    # passes) is a different tensor: it misses instead of matching a stale key
    copies = {k: v.clone() for k, v in net.named_buffers()}
    copies["bin_edges"].mul_(0.5)
    b2 = torch.func.functional_call(net, {**dict(net.named_parameters()), **copies}, ())
    ref = torch.func.functional_call(net, {**dict(net.named_parameters()), **copies}, ())
    assert torch.equal(b2, ref)
    assert not torch.equal(b2, net())
