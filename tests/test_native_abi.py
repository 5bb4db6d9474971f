"""The C-ABI library loads on a GPU-less host and exports every symbol of include/flasheq.h.

No compute calls here: only host-side entry points (layout construction,
size queries, error reporting).
"""
import ctypes
import os
import re

import pytest

from flash_eq import _native as N
from oracle import layout as OL

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "flasheq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(feq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = N.load_library()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), f"{name} not exported"
    assert set(names) == set(N.EXPORTED_SYMBOLS), "ctypes signatures out of sync with the header"


def test_abi_version():
    assert N.load_library().feq_abi_version() == 1


CONFIGS = [([0, 1, 2], [0, 1, 2]), ([0, 1], [0, 1, 2]), ([1, 2, 2], [0, 1]), ([0, 1], [2]),
           ([2], [0, 1, 2]), (list(range(7)), list(range(7))), ([0, 0], [0, 0]), ([3, 1], [0])]


@pytest.mark.parametrize("lin,lout", CONFIGS)
def test_layout_matches_oracle(lin, lout):
    L = N.make_layout(lin, lout, 5, 7)
    assert (L.cin, L.cout, L.din, L.dout) == (5, 7, OL.dim_of(lin), OL.dim_of(lout))
    assert L.wdim == OL.weight_dim(lin, lout)
    blocks = [tuple(L.blk[k]) for k in range(L.nblocks)]
    assert blocks == OL.block_params(lin, lout)
    assert list(L.lslot_in[:L.din]) == OL.slot_l(lin)
    assert list(L.lslot_out[:L.dout]) == OL.slot_l(lout)
    assert L.has_lpos == int(max(lin) + max(lout) > 0)


def test_layout_errors():
    with pytest.raises(RuntimeError, match="exceeds supported limit"):
        N.make_layout([17], [0], 1, 1)
    with pytest.raises(RuntimeError, match="dimension exceeds"):
        N.make_layout([16, 16, 16, 16, 16], [0], 1, 1)


def test_size_queries_need_no_gpu():
    lib = N.load_library()
    L = N.make_layout([0, 1, 2], [0, 1, 2], 64, 64)
    b = N.make_binning(0.0, 10.0, 100, False, 0.1)
    assert lib.feq_edgewise_workspace(ctypes.byref(L), ctypes.byref(b), 4, 160000) > 0
    assert lib.feq_csr_workspace(1000, 100) > 0
    lv = (ctypes.c_int32 * 3)(0, 1, 2)
    assert lib.feq_wigner_plan_doubles(lv, 3) == (1 + 2) + (9 + 6) + (25 + 10)


def test_noalloc_scratch_covers_every_message_passing_layout():
    """The allocation-free forward keeps the forward workspace in a static
    array of FEQ_NOALLOC_SCRATCH_BYTES: every layout with message-passing
    kernels must fit it, and the workspace query must be the fp16 hi/lo
    fragments of the rank's channel patterns plus the rank scales (the size
    the entry point checks against the array before it touches it)."""
    lib = N.load_library()
    text = open(HEADER).read()
    cap = int(eval(re.search(r"#define FEQ_NOALLOC_SCRATCH_BYTES \(([^)]*)\)", text).group(1)))
    assert cap == 256 * 1024
    b = N.make_binning(0.0, 10.0, 100, False, 0.1)
    for lin, lout, cin, cout in [([0, 1, 2], [0, 1, 2], 64, 64), ([0, 1], [0, 1, 2], 64, 64),
                                 ([0, 1], [0, 1, 2], 32, 64)]:
        L = N.make_layout(lin, lout, cin, cout)
        need = lib.feq_edgewise_fwd_workspace(ctypes.byref(L), ctypes.byref(b), 4, 160000)
        frag = 4 * cout * cin * 2 * 2                  # rank x Cout x Cin, hi + lo halves
        assert need == -(-frag // 256) * 256 + 256 + 256, (lin, lout, cin, cout, need)
        assert need <= cap


def test_support_queries_and_basis_gradient_argument_errors():
    """Host-side behaviour of the fused layer's support queries and of the
    basis-gradient entry points' argument checks (no GPU work: the checks run
    before any launch; the pointers are never dereferenced)."""
    lib = N.load_library()
    b = N.make_binning(0.0, 10.0, 100, False, 0.1)

    def lay(lin, lout, cin, cout):
        return N.make_layout(lin, lout, cin, cout)

    # the split and scalar-output families form the bases' gradients; the
    # shape-generic layouts do not
    assert lib.feq_edgewise_pq_supported(ctypes.byref(lay([0, 1, 2], [0, 1, 2], 64, 64)), ctypes.byref(b), 4) == 1
    assert lib.feq_edgewise_pq_supported(ctypes.byref(lay([0, 1, 2], [0], 64, 8)), ctypes.byref(b), 4) == 1
    assert lib.feq_edgewise_pq_supported(ctypes.byref(lay([0, 1], [0, 1], 8, 8)), ctypes.byref(b), 4) == 0
    assert lib.feq_edgewise_pq_supported(ctypes.byref(lay([0, 1, 2], [0, 1, 2], 64, 64)), ctypes.byref(b), 3) == 0
    # LDS: lvals 0..6 fit the fused pair at 32 channels, not at 64
    L6 = list(range(7))
    assert lib.feq_edgewise_fused_supported(ctypes.byref(lay(L6, L6, 32, 32)), ctypes.byref(b), 4) == 1
    assert lib.feq_edgewise_fused_supported(ctypes.byref(lay(L6, L6, 64, 64)), ctypes.byref(b), 4) == 0
    assert lib.feq_edgewise_fused_supported(ctypes.byref(lay([0, 1, 2], [0, 1, 2], 64, 64)), ctypes.byref(b), 4) == 1

    L = lay([0, 1, 2], [0, 1, 2], 64, 64)
    fake = ctypes.c_void_p(256)          # never dereferenced: the checks fail first
    E = 10
    rc = lib.feq_edgewise_bwd_pq(ctypes.byref(L), ctypes.byref(b), 4, E, fake, fake, 0, None, None, None,
                                 fake, fake, fake, fake, fake, None, fake, fake, fake, None, None, fake, 0,
                                 fake, 1 << 30, None)
    assert rc != 0 and "grad_Q needs ym" in lib.feq_last_error().decode()
    rc = lib.feq_edgewise_fwd_ym(ctypes.byref(L), ctypes.byref(b), 4, E, fake, 0, None, fake, fake, fake,
                                 fake, fake, fake, None, 0, fake, 1 << 20, None)
    assert rc != 0 and "NULL pointer" in lib.feq_last_error().decode()
    rc = lib.feq_edgewise_fwd_ym(ctypes.byref(L), ctypes.byref(b), 4, E, fake, 0, None, fake, fake, fake,
                                 fake, fake, fake, fake, 2, fake, 1 << 20, None)
    assert rc != 0 and "unknown flags" in lib.feq_last_error().decode()
    S = lay([0, 1], [0, 1], 8, 8)        # shape-generic: no kernels forming grad_P / grad_Q
    rc = lib.feq_edgewise_bwd_pq(ctypes.byref(S), ctypes.byref(b), 4, E, fake, fake, 0, None, None, None,
                                 fake, fake, fake, fake, fake, fake, fake, fake, fake, None, fake, fake, 0,
                                 fake, 1 << 30, None)
    assert rc != 0 and "bases' gradients" in lib.feq_last_error().decode()


def test_eqlinear_queries_and_argument_errors():
    """The equivariant-linear entry points' size queries and argument checks
    (host side: every check runs before a launch, so no pointer here is
    dereferenced)."""
    lib = N.load_library()
    assert lib.feq_eqlinear_supported(64, 128) == 1
    assert lib.feq_eqlinear_supported(32, 64) == 1
    assert lib.feq_eqlinear_supported(128, 64) == 1
    assert lib.feq_eqlinear_supported(8, 16) == 0
    assert lib.feq_eqlinear_supported(64, 96) == 0
    assert lib.feq_eqlinear_workspace(3, 64, 128) >= 3 * 2 * 8 * 64 * 32
    assert lib.feq_eqlinear_workspace(0, 64, 128) == 0
    lv = (ctypes.c_int32 * 3)(0, 1, 2)
    rc = lib.feq_eqlinear_fwd(lv, 3, 10, 64, 128, None, None, None, 0, None, None, None, 0, None)
    assert rc != 0 and "NULL pointer" in lib.feq_last_error().decode()
    rc = lib.feq_eqlinear_fwd(lv, 3, 10, 64, 96, None, None, None, 0, None, None, None, 0, None)
    assert rc != 0 and "no kernel" in lib.feq_last_error().decode()
    bad = (ctypes.c_int32 * 3)(0, -1, 2)
    rc = lib.feq_eqlinear_bwd_x(bad, 3, 10, 64, 128, None, None, None, None, 0, None)
    assert rc != 0 and "invalid lvals" in lib.feq_last_error().decode()
    # no rows: nothing to do
    assert lib.feq_eqlinear_bwd_x(lv, 3, 0, 64, 128, None, None, None, None, 0, None) == 0
    # the weight gradient's workspace grows with the rows (per-workgroup partials)
    w0 = lib.feq_eqlinear_bwd_w_workspace(lv, 3, 0, 64, 128)
    w1 = lib.feq_eqlinear_bwd_w_workspace(lv, 3, 100000, 64, 128)
    assert 0 < w0 < w1
    rc = lib.feq_eqlinear_bwd_w(lv, 3, 10, 64, 128, None, None, 0, None, None, None, None, 0, None)
    assert rc != 0 and "NULL grad_w" in lib.feq_last_error().decode()
    rc = lib.feq_eqlinear_bwd_w(lv, 3, 10, 64, 128, None, None, 1, None, None, ctypes.c_void_p(256), None, 0,
                                None)
    assert rc != 0 and "bias columns" in lib.feq_last_error().decode()


def test_component_major_attention_argument_checks():
    """feq_attn_softmax_fwd_cm / _bwd_cm: invalid sizes and the edge form
    (no node indices) are refused before any launch."""
    lib = N.load_library()
    one = ctypes.c_void_p(256)          # never dereferenced: the checks fail first
    rc = lib.feq_attn_softmax_fwd_cm(one, one, 128, 0, 9, one, one, 10, None, 5, 8, 8, one, 0.0, one, one,
                                     10, one, None, None)
    assert rc != 0 and "invalid sizes" in lib.feq_last_error().decode()
    rc = lib.feq_attn_softmax_fwd_cm(one, one, 128, 1280, 9, None, None, 10, None, 5, 8, 8, one, 0.0, one, one,
                                     10, one, None, None)
    assert rc != 0 and "node tables" in lib.feq_last_error().decode()
    rc = lib.feq_attn_softmax_bwd_cm(one, one, 128, 1280, 0, one, one, 10, one, one, 5, 8, 8, one, one, one, 10,
                                     one, one, one, one, one, None)
    assert rc != 0 and "invalid sizes" in lib.feq_last_error().decode()


def test_sum_tables_argument_checks():
    """feq_sum_tables refuses 0 or more than 16 tables and NULL tables before any launch."""
    lib = N.load_library()
    ptrs = (ctypes.c_void_p * 2)(256, None)
    assert lib.feq_sum_tables(ptrs, 0, 10, ctypes.c_void_p(256), None) != 0
    assert lib.feq_sum_tables(ptrs, 17, 10, ctypes.c_void_p(256), None) != 0
    assert lib.feq_sum_tables(ptrs, 2, 10, ctypes.c_void_p(256), None) != 0
    assert "NULL table" in lib.feq_last_error().decode()
