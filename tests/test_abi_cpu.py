"""Host-side checks: tables, generated code, C-ABI exports, API validation (no GPU compute)."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

import ictc_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_product_tables_match_oracle():
    from ictc_o3.basis import tables
    for l1 in range(4):
        for l2 in range(4):
            for l3 in range(7):
                assert np.abs(tables.coupling_component(l1, l2, l3) - orc.cg_component(l1, l2, l3)).max() < 1e-13
    for l in range(4):
        mono, coef = tables.harmonic_polynomials(l)
        expect = orc.direction_projection(l) * orc.direction_scale(l) * orc.multinomials(l)[:, None]
        assert np.abs(coef - expect).max() < 1e-13


def test_product_path_table_offsets():
    from ictc_o3.basis import tables
    T = tables.PathTable(tables.natural_paths(2, 2, 2))
    assert T.out_components == 35
    _, offsets, counts = orc.path_tables(orc.natural_paths(2, 2, 2))
    assert T.slot == offsets and T.counts == counts


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "ictc_mi355x.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ictc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from ictc_o3 import _native
    path = _native.library_path()
    if not os.path.exists(path):
        pytest.skip("library not built")
    lib = ctypes.CDLL(path)
    declared = _declared_symbols()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.exported_symbols())
    assert _native.lib().ictc_version() == 100


def test_host_only_entry_points():
    from ictc_o3 import _native
    if not os.path.exists(_native.library_path()):
        pytest.skip("library not built")
    assert _native.tp_shape(2, 2, 2) == (11, 35)
    assert _native.tp_shape(2, 3, 3) == (17, 71)
    assert _native.tp_shape(0, 2, 2) == (3, 9)
    with pytest.raises(ValueError):
        _native.tp_shape(4, 0, 4)
    # invalid arguments are rejected before any device work
    with pytest.raises(ValueError):
        _native.call("ictc_tp_fwd", 2, 2, 2, 300, None, None, None, None, 1, None, None)
    with pytest.raises(ValueError):
        _native.call("ictc_sh_fwd", None, 4, 5, None, None)
    assert _native.lib().ictc_csr_workspace_bytes(1000, 10) > 0
    assert _native.lib().ictc_csr_workspace_bytes(-1, 10) < 0


def test_generated_header_covers_natural_configs():
    import sys
    sys.path.insert(0, os.path.join(ROOT, "ictc-o3-hp-k100_amd", "csrc"))
    import gen_tables
    s = gen_tables.tp_struct(2, 2, 2)
    assert "NNZ = 93" in s and "NO = 35" in s and "P = 11" in s


def test_api_validation_cpu():
    from ictc_o3 import EdgeTensorProduct, direction_harmonics
    with pytest.raises(ValueError, match="CUDA device"):
        EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, channels=32, device="cpu")
    with pytest.raises(ValueError, match="nonnegative"):
        EdgeTensorProduct.create(input_lmax=-1, edge_lmax=2, channels=32, device="cuda")
    with pytest.raises(ValueError, match="positive"):
        EdgeTensorProduct.create(input_lmax=1, edge_lmax=2, channels=0, device="cuda")
    with pytest.raises(ValueError, match=r"\[E,3\]"):
        direction_harmonics(torch.zeros(3, 2), 2)
    with pytest.raises(ValueError, match="policy"):
        direction_harmonics(torch.zeros(3, 3), 2, policy="bogus")
    with pytest.raises(ValueError, match="CUDA FP32"):
        direction_harmonics(torch.zeros(3, 3), 2)


def test_tp_module_path_enumeration():
    from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
    tp = EdgeWeightedPathPreservingTensorProduct(8, 2, allowed_paths=orc.natural_paths(2, 2, 2))
    assert tp.paths == orc.natural_paths(2, 2, 2)
    assert tp.path_counts_by_l == {0: 3, 1: 4, 2: 4}
    assert tp.kernel_degrees() == (2, 2, 2)
    assert tp.weight.shape == (11, 8)


def test_receiver_rows_host_checks():
    """Argument checks of the receiver row order entry point (no device work)."""
    from ictc_o3 import _native
    if not os.path.exists(_native.library_path()):
        pytest.skip("library not built")
    lib = _native.lib()
    assert lib.ictc_receiver_rows_workspace_bytes(-1) < 0 and lib.ictc_receiver_rows_workspace_bytes(10) > 0
    with pytest.raises(ValueError, match="negative"):
        _native.call("ictc_receiver_rows", None, -1, None, None, None, 0, None)
    with pytest.raises(ValueError, match="null operand"):
        _native.call("ictc_receiver_rows", None, 10, None, None, None, 0, None)


def test_fused_and_gemm_entry_points_host_checks():
    """Coverage queries and argument checks of the fused message and GEMM entry points (no device work)."""
    from ictc_o3 import _native
    if not os.path.exists(_native.library_path()):
        pytest.skip("library not built")
    lib = _native.lib()
    assert lib.ictc_fused_supported(2, 2, 2, 64) == 1 and lib.ictc_fused_supported(0, 2, 2, 128) == 1
    assert lib.ictc_fused_supported(2, 3, 3, 64) == 0 and lib.ictc_fused_supported(2, 2, 2, 48) == 0
    assert lib.ictc_fused_weight_bytes(11, 64) == 11 * 24 * 1024
    assert lib.ictc_fused_weight_bytes(11, 48) < 0
    with pytest.raises(ValueError, match="not compiled"):
        _native.call("ictc_msg_fused_fwd", 2, 3, 3, 64, None, None, None, None, None, None, 10, 10, None, None, None,
                     None, None, None)
    with pytest.raises(ValueError, match="multiple of 64"):
        _native.call("ictc_msg_fused_fwd", 2, 2, 2, 96, None, None, None, None, None, None, 10, 10, None, None, None,
                     None, None, None)
    with pytest.raises(ValueError, match="dgates is required"):
        _native.call("ictc_msg_bwd_accumulate", 2, 2, 2, 64, None, None, None, None, None, None, None, 10, 10, None,
                     None, None, None, None, None, None, None, None, None, None, 0, None)
    with pytest.raises(ValueError, match="dr is required"):
        _native.call("ictc_msg_fused_bwd_tangent", 2, 2, 2, 64, None, None, None, None, None, None, None, None, 10,
                     10, None, None, None, None, None, None, None, None, None, None, None, None)
    # edge pairs: a graph without edges writes count 0 without touching operands; E >= 2^30 is refused
    assert lib.ictc_edge_pairs_workspace_bytes(1 << 30) < 0 and lib.ictc_edge_pairs_workspace_bytes(1000) > 12000
    with pytest.raises(ValueError, match="negative"):
        _native.call("ictc_edge_pairs", None, None, None, 4, -1, None, None, None, None, None, None, 0, None)
    with pytest.raises(ValueError, match="null count"):
        _native.call("ictc_edge_pairs", None, None, None, 4, 10, None, None, None, None, None, None, 0, None)
    with pytest.raises(ValueError, match="null operand"):
        _native.call("ictc_edge_pairs", None, None, None, 4, 10, None, None, None, None, 1, None, 0, None)
    with pytest.raises(ValueError, match="null source order"):
        _native.call("ictc_edge_pairs_src_csr", None, None, None, 4, 10, None, None, None, None, 1, None, None, None,
                     0, None)
    with pytest.raises(ValueError, match="lda >= k"):
        _native.call("ictc_gemm_nt", None, 4, 8, 4, None, 4, 8, None, 4, 0, None)
    with pytest.raises(ValueError, match="pitch"):
        _native.call("ictc_gate_gemm_bwd_strided", None, 100, 10, 128, None, 64, None, 0, None)
    with pytest.raises(ValueError, match="static scratch"):
        _native.call("ictc_radial_gates_tangent_fwd_noalloc", None, 10, 8, 64, 4.5, 5, None, None, None, None,
                     4096 + 16, 1.0, None, None, None)


def test_weight_operand_cache_follows_versions():
    """The packed linears' weight operands: contiguous weights pass through; a view or transpose is copied
    once per live base, view and version, and an in-place update (new version) gives a fresh copy."""
    from ictc_o3.ops.linear import _weight_operand
    w = torch.randn(3 * 16 * 16)
    blk = w[256:512].view(16, 16).t()
    a = _weight_operand(blk)
    assert a.is_contiguous() and torch.equal(a, blk) and _weight_operand(blk) is a
    assert _weight_operand(w[256:512].view(16, 16).t()) is a          # the same view taken anew
    t = _weight_operand(a, transpose=True)
    assert torch.equal(t, a.t()) and _weight_operand(a, transpose=True) is t
    with torch.no_grad():
        w.mul_(2.0)
    b = _weight_operand(blk)
    assert b is not a and torch.equal(b, blk)
    c = torch.randn(16, 16)
    assert _weight_operand(c) is not None and _weight_operand(c).data_ptr() == c.data_ptr()


def test_species_entry_points_host_checks():
    """Argument checks of the species-sorted self connection and its weight gradient (no device work)."""
    from ictc_o3 import _native
    if not os.path.exists(_native.library_path()):
        pytest.skip("library not built")
    lib = _native.lib()
    assert lib.ictc_species_outer_workspace_bytes(1000, 128, 10, 128) == (8 + 10) * 128 * 128 * 4
    assert lib.ictc_species_outer_workspace_bytes(1000, 128, 10, 100) < 0      # tile rows not a multiple of 32
    assert lib.ictc_species_outer_workspace_bytes(1000, 64, 0, 128) < 0        # no species
    # zero nodes: nothing to do, no operand is touched
    _native.call("ictc_species_linear", None, 64, 0, 64, None, 3, None, None, 0, None, 64, None)
    with pytest.raises(ValueError, match="64 and 128"):
        _native.call("ictc_species_linear", None, 32, 10, 32, None, 3, None, None, 0, None, 32, None)
    with pytest.raises(ValueError, match="pitch"):
        _native.call("ictc_species_linear", None, 66, 10, 64, None, 3, None, None, 0, None, 64, None)
    with pytest.raises(ValueError, match="null operand"):
        _native.call("ictc_species_linear", None, 64, 10, 64, None, 3, None, None, 0, None, 64, None)
    with pytest.raises(ValueError, match="multiple of 32"):
        _native.call("ictc_species_outer", None, 64, None, 64, 10, 64, 3, None, None, 48, None, None, 0, None)
    with pytest.raises(ValueError, match="64 and 128"):
        _native.call("ictc_species_outer", None, 96, None, 96, 10, 96, 3, None, None, 128, None, None, 0, None)
