"""Pins the float64 oracle against the reference's fixtures and the mathematics.

Fixture: the SHA-256 table of the frozen basis (ictc_o3/basis/ictd_irreps.py:659-673).
Mathematics: harmonicity, Gaussian orthonormality, |Y_l|^2 = 2l+1, parity,
rotation covariance, CG equivariance, closed-form l=0 couplings, element
normalisation, multilinearity, edge-order invariance, finite differences.
"""
import hashlib
import math

import numpy as np
import pytest
import torch

import ictc_oracle as orc
from helpers import random_rotation, rel_err, unit_vectors, wigner_ictc

# ictc_o3/basis/ictd_irreps.py:659-673
SHA = {
    0: "6c3c396ed6b5c36dcae172271f462051b1266b851e92df3deea8ac65478fd712",
    1: "1332df685c45a61a0ac008a6a653295b8c5655361c1d34b6304b22ec40235fb8",
    2: "0881fbfd2a1866b76334d823d216ec74773a91a5f77234c45bb956838df7c315",
    3: "a7440553d51231cc044287b305d35cb5cafc59f77d7528d8189956c51a52a9e0",
    4: "f89f4b7f49ed9be8cc7fbbcec5e1a8947442c612d239bd42ce36180c6c644225",
    5: "8cce9bfb0a710f2c19d50ca3bcf6a79593697b5bd129085f10422066c2030ea8",
    6: "01cc08fe54c00daaff6899a86c923b62433f1691b7f283b95643c7be78ce9a96",
    12: "761c7af5c246722d57a910b32ffe82741ac39326d6cba627be7db3b14d4ab689",
}


@pytest.mark.parametrize("l", sorted(SHA))
def test_basis_fixture_sha(l):
    B = orc.harmonic_basis(l)
    assert B.shape == (orc.sym_dim(l), 2 * l + 1)
    assert hashlib.sha256(np.ascontiguousarray(B, dtype="<f8").tobytes()).hexdigest() == SHA[l]


@pytest.mark.parametrize("l", range(2, 7))
def test_basis_is_harmonic_and_gaussian_orthonormal(l):
    B = orc.harmonic_basis(l)
    assert np.abs(orc.laplacian_matrix(l) @ B).max() < 1e-12
    G = orc.gram_gaussian(l)
    assert np.abs(B.T @ G @ B - np.eye(2 * l + 1)).max() < 1e-10


def test_counts_order_matches_reference_docstring():
    # ictd_irreps.py:1216-1218: l=2 monomial order z^2, yz, y^2, xz, xy, x^2
    assert orc.counts_list(2) == [(0, 0, 2), (0, 1, 1), (0, 2, 0), (1, 0, 1), (1, 1, 0), (2, 0, 0)]


@pytest.mark.parametrize("lmax", [3])
def test_harmonics_norm_parity_and_l0(lmax):
    n = unit_vectors(100, 1)
    Y = orc.direction_harmonics(n, lmax)
    Yn = orc.direction_harmonics(-n, lmax)
    assert torch.allclose(Y[0], torch.ones(100, 1, dtype=torch.float64))
    for l in range(lmax + 1):
        assert torch.allclose((Y[l] ** 2).sum(-1), torch.full((100,), 2.0 * l + 1, dtype=torch.float64))
        assert torch.allclose(Yn[l], (-1) ** l * Y[l])


def test_harmonics_component_rms_on_sphere():
    # component normalisation: each component has mean square 1 over the sphere (ictd_irreps.py:952-985)
    n = unit_vectors(200000, 2)
    for l, Y in enumerate(orc.direction_harmonics(n, 3)):
        ms = (Y ** 2).mean(0)
        assert (ms - 1).abs().max() < 0.03


def test_harmonics_rotation_covariance_is_orthogonal():
    R = random_rotation(3)
    for l in range(1, 4):
        D = wigner_ictc(R, l)
        assert torch.allclose(D @ D.T, torch.eye(2 * l + 1, dtype=torch.float64), atol=1e-10)
        n = unit_vectors(10, 4)
        lhs = orc.direction_harmonics(n @ torch.tensor(R).T, l)[l]
        assert torch.allclose(lhs, orc.direction_harmonics(n, l)[l] @ D.T, atol=1e-10)


def test_l1_harmonics_closed_form():
    # Y_1 = sqrt(3) (z, y, x) in the monomial order of counts_list(1)
    n = unit_vectors(7, 5)
    Y1 = orc.direction_harmonics(n, 1)[1]
    assert torch.allclose(Y1, math.sqrt(3) * n[:, [2, 1, 0]], atol=1e-12)


@pytest.mark.parametrize("path", orc.natural_paths(3, 3, 3))
def test_cg_equivariance_and_norm(path):
    l1, l2, l3 = path
    C = torch.tensor(orc.cg_component(l1, l2, l3))
    assert abs(C.norm().item() - math.sqrt(2 * l3 + 1)) < 1e-10
    R = random_rotation(11)
    D1, D2, D3 = (wigner_ictc(R, l) for l in (l1, l2, l3))
    lhs = torch.einsum("ai,bj,ijk->abk", D1, D2, C)
    rhs = torch.einsum("abk,kc->abc", C, D3.T)
    # C(D1 a, D2 b) = D3 C(a, b)  <=>  D1^T ... ; check on random vectors
    g = torch.Generator().manual_seed(12)
    a = torch.randn(2 * l1 + 1, generator=g, dtype=torch.float64)
    b = torch.randn(2 * l2 + 1, generator=g, dtype=torch.float64)
    out_rot = torch.einsum("i,j,ijk->k", D1 @ a, D2 @ b, C)
    rot_out = D3 @ torch.einsum("i,j,ijk->k", a, b, C)
    assert torch.allclose(out_rot, rot_out, atol=1e-9)


@pytest.mark.parametrize("l", range(4))
def test_cg_scalar_paths_are_identities(l):
    # (0,l,l) and (l,0,l) couple through the identity: t_l * 1 projected back onto degree l
    eye = np.eye(2 * l + 1)
    assert np.abs(orc.cg_component(0, l, l)[0] - eye).max() < 1e-12
    assert np.abs(orc.cg_component(l, 0, l)[:, 0, :] - eye).max() < 1e-12


def test_cg_forbidden_paths_zero():
    assert not orc.cg_tensor(1, 1, 1).any()
    assert not orc.cg_tensor(2, 1, 4).any()


def test_path_tables_p11():
    paths = orc.natural_paths(2, 2, 2)
    assert paths == [(0, 0, 0), (0, 1, 1), (0, 2, 2), (1, 0, 1), (1, 1, 0), (1, 1, 2), (1, 2, 1),
                     (2, 0, 2), (2, 1, 1), (2, 2, 0), (2, 2, 2)]
    cgs, offsets, counts = orc.path_tables(paths)
    assert counts == {0: 3, 1: 4, 2: 4}
    assert offsets == [0, 0, 0, 1, 1, 1, 2, 2, 3, 2, 3]
    # element normalisation: 1/sqrt(count_l3)
    for p, (l1, l2, l3) in enumerate(paths):
        assert abs(np.linalg.norm(cgs[p]) - math.sqrt(2 * l3 + 1) / math.sqrt(counts[l3])) < 1e-12
    assert sum(c * (2 * l + 1) for l, c in counts.items()) == 35


def _tp_inputs(E, C, li, le, seed):
    g = torch.Generator().manual_seed(seed)
    x = {l: torch.randn(E, C, 2 * l + 1, generator=g, dtype=torch.float64) for l in range(li + 1)}
    n = unit_vectors(E, seed + 1)
    Yl = orc.direction_harmonics(n, le)
    Y = {l: Yl[l] for l in range(le + 1)}
    return x, Y, n


def test_edge_tp_equivariance():
    li, le, lo, C, E = 2, 2, 2, 3, 5
    paths = orc.natural_paths(li, le, lo)
    x, Y, n = _tp_inputs(E, C, li, le, 20)
    gates = torch.randn(E, len(paths), C, dtype=torch.float64)
    out = orc.edge_tp_blocks(x, Y, gates, paths)
    R = random_rotation(21)
    D = {l: wigner_ictc(R, l) for l in range(3)}
    xr = {l: x[l] @ D[l].T for l in x}
    Yr = {l: orc.direction_harmonics(n @ torch.tensor(R).T, le)[l] for l in Y}
    outr = orc.edge_tp_blocks(xr, Yr, gates, paths)
    for l in out:
        assert torch.allclose(outr[l], out[l] @ D[l].T, atol=1e-9)


def test_edge_tp_scalar_path_closed_form():
    # path (0, l, l) with unit weight: out = x0 * Y_l * g / sqrt(count_l)
    paths = orc.natural_paths(0, 2, 2)
    x, Y, _ = _tp_inputs(4, 3, 0, 2, 30)
    gates = torch.randn(4, 3, 3, dtype=torch.float64)
    out = orc.edge_tp_blocks(x, Y, gates, paths)
    for p, (_, l, _) in enumerate(paths):
        expect = x[0] * Y[l].unsqueeze(1) * gates[:, p, :].unsqueeze(-1)
        assert torch.allclose(out[l], expect, atol=1e-12)


def test_edge_tp_multilinear():
    paths = orc.natural_paths(2, 2, 2)
    x, Y, _ = _tp_inputs(3, 2, 2, 2, 40)
    x2, _, _ = _tp_inputs(3, 2, 2, 2, 41)
    g = torch.randn(3, len(paths), 2, dtype=torch.float64)
    a = orc.edge_tp_blocks({l: 2 * x[l] + 3 * x2[l] for l in x}, Y, g, paths)
    b1 = orc.edge_tp_blocks(x, Y, g, paths)
    b2 = orc.edge_tp_blocks(x2, Y, g, paths)
    for l in a:
        assert torch.allclose(a[l], 2 * b1[l] + 3 * b2[l], atol=1e-12)


def test_packed_layout_roundtrip():
    x, _, _ = _tp_inputs(3, 4, 2, 0, 50)
    flat = orc.pack_ir_mul(x, 2)
    assert flat.shape == (3, 36)
    # component k of degree l at (l*l+m)*C + c
    assert flat[1, (1 + 2) * 4 + 3] == x[1][1, 3, 2]
    back = orc.unpack_ir_mul(flat, 4, 2)
    for l in x:
        assert torch.equal(back[l], x[l])


def test_message_edge_order_invariance():
    N, E, C = 6, 20, 2
    g = torch.Generator().manual_seed(60)
    feats = torch.randn(N, C * 9, generator=g, dtype=torch.float64)
    n = unit_vectors(E, 61)
    sh = torch.cat(orc.direction_harmonics(n, 2), -1)
    gates = torch.randn(E, 11 * C, generator=g, dtype=torch.float64)
    src = torch.randint(0, N, (E,), generator=g)
    dst = torch.randint(0, N, (E,), generator=g)
    out = orc.message_packed(feats, sh, gates, src, dst, None, 2, 2, 2, C)
    perm = torch.randperm(E, generator=g)
    out2 = orc.message_packed(feats, sh[perm], gates[perm], src[perm], dst[perm], None, 2, 2, 2, C)
    assert torch.allclose(out, out2, atol=1e-12)
    # a single edge equals the edge TP of its gathered source row
    one = orc.message_packed(feats, sh[:1], gates[:1], src[:1], dst[:1], None, 2, 2, 2, C)
    edge = orc.edge_tp_packed(feats[src[:1]], sh[:1], gates[:1], 2, 2, 2, C)
    assert torch.allclose(one[dst[0]], edge[0])


def test_oracle_gradcheck_tiny():
    C = 2
    g = torch.Generator().manual_seed(70)
    feats = torch.randn(3, C * 4, generator=g, dtype=torch.float64, requires_grad=True)
    n = unit_vectors(3, 71).requires_grad_(True)
    gates = torch.randn(3, 4 * C, generator=g, dtype=torch.float64, requires_grad=True)

    def f(x, nn, gg):
        sh = torch.cat(orc.direction_harmonics(nn, 1), -1)
        return orc.edge_tp_packed(x, sh, gg, 1, 1, 1, C)
    assert torch.autograd.gradcheck(f, (feats, n, gates))
    assert torch.autograd.gradgradcheck(f, (feats, n, gates))


def _cg0(l1, l2, l3):
    """<l1 0 l2 0 | l3 0> from sympy (Racah's closed form), float."""
    from sympy.physics.quantum.cg import CG
    return float(CG(l1, 0, l2, 0, l3, 0).doit())


def _coupling_identity_error(cg, l1, l2, l3, seed):
    """max |sum_{m1 m2} C[m1,m2,m3] Y_l1(n)[m1] Y_l2(n)[m2] - s Y_l3(n)[m3]| with
    s = +sqrt((2l1+1)(2l2+1)/(2l3+1)) |<l1 0 l2 0|l3 0>|.

    The reference's coupling tensor is the harmonic projection of the product
    polynomial (ictd_irreps.py:1245-1304), scaled by a positive factor
    (:151-157), so contracting it with two harmonics of the same direction
    returns a positive multiple of Y_l3: this fixes the sign and the magnitude
    of every path, which equivariance and the Frobenius norm leave open.
    """
    n = unit_vectors(16, seed)
    Y = orc.direction_harmonics(n, max(l1, l2, l3))
    lhs = torch.einsum("ei,ej,ijk->ek", Y[l1], Y[l2], torch.as_tensor(cg, dtype=torch.float64))
    s = math.sqrt((2 * l1 + 1) * (2 * l2 + 1) / (2 * l3 + 1)) * abs(_cg0(l1, l2, l3))
    return float((lhs - s * Y[l3]).abs().max())


@pytest.mark.parametrize("path", orc.natural_paths(3, 3, 3))
def test_cg_sign_and_magnitude_pinned_by_harmonic_product(path):
    l1, l2, l3 = path
    assert _coupling_identity_error(orc.cg_component(l1, l2, l3), l1, l2, l3, 20 + l1 + 4 * l2 + 16 * l3) < 1e-10


@pytest.mark.parametrize("path", orc.natural_paths(3, 3, 3))
def test_product_coupling_tables_pinned_by_harmonic_product(path):
    """The tables the kernels are generated from (ictc_o3/basis/tables.py) obey the same identity."""
    from ictc_o3.basis import tables
    l1, l2, l3 = path
    assert _coupling_identity_error(tables.coupling_component(l1, l2, l3), l1, l2, l3, 7 + l1 + 4 * l2) < 1e-10


def test_coupling_identity_detects_a_sign_flip():
    """A single path with its sign flipped fails the identity (the check is not vacuous)."""
    C = -orc.cg_component(1, 1, 2)
    assert _coupling_identity_error(C, 1, 1, 2, 3) > 0.1
    C = orc.cg_component(2, 2, 2).copy()
    C[..., 0] *= -1     # one flipped m3 column
    assert _coupling_identity_error(C, 2, 2, 2, 3) > 0.1
