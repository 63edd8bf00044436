"""Pins the symmetric-contraction constants (CPU).

e3nn is absent, so its algorithm is restated twice (product: own Racah
formula + own Procrustes; oracle: sympy CG + the reference's bridge-Q
fixture) and pinned by: sympy's CG, the reference fixture
lammps_user_mfftorch/.../mff_mace_basis.h (Q_L4), equivariance of every
coupling and of every U polynomial under random rotations.
"""
import math

import numpy as np
import pytest
import torch

import sc_oracle as so
from helpers import random_rotation, wigner_ictc


def test_su2_cg_matches_sympy():
    from ictc_o3.basis import e3nn_basis as e
    for j1 in range(4):
        for j2 in range(4):
            for j3 in range(abs(j1 - j2), j1 + j2 + 1):
                assert np.abs(e.su2_cg_tensor(j1, j2, j3) - so._cg_su2(j1, j2, j3)).max() < 1e-12


@pytest.mark.parametrize("l", range(5))
def test_e3nn_sh_reproduce_reference_bridge_fixture(l):
    """Y_ictc @ Q_fixture == e3nn SH: pins the SH convention (and the bridge) for l <= 4."""
    from ictc_o3.basis import e3nn_basis as e
    assert np.abs(e.bridge_q(l) - so.q_block(l)).max() < 1e-12
    rng = np.random.default_rng(l)
    n = rng.standard_normal((50, 3))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    import ictc_oracle as orc
    y_ictc = orc.direction_harmonics(torch.tensor(n), l)[l].numpy()
    assert np.abs(y_ictc @ so.q_block(l) - e.spherical_harmonics(l, n)).max() < 1e-12


def _e3nn_wigner(R, l):
    from ictc_o3.basis import e3nn_basis as e
    rng = np.random.default_rng(3)
    n = rng.standard_normal((64, 3))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    Y, YR = e.spherical_harmonics(l, n), e.spherical_harmonics(l, n @ R.T)
    return np.linalg.lstsq(Y, YR, rcond=None)[0].T


@pytest.mark.parametrize("l1,l2,l3", [(1, 1, 0), (1, 1, 2), (2, 1, 1), (2, 2, 2), (3, 2, 1), (2, 3, 3), (4, 2, 2)])
def test_wigner_3j_is_intertwiner(l1, l2, l3):
    from ictc_o3.basis import e3nn_basis as e
    C = e.wigner_3j(l1, l2, l3)
    assert abs(np.linalg.norm(C) - 1) < 1e-12
    R = random_rotation(5)
    D1, D2, D3 = (_e3nn_wigner(R, l) for l in (l1, l2, l3))
    lhs = np.einsum("ia,jb,kc,abc->ijk", D1, D2, D3, C)
    assert np.abs(lhs - C).max() < 1e-9


@pytest.mark.parametrize("lmax,lout,nu", [(2, 0, 3), (2, 1, 3), (2, 2, 3), (2, 1, 2), (3, 0, 3), (3, 2, 2)])
def test_u_product_matches_oracle(lmax, lout, nu):
    from ictc_o3.basis import e3nn_basis as e
    a, b = e.mace_u_ictc(lmax, lout, nu), so.u_ictc(lmax, lout, nu)
    assert a.shape == b.shape
    assert np.abs(a - b).max() < 1e-12


@pytest.mark.parametrize("lmax,lout", [(2, 0), (2, 1), (2, 2)])
def test_u_polynomials_equivariant_in_ictc_basis(lmax, lout):
    R = random_rotation(9)
    D = torch.block_diag(*[wigner_ictc(R, l) for l in range(lmax + 1)]).numpy()
    Dout = wigner_ictc(R, lout).numpy()
    rng = np.random.default_rng(1)
    x = rng.standard_normal((lmax + 1) ** 2)
    for nu in (1, 2, 3):
        U = so.u_ictc(lmax, lout, nu)
        if lout == 0:
            U = U[None]
        def full(v):
            T = U
            for _ in range(nu):
                T = np.moveaxis(np.tensordot(T, v, axes=([T.ndim - 2], [0])), -1, -1)
            return T
        a = full(D @ x)
        b = Dout @ full(x)
        assert np.abs(a - b).max() < 1e-9


def test_sc_oracle_path_counts():
    # MACE coupling counts for 0e+1o+2e input, correlation 3
    assert [so.u_matrix(2, 0, nu).shape[-1] for nu in (1, 2, 3)] == [1, 3, 11]
    assert [so.u_matrix(2, 1, nu).shape[-1] for nu in (1, 2, 3)] == [1, 4, 21]
    assert [so.u_matrix(2, 2, nu).shape[-1] for nu in (1, 2, 3)] == [1, 4, 23]


def test_sc_oracle_equivariance_and_species():
    lmax, C, N, S = 2, 3, 6, 2
    g = torch.Generator().manual_seed(2)
    x = torch.randn(N, C, 9, generator=g, dtype=torch.float64)
    species = torch.tensor([0, 1, 1, 0, 1, 0])
    W = {L: {nu: torch.randn(S, so.u_matrix(2, L, nu).shape[-1], C, generator=g, dtype=torch.float64)
             for nu in (1, 2, 3)} for L in range(3)}
    out = so.symmetric_contraction(x, species, W, lmax, 2, 3)
    R = random_rotation(4)
    D = torch.block_diag(*[wigner_ictc(R, l) for l in range(3)])
    outr = so.symmetric_contraction(x @ D.T, species, W, lmax, 2, 3)
    # channel-major blocks per L: [N, C, 2L+1]
    off = 0
    for L in range(3):
        w = C * (2 * L + 1)
        a = outr[:, off:off + w].reshape(N, C, -1)
        b = out[:, off:off + w].reshape(N, C, -1) @ wigner_ictc(R, L).T
        assert torch.allclose(a, b, atol=1e-9)
        off += w
    # species selection: swapping species swaps weight banks
    W2 = {L: {nu: W[L][nu].flip(0) for nu in W[L]} for L in W}
    assert torch.allclose(so.symmetric_contraction(x, 1 - species, W2, lmax, 2, 3), out)
