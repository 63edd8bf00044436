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


# ---------------------------------------------------------------------------
# Pins of e3nn's wigner_3j convention (the blocks the U matrices are built from, reference
# ictc_o3/basis/_mace_cg.py:80) against what the mathematics fixes, independently of both restatements.
#
# e3nn: w3j(l1,l2,l3)[j,k,m] = normalise( sum Q1[a,j] Q2[b,k] conj(Q3[c,m]) CG[a,b,c] ), Q_l = (-i)^l q_l,
# q_l the real->complex change of basis of the real spherical harmonics, CG Condon-Shortley.  With
# q_l taken from the reference's own SH (bridge fixture) and an independent library's complex SH,
# the closed forms below follow (derivations in the test docstrings).
# ---------------------------------------------------------------------------

def _triangles(lmax):
    return [(a, b, c) for a in range(lmax + 1) for b in range(lmax + 1) for c in range(lmax + 1)
            if abs(a - b) <= c <= a + b]


def _w3j_both(l1, l2, l3):
    from ictc_o3.basis import e3nn_basis as e
    return {"oracle": so.wigner_3j(l1, l2, l3), "product": e.wigner_3j(l1, l2, l3)}


def _reference_real_sh(l, n):
    """e3nn real SH of the reference's convention: ICTC harmonics times the reference's bridge Q fixture."""
    import ictc_oracle as orc
    return orc.direction_harmonics(torch.tensor(n), l)[l].numpy() @ so.q_block(l)


def _sphere_quadrature(deg=12):
    """Nodes and weights on S^2 exact for polynomials of degree <= deg (Gauss-Legendre x trapezoid)."""
    nt, nphi = deg // 2 + 2, deg + 2
    x, w = np.polynomial.legendre.leggauss(nt)
    phi = 2 * np.pi * np.arange(nphi) / nphi
    st = np.sqrt(1 - x ** 2)
    n = np.stack([np.outer(st, np.cos(phi)), np.outer(st, np.sin(phi)), np.outer(x, np.ones(nphi))], -1)
    return n.reshape(-1, 3), np.outer(w, np.full(nphi, 2 * np.pi / nphi)).reshape(-1)


def _q_from_library(l):
    """q_l fitted from scipy's complex Condon-Shortley SH against the reference's real SH: Y_m = sum_j q[m,j] y_j,
    scaled so that q is unitary (the two SH normalisations differ by a positive constant).

    e3nn's polar axis is y: its real SH at (x, y, z) are the textbook real SH at (x', y', z') = (z, x, y),
    whose l = 1 components (m = -1, 0, 1) are (y', z', x') = (x, y, z).  scipy is evaluated in that frame."""
    from scipy.special import sph_harm_y
    rng = np.random.default_rng(40 + l)
    n = rng.standard_normal((200, 3))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    xs, ys, zs = n[:, 2], n[:, 0], n[:, 1]
    theta, phi = np.arccos(np.clip(zs, -1, 1)), np.arctan2(ys, xs)
    Yc = np.stack([sph_harm_y(l, m, theta, phi) for m in range(-l, l + 1)], 1)      # [S, 2l+1]
    y = _reference_real_sh(l, n)
    A = np.linalg.lstsq(y.astype(complex), Yc, rcond=None)[0].T                       # Yc = y @ A^T
    assert np.abs(y @ A.T - Yc).max() < 1e-10
    s = np.sqrt((2 * l + 1) / np.real(np.trace(A.conj().T @ A)))
    return A * s


@pytest.mark.parametrize("l", range(5))
def test_real_to_complex_basis_matches_library_harmonics(l):
    """Both restatements' q_l (without e3nn's (-i)^l factor) equal the map from the reference's real SH to scipy's
    complex SH: pins every per-m sign and the ordering of the real basis (y as polar axis)."""
    from ictc_o3.basis import e3nn_basis as e
    ql = _q_from_library(l)
    assert np.abs(ql.conj().T @ ql - np.eye(2 * l + 1)).max() < 1e-10
    assert np.abs(so._q_real_complex(l) / (-1j) ** l - ql).max() < 1e-10
    assert np.abs(e.real_to_complex(l) / (-1j) ** l - ql).max() < 1e-10


@pytest.mark.parametrize("l", range(5))
def test_w3j_blocks_with_a_scalar_leg_are_plus_identity(l):
    """w3j(0,l,l) = w3j(l,0,l) = w3j(l,l,0) = +I / sqrt(2l+1).

    <00;lm|lm> = <lm;00|lm> = 1, and Q_0 = 1, so the first two are q_l^T conj(q_l) = I (q unitary, real
    result), normalised.  For (l,l,0): <lm;l,-m|00> = (-1)^(l-m)/sqrt(2l+1) and q_l[-m,:] = (-1)^m conj(q_l[m,:])
    give sum_m (-1)^(l-m) q[m,j] q[-m,k] = (-1)^l delta_jk, times (-i)^(2l) = (-1)^l from Q_l twice: +delta."""
    eye = np.eye(2 * l + 1) / math.sqrt(2 * l + 1)
    for name, blocks in (("0ll", _w3j_both(0, l, l)), ("l0l", _w3j_both(l, 0, l)), ("ll0", _w3j_both(l, l, 0))):
        for who, C in blocks.items():
            shape = {"0ll": (1, 2 * l + 1, 2 * l + 1), "l0l": (2 * l + 1, 1, 2 * l + 1),
                     "ll0": (2 * l + 1, 2 * l + 1, 1)}[name]
            assert C.shape == shape, (name, who)
            assert np.abs(C.reshape(2 * l + 1, 2 * l + 1) - eye).max() < 1e-12, (name, who)


def test_w3j_111_is_plus_levi_civita_in_yzx_order():
    """w3j(1,1,1)[j,k,m] = +eps_jkm / sqrt(6) in e3nn's l=1 basis, the textbook (y', z', x') order.

    Textbook spherical components v_{+1} = -(v_x' + i v_y')/sqrt2, v_0 = v_z', v_{-1} = (v_x' - i v_y')/sqrt2 are
    q_1 v in the (y', z', x') basis (checked against scipy above).  Condon-Shortley coupling of two vectors: [a (x) b]^1 = (i/sqrt2) q_1 (a x b).  With
    Q_1 = -i q_1 on both inputs and conj(Q_1) = i conj(q_1) on the output:
    sum_jk R[j,k,m] a_j b_k = i * (-i)^2 * (i/sqrt2) (q_1^H q_1 (a x b))_m = (a x b)_m / sqrt2, so R is
    +eps/sqrt2 in the (y', z', x') basis, a cyclic relabelling of (x', y', z'), hence +eps_jkm; normalised:
    / sqrt6.  (e3nn's (x, y, z) is that same (y', z', x'), so the cross product reads directly in e3nn axes.)"""
    eps = np.zeros((3, 3, 3))
    for (i, j, k), s in {(0, 1, 2): 1, (1, 2, 0): 1, (2, 0, 1): 1, (0, 2, 1): -1, (2, 1, 0): -1, (1, 0, 2): -1}.items():
        eps[i, j, k] = s
    for who, C in _w3j_both(1, 1, 1).items():
        assert np.abs(C - eps / math.sqrt(6)).max() < 1e-12, who
    # and the cross product it encodes, on the reference's own l = 1 harmonics (y, z, x up to a positive scale)
    a, b = np.array([0.3, -1.2, 0.7]), np.array([1.1, 0.4, -0.5])
    y = lambda v: _reference_real_sh(1, (v / np.linalg.norm(v))[None])[0] * np.linalg.norm(v)
    got = np.einsum("jkm,j,k->m", so.wigner_3j(1, 1, 1), y(a), y(b))
    want = y(np.cross(a, b))
    assert np.abs(got / np.linalg.norm(got) - want / np.linalg.norm(want)).max() < 1e-12


def _gaunt_real(l1, l2, l3):
    n, w = _sphere_quadrature(l1 + l2 + l3 + 2)
    Y1, Y2, Y3 = (_reference_real_sh(l, n) for l in (l1, l2, l3))
    return np.einsum("s,sa,sb,sc->abc", w, Y1, Y2, Y3)


@pytest.mark.parametrize("l1,l2,l3", [t for t in _triangles(4) if sum(t) % 2 == 0])
def test_w3j_even_blocks_are_positive_gaunt_integrals(l1, l2, l3):
    """For l1+l2+l3 even, w3j(l1,l2,l3) = +G / |G| with G[a,b,c] = integral of y_a y_b y_c over the sphere
    (the reference's real SH).  The complex Gaunt integral is kappa <l1 0 l2 0|l3 0> <l1 m1 l2 m2|l3 m3>,
    kappa > 0; in the real basis G = kappa <l1 0 l2 0|l3 0> R, R = sum q1 q2 conj(q3) CG (real for an even
    sum).  e3nn's phases give w3j = (-i)^(l1+l2-l3) R / |R| = (-1)^((l1+l2-l3)/2) R / |R|, and
    sign <l1 0 l2 0|l3 0> = (-1)^((l1+l2-l3)/2): the signs cancel, so every even block is +G/|G|."""
    G = _gaunt_real(l1, l2, l3)
    assert np.linalg.norm(G) > 1e-3
    G = G / np.linalg.norm(G)
    for who, C in _w3j_both(l1, l2, l3).items():
        assert np.abs(C - G).max() < 1e-10, who


@pytest.mark.parametrize("l1,l2,l3", [t for t in _triangles(4) if sum(t) % 2 == 1])
def test_w3j_odd_blocks_from_library_basis_and_sympy_cg(l1, l2, l3):
    """For l1+l2+l3 odd the Gaunt integral vanishes (parity), so these blocks are pinned through their
    ingredients: sympy's Condon-Shortley CG, q_l fitted from scipy's complex SH to the reference's real SH,
    and e3nn's phase (-i)^l, whose choice over i^l the (1,1,1) closed form fixes."""
    C3 = so._cg_su2(l1, l2, l3).astype(complex)
    Q = [(-1j) ** l * _q_from_library(l) for l in (l1, l2, l3)]
    R = np.einsum("aj,bk,cm,abc->jkm", Q[0], Q[1], Q[2].conj(), C3)
    assert np.abs(R.imag).max() < 1e-10
    R = R.real / np.linalg.norm(R.real)
    for who, C in _w3j_both(l1, l2, l3).items():
        assert np.abs(C - R).max() < 1e-10, who


def test_w3j_pins_reject_a_flipped_block_and_the_other_phase():
    """Negative controls: a sign-flipped even block fails the Gaunt pin; i^l in place of (-i)^l turns (1,1,1)
    into -eps/sqrt6 and fails its closed form."""
    G = _gaunt_real(2, 1, 1)
    G = G / np.linalg.norm(G)
    assert np.abs(-so.wigner_3j(2, 1, 1) - G).max() > 0.1
    C3 = so._cg_su2(1, 1, 1).astype(complex)
    q = (1j) * so._q_real_complex(1) / (-1j)
    R = np.einsum("aj,bk,cm,abc->jkm", q, q, q.conj(), C3).real
    R = R / np.linalg.norm(R)
    assert np.abs(R + so.wigner_3j(1, 1, 1)).max() < 1e-12


def _block(l):
    return slice(l * l, (l + 1) ** 2)


@pytest.mark.parametrize("who", ["oracle", "product"])
def test_u_correlation2_closed_forms(who):
    """Correlation 2 by hand from _mace_cg.py:39-117: a right leg l2 (input order) couples to each left row
    l1 (rows sorted by irrep (l, p)) through sqrt(2L+1) w3j(L, l1, l2) ("component" normalisation, out leg
    first), so with 0e+1o+2e inputs:
      L = 0: paths (0,0), (1,1), (2,2), each +I/sqrt(2l+1) on its diagonal block (the pinned w3j(0,l,l));
      L = 1: paths (0,1), (1,0), (1,2), (2,1), each sqrt3 w3j(1, l1, l2) on block (l1, l2);
      L = 2: paths (0,2), (1,1), (2,0), (2,2), each sqrt5 w3j(2, l1, l2).
    Pins the path order, the leg order and the normalisation at correlation 2, where every coupling is one
    w3j block whose sign is pinned above."""
    from ictc_o3.basis import e3nn_basis as e
    U_of = (lambda L: so.u_matrix(2, L, 2)) if who == "oracle" else (lambda L: e.mace_u(2, L, 2))
    paths = {0: [(0, 0), (1, 1), (2, 2)], 1: [(0, 1), (1, 0), (1, 2), (2, 1)], 2: [(0, 2), (1, 1), (2, 0), (2, 2)]}
    for L, plist in paths.items():
        U = U_of(L)
        if L == 0:
            U = U[None]
        assert U.shape == (2 * L + 1, 9, 9, len(plist)), (L, U.shape)
        for p, (l1, l2) in enumerate(plist):
            want = np.zeros((2 * L + 1, 9, 9))
            want[:, _block(l1), _block(l2)] = math.sqrt(2 * L + 1) * so.wigner_3j(L, l1, l2)
            assert np.abs(U[..., p] - want).max() < 1e-12, (L, p)


# Correlation-3 paths written out by hand from _mace_cg.py:39-117 for 0e+1o+2e inputs: the correlation-2
# rows, unfiltered, sorted (stably) by e3nn's irrep order (l, then parity with o = -1 before e = +1):
#   0e: (0,0) (1,1) (2,2) | 1o: (0,1) (1,0) (1,2) (2,1) | 1e: (1,1) (2,2) | 2o: (1,2) (2,1)
#   2e: (0,2) (1,1) (2,0) (2,2) | 3o: (1,2) (2,1) | 3e: (2,2) | 4e: (2,2)
# then, per row in that order, the right leg l3 in input order, keeping the couplings to the target.
_MID = [(0, 1, (0, 0)), (0, 1, (1, 1)), (0, 1, (2, 2)),
        (1, -1, (0, 1)), (1, -1, (1, 0)), (1, -1, (1, 2)), (1, -1, (2, 1)),
        (1, 1, (1, 1)), (1, 1, (2, 2)), (2, -1, (1, 2)), (2, -1, (2, 1)),
        (2, 1, (0, 2)), (2, 1, (1, 1)), (2, 1, (2, 0)), (2, 1, (2, 2)),
        (3, -1, (1, 2)), (3, -1, (2, 1)), (3, 1, (2, 2)), (4, 1, (2, 2))]


def _paths3(L):
    pL = 1 if L % 2 == 0 else -1
    out = []
    for lm, pm, (l1, l2) in _MID:
        for l3 in (0, 1, 2):
            if abs(lm - l3) <= L <= lm + l3 and pm * (1 if l3 % 2 == 0 else -1) == pL:
                out.append((lm, l1, l2, l3))
    return out


@pytest.mark.parametrize("L,count", [(0, 11), (1, 21), (2, 23)])
@pytest.mark.parametrize("who", ["oracle", "product"])
def test_u_correlation3_path_order_and_values(who, L, count):
    """Each correlation-3 path (Lmid from (l1, l2), then l3) is
    sqrt(2L+1) w3j(L, Lmid, l3) contracted with sqrt(2Lmid+1) w3j(Lmid, l1, l2) on block (l1, l2, l3), in the
    hand-written order above; every w3j block is pinned by the tests above."""
    from ictc_o3.basis import e3nn_basis as e
    paths = _paths3(L)
    assert len(paths) == count
    U = so.u_matrix(2, L, 3) if who == "oracle" else e.mace_u(2, L, 3)
    if L == 0:
        U = U[None]
    assert U.shape == (2 * L + 1, 9, 9, 9, count)
    for p, (lm, l1, l2, l3) in enumerate(paths):
        inner = math.sqrt(2 * lm + 1) * so.wigner_3j(lm, l1, l2)                 # [Lmid, l1, l2]
        outer = math.sqrt(2 * L + 1) * so.wigner_3j(L, lm, l3)                   # [L, Lmid, l3]
        want = np.zeros((2 * L + 1, 9, 9, 9))
        want[:, _block(l1), _block(l2), _block(l3)] = np.einsum("imc,mab->iabc", outer, inner)
        assert np.abs(U[..., p] - want).max() < 1e-12, (L, p, (lm, l1, l2, l3))
