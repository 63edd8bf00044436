"""e3nn / MACE angular conventions needed by the bridge-U symmetric contraction.

The reference builds its contraction tensors with e3nn (pinned
``e3nn>=0.4.4,<0.6``, reference pyproject.toml:12) at two call sites:
``o3.wigner_3j`` (ictc_o3/basis/_mace_cg.py:80) and ``o3.spherical_harmonics``
(ictc_o3/basis/bridge.py:48).  e3nn is not a dependency of this build; its
published algorithm is restated here:

* SU(2) Clebsch-Gordan coefficients by the Racah formula (Condon-Shortley phase);
* the real<->complex change of basis of the real spherical harmonics
  (Wikipedia "real form", times (-i)^l so the coupling comes out real);
* wigner_3j(l1, l2, l3) = Re[ Q1 (x) Q2 (x) Q3^H applied to CG ], unit Frobenius norm;
* real spherical harmonics, component normalisation, generated recursively by
  coupling Y_l with Y_1 = sqrt(3) (x, y, z) through wigner_3j(l+1, l, 1).

The MACE generalised coupling U_matrix_real (ictc_o3/basis/_mace_cg.py:39-190)
is restated in ``mace_u``; the ICTC <-> e3nn bridge (bridge.py:26-62) in
``bridge_q``.  All results are float64 numpy arrays.
"""
from __future__ import annotations

import math
from fractions import Fraction
from functools import lru_cache
from typing import Dict, List, Tuple

import numpy as np


# ---------------------------------------------------------------------------
# SU(2) Clebsch-Gordan (Racah formula) and the real basis
# ---------------------------------------------------------------------------


def _fact(n) -> int:
    n = int(round(n))
    if n < 0:
        raise ValueError("negative factorial")
    return math.factorial(n)


def su2_cg(j1: int, m1: int, j2: int, m2: int, j3: int, m3: int) -> float:
    """<j1 m1 j2 m2 | j3 m3> for integer spins (Racah's closed form)."""
    if m3 != m1 + m2 or abs(m1) > j1 or abs(m2) > j2 or abs(m3) > j3:
        return 0.0
    if not (abs(j1 - j2) <= j3 <= j1 + j2):
        return 0.0
    pref = Fraction((2 * j3 + 1) * _fact(j3 + j1 - j2) * _fact(j3 - j1 + j2) * _fact(j1 + j2 - j3),
                    _fact(j1 + j2 + j3 + 1))
    pref *= Fraction(_fact(j3 + m3) * _fact(j3 - m3),
                     _fact(j1 - m1) * _fact(j1 + m1) * _fact(j2 - m2) * _fact(j2 + m2))
    s = Fraction(0)
    for v in range(0, j1 + j2 + j3 + 2):
        den = [v, j3 - j1 + j2 - v, j3 + m3 - v, v + j1 - j2 - m3]
        num = [j2 + j3 + m1 - v, j1 - m1 + v]
        if min(den) < 0 or min(num) < 0:
            continue
        s += (-1) ** (v + j2 + m2) * Fraction(_fact(num[0]) * _fact(num[1]),
                                              _fact(den[0]) * _fact(den[1]) * _fact(den[2]) * _fact(den[3]))
    return float(math.sqrt(pref)) * float(s)


def su2_cg_tensor(j1: int, j2: int, j3: int) -> np.ndarray:
    out = np.zeros((2 * j1 + 1, 2 * j2 + 1, 2 * j3 + 1))
    for m1 in range(-j1, j1 + 1):
        for m2 in range(-j2, j2 + 1):
            m3 = m1 + m2
            if abs(m3) <= j3:
                out[j1 + m1, j2 + m2, j3 + m3] = su2_cg(j1, m1, j2, m2, j3, m3)
    return out


def real_to_complex(l: int) -> np.ndarray:
    """q[complex m + l, real index]: complex SH = q @ real SH, times (-i)^l."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=np.complex128)
    s = 1 / math.sqrt(2)
    for m in range(-l, 0):
        q[l + m, l + abs(m)] = s
        q[l + m, l - abs(m)] = -1j * s
    q[l, l] = 1.0
    for m in range(1, l + 1):
        q[l + m, l + m] = (-1) ** m * s
        q[l + m, l - m] = 1j * (-1) ** m * s
    return ((-1j) ** l) * q


@lru_cache(maxsize=None)
def wigner_3j(l1: int, l2: int, l3: int) -> np.ndarray:
    """Real, unit-norm coupling [2l1+1, 2l2+1, 2l3+1] of e3nn's real irreps."""
    if not (abs(l2 - l3) <= l1 <= l2 + l3):
        raise ValueError("triangle condition")
    Q1, Q2, Q3 = real_to_complex(l1), real_to_complex(l2), real_to_complex(l3)
    C = su2_cg_tensor(l1, l2, l3).astype(np.complex128)
    R = np.einsum("ij,kl,nm,ikn->jlm", Q1, Q2, Q3.conj(), C)
    if np.abs(R.imag).max() > 1e-8:
        raise RuntimeError("coupling did not come out real")
    R = R.real
    return R / np.linalg.norm(R)


# ---------------------------------------------------------------------------
# Real spherical harmonics (component normalisation)
# ---------------------------------------------------------------------------


@lru_cache(maxsize=None)
def _sh_polynomials(l: int) -> Dict[Tuple[int, int, int], np.ndarray]:
    """Y_l as {(a,b,c): coefficient vector over m} of x^a y^b z^c, |Y_l|^2 = 2l+1 on the sphere."""
    if l == 0:
        return {(0, 0, 0): np.ones(1)}
    if l == 1:
        r3 = math.sqrt(3)
        return {(1, 0, 0): np.array([r3, 0, 0]), (0, 1, 0): np.array([0, r3, 0]), (0, 0, 1): np.array([0, 0, r3])}
    prev = _sh_polynomials(l - 1)
    C = wigner_3j(l, l - 1, 1)        # [out, left, right]
    unit = [(1, 0, 0), (0, 1, 0), (0, 0, 1)]
    poly: Dict[Tuple[int, int, int], np.ndarray] = {}
    for mono, coef in prev.items():
        for j, e in enumerate(unit):
            key = (mono[0] + e[0], mono[1] + e[1], mono[2] + e[2])
            poly[key] = poly.get(key, 0) + C[:, :, j] @ coef
    # component normalisation on the unit sphere: mean of each component squared = 1
    rng = np.random.default_rng(0)
    n = rng.standard_normal((4096, 3))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    vals = _eval(poly, n, 2 * l + 1)
    scale = math.sqrt((2 * l + 1) / np.mean(np.sum(vals ** 2, axis=1)))
    return {k: v * scale for k, v in poly.items()}


def _eval(poly, n, width):
    out = np.zeros((n.shape[0], width))
    for (a, b, c), coef in poly.items():
        out += np.outer(n[:, 0] ** a * n[:, 1] ** b * n[:, 2] ** c, coef)
    return out


def spherical_harmonics(l: int, n: np.ndarray) -> np.ndarray:
    """e3nn-convention real SH of degree l at unit vectors n [E,3] -> [E, 2l+1]."""
    return _eval(_sh_polynomials(l), np.asarray(n, dtype=np.float64), 2 * l + 1)


# ---------------------------------------------------------------------------
# ICTC <-> e3nn bridge (bridge.py:26-62)
# ---------------------------------------------------------------------------


@lru_cache(maxsize=None)
def bridge_q(l: int) -> np.ndarray:
    """Orthogonal Q_l with Y_ictc_l @ Q_l = Y_e3nn_l (Procrustes fit on sample directions)."""
    from ictc_o3.basis import tables
    rng = np.random.default_rng(20260426)
    n = rng.standard_normal((2048, 3))
    n /= np.linalg.norm(n, axis=1, keepdims=True)
    mono, coef = tables.harmonic_polynomials(l)
    a = np.zeros((n.shape[0], 2 * l + 1))
    for k, (p, q, r) in enumerate(mono):
        a += np.outer(n[:, 0] ** p * n[:, 1] ** q * n[:, 2] ** r, coef[k])
    b = spherical_harmonics(l, n)
    u, _, vh = np.linalg.svd(a.T @ b)
    return u @ vh


# ---------------------------------------------------------------------------
# MACE generalised coupling U (ictc_o3/basis/_mace_cg.py:39-190)
# ---------------------------------------------------------------------------

# An irrep is (l, p) with p = +1 (even) / -1 (odd); ordering is that of the tuple.
Irrep = Tuple[int, int]


def hidden_irreps(lmax: int) -> List[Irrep]:
    """0e + 1o + 2e + ... (bridge.py:10-11)."""
    return [(l, 1 if l % 2 == 0 else -1) for l in range(lmax + 1)]


def _irrep_products(a: Irrep, b: Irrep):
    return [(l, a[1] * b[1]) for l in range(abs(a[0] - b[0]), a[0] + b[0] + 1)]


def _coupled_bases(irreps: List[Irrep], order: int, keep_out: List[Irrep] | None):
    """[(irrep, tensor [2l+1, dim, ..., dim])] for the order-fold coupling, in MACE's path order.

    order 1 is the identity embedding of each input irrep; order k couples the
    (sorted) order k-1 list with each input irrep through wigner_3j scaled by
    sqrt(2 l_out + 1), then stably sorts by irrep (only the outermost level is
    filtered by ``keep_out``).
    """
    dim = sum(2 * l + 1 for l, _ in irreps)
    offsets, o = [], 0
    for l, _ in irreps:
        offsets.append(o)
        o += 2 * l + 1
    if order == 1:
        eye = np.eye(dim)
        base = [((l, p), eye[offsets[i]:offsets[i] + 2 * l + 1]) for i, (l, p) in enumerate(irreps)]
        return base if keep_out is None else [row for row in base if row[0] in keep_out]
    left = _coupled_bases(irreps, order - 1, None)
    rows = []
    for ir_left, c_left in left:
        for i, ir in enumerate(irreps):
            for ir_out in _irrep_products(ir_left, ir):
                if keep_out is not None and ir_out not in keep_out:
                    continue
                w = wigner_3j(ir_out[0], ir_left[0], ir[0]) * math.sqrt(2 * ir_out[0] + 1)
                c = np.einsum("jk,ijl->ikl", c_left.reshape(c_left.shape[0], -1), w)
                c = c.reshape(2 * ir_out[0] + 1, *([dim] * (order - 1)), 2 * ir[0] + 1)
                e = np.zeros((2 * ir_out[0] + 1, *([dim] * order)))
                e[..., offsets[i]:offsets[i] + 2 * ir[0] + 1] = c
                rows.append((ir_out, e))
    rows.sort(key=lambda r: r[0])
    return rows


@lru_cache(maxsize=None)
def mace_u(lmax_in: int, l_out: int, order: int) -> np.ndarray:
    """U for output irrep l_out (natural parity), e3nn basis.

    Shape [2l_out+1, dim^order..., P] (the leading axis dropped when l_out = 0),
    paths in MACE's order (_mace_cg.py:118-190); P may be 0.
    """
    irreps = hidden_irreps(lmax_in)
    dim = sum(2 * l + 1 for l, _ in irreps)
    target = (l_out, 1 if l_out % 2 == 0 else -1)
    rows = [e for ir, e in _coupled_bases(irreps, order, [target]) if ir == target]
    if not rows:
        shape = ([2 * l_out + 1] if l_out else []) + [dim] * order + [0]
        return np.zeros(shape)
    U = np.stack(rows, -1)
    return U[0] if l_out == 0 else U


def mace_u_ictc(lmax_in: int, l_out: int, order: int) -> np.ndarray:
    """U with the bridge folded in: ICTC-basis inputs and outputs (symmetric_contraction.py:50-96)."""
    U = mace_u(lmax_in, l_out, order)
    q_in = np.zeros((0, 0))
    blocks = [bridge_q(l) for l in range(lmax_in + 1)]
    dim = sum(b.shape[0] for b in blocks)
    q_in = np.zeros((dim, dim))
    o = 0
    for b in blocks:
        q_in[o:o + b.shape[0], o:o + b.shape[0]] = b
        o += b.shape[0]
    lead = 0 if l_out == 0 else 1
    R = U
    for axis in range(lead, lead + order):
        R = np.moveaxis(np.tensordot(q_in, R, axes=([1], [axis])), 0, axis)
    if l_out:
        R = np.tensordot(bridge_q(l_out), R, axes=([1], [0]))
    return R
