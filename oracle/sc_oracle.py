"""CPU float64 oracle of the correlation-nu symmetric contraction (bridge-U, ICTC basis).

TEST INFRASTRUCTURE ONLY (see ictc_oracle.py).  Restates, independently of the
product's code:
  * e3nn's wigner_3j (pinned e3nn>=0.4.4,<0.6, reference pyproject.toml:12) from
    sympy's SU(2) Clebsch-Gordan coefficients and the real<->complex basis
    change of the real spherical harmonics;
  * MACE's _wigner_nj / U_matrix_real recursion (ictc_o3/basis/_mace_cg.py:39-190);
  * the bridge fold of U into the ICTC basis (ictc_o3/ops/symmetric_contraction.py:50-96)
    with the bridge Q taken from the reference fixture
    lammps_user_mfftorch/src/USER-MFFTORCH/mff_mace_basis.h (tests/golden/bridge_q_lmax4.json);
  * the species-selected contraction recursion
    (ictc_o3/ops/_mace_symmetric_contraction.py:298-355).

Pinning (tests/test_sc_oracle.py): SU(2) CG from sympy; the real->complex
basis q_l against scipy's complex SH and the reference's real SH (fixture Q);
every wigner_3j block up to l = 4 against closed forms ((0,l,l), (l,0,l),
(l,l,0), (1,1,1)), positive Gaunt integrals (even blocks) and the sympy/scipy
construction (odd blocks); U at correlations 2 and 3 path by path against
lists written out by hand from the recursion; U symmetric-part equivariance.
The one rule taken from e3nn rather than mathematics: rows sort by irrep
(l, then parity o before e).
"""
from __future__ import annotations

import json
import math
import os
from functools import lru_cache

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_Q_FIXTURE = os.path.join(_HERE, "..", "tests", "golden", "bridge_q_lmax4.json")


@lru_cache(maxsize=None)
def _cg_su2(j1, j2, j3):
    from sympy.physics.quantum.cg import CG
    out = np.zeros((2 * j1 + 1, 2 * j2 + 1, 2 * j3 + 1))
    for m1 in range(-j1, j1 + 1):
        for m2 in range(-j2, j2 + 1):
            if abs(m1 + m2) <= j3:
                out[j1 + m1, j2 + m2, j3 + m1 + m2] = float(CG(j1, m1, j2, m2, j3, m1 + m2).doit())
    return out


def _q_real_complex(l):
    """e3nn change_basis_real_to_complex (Wikipedia real form, times (-i)^l)."""
    q = np.zeros((2 * l + 1, 2 * l + 1), dtype=complex)
    r = 2 ** -0.5
    for m in range(-l, l + 1):
        if m < 0:
            q[l + m, l - m] = r
            q[l + m, l + m] = -1j * r
        elif m == 0:
            q[l, l] = 1
        else:
            q[l + m, l + m] = (-1) ** m * r
            q[l + m, l - m] = 1j * (-1) ** m * r
    return (-1j) ** l * q


@lru_cache(maxsize=None)
def wigner_3j(l1, l2, l3):
    C = _cg_su2(l1, l2, l3).astype(complex)
    Q1, Q2, Q3 = _q_real_complex(l1), _q_real_complex(l2), _q_real_complex(l3)
    R = np.einsum("ij,kl,mn,ikn->jlm", Q1, Q2, np.conj(Q3.T), C)
    assert np.abs(R.imag).max() < 1e-10
    R = R.real
    return R / np.linalg.norm(R)


def _mul(ir1, ir2):
    return [(l, ir1[1] * ir2[1]) for l in range(abs(ir1[0] - ir2[0]), ir1[0] + ir2[0] + 1)]


def _wigner_nj(irreps_list, filter_out=None):
    """Recursive coupling of len(irreps_list) copies (_mace_cg.py:39-115); irreps are (l, p), mul 1."""
    if len(irreps_list) == 1:
        irreps = irreps_list[0]
        dim = sum(2 * l + 1 for l, _ in irreps)
        e = np.eye(dim)
        ret, i = [], 0
        for ir in irreps:
            d = 2 * ir[0] + 1
            ret.append((ir, e[i:i + d]))
            i += d
        return ret if filter_out is None else [r for r in ret if r[0] in filter_out]
    *left_list, right = irreps_list
    dims_left = [sum(2 * l + 1 for l, _ in irr) for irr in left_list]
    dim_right = sum(2 * l + 1 for l, _ in right)
    ret = []
    for ir_left, c_left in _wigner_nj(left_list):
        i = 0
        for ir in right:
            for ir_out in _mul(ir_left, ir):
                if filter_out is not None and ir_out not in filter_out:
                    continue
                c = wigner_3j(ir_out[0], ir_left[0], ir[0]) * math.sqrt(2 * ir_out[0] + 1)
                c = np.einsum("jk,ijl->ikl", c_left.reshape(c_left.shape[0], -1), c)
                c = c.reshape(2 * ir_out[0] + 1, *dims_left, 2 * ir[0] + 1)
                e = np.zeros((2 * ir_out[0] + 1, *dims_left, dim_right))
                e[..., i:i + 2 * ir[0] + 1] = c
                ret.append((ir_out, e))
            i += 2 * ir[0] + 1
    return sorted(ret, key=lambda r: r[0])


@lru_cache(maxsize=None)
def u_matrix(lmax, l_out, nu):
    irreps = [(l, 1 if l % 2 == 0 else -1) for l in range(lmax + 1)]
    target = (l_out, 1 if l_out % 2 == 0 else -1)
    rows = [e for ir, e in _wigner_nj([irreps] * nu, filter_out=[target])]
    dim = (lmax + 1) ** 2
    if not rows:
        return np.zeros(([2 * l_out + 1] if l_out else []) + [dim] * nu + [0])
    U = np.stack(rows, -1)
    return U[0] if l_out == 0 else U


@lru_cache(maxsize=None)
def bridge_q_fixture():
    d = json.load(open(_Q_FIXTURE))
    return np.array(d["row_major"]).reshape(25, 25)


def q_block(l):
    Q = bridge_q_fixture()
    o = l * l
    return Q[o:o + 2 * l + 1, o:o + 2 * l + 1]


@lru_cache(maxsize=None)
def u_ictc(lmax, l_out, nu):
    """U folded into the ICTC basis with the fixture Q (symmetric_contraction.py:50-96)."""
    U = u_matrix(lmax, l_out, nu)
    dim = (lmax + 1) ** 2
    qin = np.zeros((dim, dim))
    for l in range(lmax + 1):
        qin[l * l:(l + 1) ** 2, l * l:(l + 1) ** 2] = q_block(l)
    letters = "abcdefgh"
    if l_out == 0:
        spec = ",".join(f"{letters[k]}{'ijk'[k]}" for k in range(nu)) + "," + "ijk"[:nu] + "p->" + letters[:nu] + "p"
        return np.einsum(spec, *([qin] * nu), U, optimize="optimal")
    spec = "ro," + ",".join(f"{letters[k]}{'ijk'[k]}" for k in range(nu)) + ",o" + "ijk"[:nu] + "p->r" + letters[:nu] + "p"
    return np.einsum(spec, q_block(l_out), *([qin] * nu), U, optimize="optimal")


def contraction(x, species, weights, lmax, l_out, corr):
    """One output irrep (_mace_symmetric_contraction.py:298-355).

    x [N, C, dim] (ICTC basis), species [N] int64, weights[nu] [S, P_nu, C] for nu = 1..corr.
    Returns [N, C * (2 l_out + 1)] (channel-major, as the reference reshapes).

    The reference selects each node's weights (index_select by species) and
    runs the Horner recursion out = ((c3 x + c2) x + c1) x on per-node
    coefficients c_nu = U_nu . W_nu[s_n].  The same recursion here runs per
    species on that species' nodes, so the coefficient tensors are formed once
    per species instead of once per node (identical arithmetic per node).
    """
    N, C = x.shape[0], x.shape[1]
    U = {nu: torch.tensor(u_ictc(lmax, l_out, nu), dtype=x.dtype) for nu in range(1, corr + 1)}

    def coeff(nu, s):
        W = weights[nu][s]                                             # [P, C]
        if l_out == 0:
            return torch.einsum("...p,pc->c...", U[nu], W)
        return torch.einsum("m...p,pc->cm...", U[nu], W)

    out = x.new_zeros(N, C * (2 * l_out + 1))
    for s in torch.unique(species).tolist():
        idx = torch.nonzero(species == s).flatten()
        xs = x.index_select(0, idx)
        o = torch.einsum("c...i,nci->nc...", coeff(corr, s), xs)
        for nu in range(corr - 1, 0, -1):
            o = o + coeff(nu, s)
            o = torch.einsum("nc...i,nci->nc...", o, xs)
        out = out.index_copy(0, idx, o.reshape(o.shape[0], -1))
    return out


def symmetric_contraction(x, species, weights_by_L, lmax, target_lmax, corr):
    """Concatenation over output degrees 0..target_lmax; weights_by_L[L][nu] [S, P, C]."""
    return torch.cat([contraction(x, species, weights_by_L[L], lmax, L, corr) for L in range(target_lmax + 1)], -1)
