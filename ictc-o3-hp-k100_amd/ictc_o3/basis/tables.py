"""Constant tables of the ICTC angular algebra (host side, float64).

Everything the kernels need is a closed-form function of the frozen ICTC
harmonic basis ``B_l`` (reference: ictc_o3/basis/ictd_irreps.py:676-720, frozen
bytes verified by SHA-256 against ictd_irreps.py:659-673):

* Gaussian Gram on Sym^L monomials      (ictd_irreps.py:641-655)
* direction harmonics Y_l = s_l t(n) G_l B_l  (ictd_irreps.py:939-985, 1153-1208)
* coupling tensors C[m1,m2,m3]          (ictd_irreps.py:1264-1304)
* component / element normalisation     (ictd_irreps.py:116-157)
* natural-parity path order and path-preserving output offsets
  (operators.py:206-207, ictd_irreps.py:2335-2357, 2692-2705)

The coupling tensor is computed here from Schur's lemma instead of the
reference's least-squares solve: the r^{2k}-lifted degree-l3 harmonics span
one irreducible block of Sym^L, and the rotation-invariant Gram restricted to
it is a multiple of the identity, V^T G V = lambda I.  The projector then
reduces to V^T G / lambda, which is what ``coupling`` evaluates.
"""
from __future__ import annotations

import hashlib
import math
import os
from functools import lru_cache
from typing import Dict, List, Tuple

import numpy as np

_DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data", "harmonic_basis_v1.npz")

# ictc_o3/basis/ictd_irreps.py:659-673 (float64 little-endian bytes of each B_l)
BASIS_SHA256 = {
    0: "6c3c396ed6b5c36dcae172271f462051b1266b851e92df3deea8ac65478fd712",
    1: "1332df685c45a61a0ac008a6a653295b8c5655361c1d34b6304b22ec40235fb8",
    2: "0881fbfd2a1866b76334d823d216ec74773a91a5f77234c45bb956838df7c315",
    3: "a7440553d51231cc044287b305d35cb5cafc59f77d7528d8189956c51a52a9e0",
    4: "f89f4b7f49ed9be8cc7fbbcec5e1a8947442c612d239bd42ce36180c6c644225",
    5: "8cce9bfb0a710f2c19d50ca3bcf6a79593697b5bd129085f10422066c2030ea8",
    6: "01cc08fe54c00daaff6899a86c923b62433f1691b7f283b95643c7be78ce9a96",
    7: "bde0ef7cf352a8cc83b4df959405616a390d270cf0b10bd93eed01da80e1a531",
    8: "85cdd2180f8078d9016110556076bf0464d12985ef079f51fee6c8f2641acf28",
    9: "190d6891295881dd5db122b80442a8feea21d0d716c6ff97faddcb0720509c6b",
    10: "fed2be677a84dc357b0e9b27e14b5bbc4c8a110520f44e536e7bc11365d70586",
    11: "4708bb0367de5a1c0d8d6bb01de80cb1a9a84ce6e128bc1913fecceabdf834ec",
    12: "761c7af5c246722d57a910b32ffe82741ac39326d6cba627be7db3b14d4ab689",
}

# Coefficients below this magnitude are structural zeros (bond_projection.py:63-65).
ZERO = 1e-12


def monomials(L: int) -> List[Tuple[int, int, int]]:
    """Exponents (a, b, c) of x^a y^b z^c, a outer then b (ictd_fast.py:41-48)."""
    return [(a, b, L - a - b) for a in range(L + 1) for b in range(L - a + 1)]


@lru_cache(maxsize=None)
def basis(l: int) -> np.ndarray:
    """Frozen B_l with its SHA-256 verified; raises on any mismatch."""
    with np.load(_DATA) as z:
        B = np.ascontiguousarray(z[f"l{l}"], dtype="<f8")
    if hashlib.sha256(B.tobytes()).hexdigest() != BASIS_SHA256[l]:
        raise RuntimeError(f"ICTC harmonic basis l={l} failed its SHA-256 check")
    return B


def _moment(n: int) -> float:
    if n % 2:
        return 0.0
    out = 1
    for k in range(n - 1, 0, -2):
        out *= k
    return float(out)


@lru_cache(maxsize=None)
def gram(L: int) -> np.ndarray:
    m = monomials(L)
    return np.array([[_moment(a + p) * _moment(b + q) * _moment(c + r) for (p, q, r) in m]
                     for (a, b, c) in m])


def _lift(l: int, k: int) -> np.ndarray:
    """Coefficients of (x^2+y^2+z^2)^k * monomial, as a Sym^l -> Sym^{l+2k} matrix."""
    src, dst = monomials(l), monomials(l + 2 * k)
    row = {t: i for i, t in enumerate(dst)}
    M = np.zeros((len(dst), len(src)))
    for j, (a, b, c) in enumerate(src):
        for u in range(k + 1):
            for v in range(k - u + 1):
                w = k - u - v
                M[row[(a + 2 * u, b + 2 * v, c + 2 * w)], j] += (
                    math.factorial(k) / (math.factorial(u) * math.factorial(v) * math.factorial(w)))
    return M


@lru_cache(maxsize=None)
def coupling(l1: int, l2: int, l3: int) -> np.ndarray:
    """Raw C[m1, m2, m3]: harmonic coordinates of the product polynomial's l3 block."""
    shape = (2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1)
    if not (abs(l1 - l2) <= l3 <= l1 + l2) or (l1 + l2 + l3) % 2:
        return np.zeros(shape)
    L = l1 + l2
    V = _lift(l3, (L - l3) // 2) @ basis(l3)
    G = gram(L)
    lam = float(np.trace(V.T @ G @ V)) / (2 * l3 + 1)
    m1, m2, mL = monomials(l1), monomials(l2), {t: i for i, t in enumerate(monomials(L))}
    B1, B2 = basis(l1), basis(l2)
    # product polynomial coefficients for every (m1, m2) pair
    prod = np.zeros((len(mL), shape[0], shape[1]))
    for i, a in enumerate(m1):
        for j, b in enumerate(m2):
            prod[mL[(a[0] + b[0], a[1] + b[1], a[2] + b[2])]] += np.outer(B1[i], B2[j])
    C = np.einsum("dk,de,eij->ijk", V, G, prod) / lam
    return C


def coupling_component(l1: int, l2: int, l3: int) -> np.ndarray:
    C = coupling(l1, l2, l3)
    n = float(np.sqrt((C * C).sum()))
    return C * (math.sqrt(2 * l3 + 1) / n) if n > 1e-30 else C


# ---------------------------------------------------------------------------
# Direction harmonics as explicit polynomials
# ---------------------------------------------------------------------------


def _sphere_moment(a: int, b: int, c: int) -> float:
    if a % 2 or b % 2 or c % 2:
        return 0.0

    def df(n):
        out = 1
        for k in range(n, 0, -2):
            out *= k
        return out
    p, q, r = a // 2, b // 2, c // 2
    return df(2 * p - 1) * df(2 * q - 1) * df(2 * r - 1) / df(2 * (p + q + r) + 1)


@lru_cache(maxsize=None)
def harmonic_polynomials(l: int) -> Tuple[List[Tuple[int, int, int]], np.ndarray]:
    """Y_l[m] = sum_k coef[k, m] x^a_k y^b_k z^c_k, component-normalised on the sphere."""
    mono = monomials(l)
    if l == 0:
        return mono, np.ones((1, 1))
    multi = np.array([math.factorial(l) / (math.factorial(a) * math.factorial(b) * math.factorial(c))
                      for a, b, c in mono])
    P = gram(l) @ basis(l)
    S = np.array([[_sphere_moment(a + p, b + q, c + r) for (p, q, r) in mono] for (a, b, c) in mono])
    S = S * np.outer(multi, multi)
    mean_square = float(np.trace(P.T @ S @ P)) / (2 * l + 1)
    scale = 1.0 / math.sqrt(max(mean_square, 1e-30))
    return mono, multi[:, None] * P * scale


# ---------------------------------------------------------------------------
# Path tables
# ---------------------------------------------------------------------------


def natural_paths(input_lmax: int, edge_lmax: int, output_lmax: int) -> List[Tuple[int, int, int]]:
    """Natural-parity triangle paths in gate order (operators.py:206-207)."""
    return [(i, j, k) for i in range(input_lmax + 1) for j in range(edge_lmax + 1)
            for k in range(output_lmax + 1) if abs(i - j) <= k <= i + j and (i + j + k) % 2 == 0]


class PathTable:
    """Per-path scaled coupling, output placement and packed offsets.

    Output layout (packed ir_mul): degree-major; within degree l the path slots
    in offset order, each slot ``[2l+1, C]`` (operators.py:296-308).
    """

    def __init__(self, paths, lmax_out=None):
        self.paths = [tuple(int(v) for v in p) for p in paths]
        self.counts: Dict[int, int] = {}
        for _, _, l3 in self.paths:
            self.counts[l3] = self.counts.get(l3, 0) + 1
        self.lmax_out = max(l3 for *_, l3 in self.paths) if lmax_out is None else lmax_out
        self.input_lmax = max(p[0] for p in self.paths)
        self.edge_lmax = max(p[1] for p in self.paths)
        seen: Dict[int, int] = {}
        self.slot = []
        for (_, _, l3) in self.paths:
            self.slot.append(seen.get(l3, 0))
            seen[l3] = seen.get(l3, 0) + 1
        # components (units of C) before each output degree
        self.degree_offset, off = {}, 0
        for l in range(self.lmax_out + 1):
            self.degree_offset[l] = off
            off += self.counts.get(l, 0) * (2 * l + 1)
        self.out_components = off
        self.coef = [coupling_component(*p) / math.sqrt(self.counts[p[2]]) for p in self.paths]

    def out_component(self, p: int, m3: int) -> int:
        l3 = self.paths[p][2]
        return self.degree_offset[l3] + self.slot[p] * (2 * l3 + 1) + m3

    def nonzeros(self, p: int):
        """[(m1, m2, m3, value)] of path p's scaled coupling."""
        C = self.coef[p]
        return [(i, j, k, float(C[i, j, k])) for i in range(C.shape[0]) for j in range(C.shape[1])
                for k in range(C.shape[2]) if abs(C[i, j, k]) > ZERO]
