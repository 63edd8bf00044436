"""CPU float64 oracle for the ICTC-O3 equivariant hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use
it, as the checker.  Every function restates the reference algorithm in plain
numpy / torch-float64 and cites the reference file:line it follows
(paths relative to the reference repository root).

Pinning (what checks each function, beyond retyping):
  basis            SHA-256 of the frozen bytes (ictd_irreps.py:659-673),
                   harmonicity (Laplacian kernel), Gaussian orthonormality.
  projectors / CG  equivariance under random rotations, closed form l=0 paths
                   (identity scaled by sqrt((2l+1))/||I||), Frobenius norm
                   sqrt(2 l3 + 1) after component normalisation.
  harmonics        |Y_l|^2 = 2l+1 on unit vectors, parity (-1)^l, Y_0 = 1,
                   rotation covariance with D_l from the CG-free fit.
  edge TP          brute-force dense einsum on tiny inputs, multilinearity,
                   equivariance, element normalisation 1/sqrt(count_l).
  message          index_add of the edge TP; edge-permutation invariance.
  derivatives      torch.autograd on the float64 restatement, pinned with
                   gradcheck / gradgradcheck (finite differences).
"""
from __future__ import annotations

import math
import os
from functools import lru_cache
from typing import Dict, List, Tuple

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_BASIS_NPZ = os.path.join(_HERE, "..", "ictc-o3-hp-k100_amd", "ictc_o3", "basis", "data",
                          "harmonic_basis_v1.npz")

# ---------------------------------------------------------------------------
# Monomial bookkeeping  (ictc_o3/basis/ictd_fast.py:41-48, 87-114, 240-266)
# ---------------------------------------------------------------------------


def counts_list(L: int) -> List[Tuple[int, int, int]]:
    """(a,b,c), a+b+c=L, a outer then b (ictd_fast.py:41-48)."""
    return [(a, b, L - a - b) for a in range(L + 1) for b in range(L - a + 1)]


def sym_dim(L: int) -> int:
    return (L + 2) * (L + 1) // 2


def laplacian_matrix(L: int) -> np.ndarray:
    """Laplacian Sym^L -> Sym^{L-2} on monomial coefficients (ictd_fast.py:87-114)."""
    src, dst = counts_list(L), counts_list(L - 2)
    j = {t: i for i, t in enumerate(dst)}
    D = np.zeros((len(dst), len(src)))
    for col, (a, b, c) in enumerate(src):
        if a >= 2:
            D[j[(a - 2, b, c)], col] += a * (a - 1)
        if b >= 2:
            D[j[(a, b - 2, c)], col] += b * (b - 1)
        if c >= 2:
            D[j[(a, b, c - 2)], col] += c * (c - 1)
    return D


def r2k_lift(l: int, k: int) -> np.ndarray:
    """Multiplication by (x^2+y^2+z^2)^k, Sym^l -> Sym^{l+2k} (ictd_fast.py:240-266)."""
    src = counts_list(l)
    if k == 0:
        return np.eye(len(src))
    dst = counts_list(l + 2 * k)
    j = {t: i for i, t in enumerate(dst)}
    M = np.zeros((len(dst), len(src)))
    for col, (a, b, c) in enumerate(src):
        for u in range(k + 1):
            for v in range(k - u + 1):
                w = k - u - v
                coef = math.factorial(k) / (math.factorial(u) * math.factorial(v) * math.factorial(w))
                M[j[(a + 2 * u, b + 2 * v, c + 2 * w)], col] += coef
    return M


def _dfact(n: int) -> int:
    out = 1
    for k in range(n, 0, -2):
        out *= k
    return out


def gaussian_moment(n: int) -> float:
    """E[x^n], x ~ N(0,1) (ictd_irreps.py:614-618)."""
    return 0.0 if n % 2 else float(_dfact(n - 1))


def sphere_moment(a: int, b: int, c: int) -> float:
    """E[x^a y^b z^c] on the unit sphere (ictd_irreps.py:621-638)."""
    if a % 2 or b % 2 or c % 2:
        return 0.0
    p, q, r = a // 2, b // 2, c // 2
    return _dfact(2 * p - 1) * _dfact(2 * q - 1) * _dfact(2 * r - 1) / _dfact(2 * (p + q + r) + 1)


@lru_cache(maxsize=None)
def gram_gaussian(L: int) -> np.ndarray:
    """Rotation-invariant Gram on Sym^L monomials (ictd_irreps.py:641-655)."""
    cl = counts_list(L)
    G = np.zeros((len(cl), len(cl)))
    for i, (a, b, c) in enumerate(cl):
        for j, (a2, b2, c2) in enumerate(cl):
            G[i, j] = gaussian_moment(a + a2) * gaussian_moment(b + b2) * gaussian_moment(c + c2)
    return G


@lru_cache(maxsize=None)
def _basis_table():
    return np.load(_BASIS_NPZ)


def harmonic_basis(l: int) -> np.ndarray:
    """Frozen B_l [sym_dim(l), 2l+1] (ictd_irreps.py:676-720)."""
    return np.array(_basis_table()[f"l{l}"])


@lru_cache(maxsize=None)
def projector(L: int, l: int) -> np.ndarray:
    """P_{L->l} = (V^T G V)^{-1} V^T G with V = lift(l, k) B_l (ictd_irreps.py:844-869)."""
    k = (L - l) // 2
    V = r2k_lift(l, k) @ harmonic_basis(l)
    G = gram_gaussian(L)
    return np.linalg.solve(V.T @ G @ V, V.T @ G)


def poly_mult_matrix(l1: int, l2: int) -> np.ndarray:
    """Monomial product map Sym^l1 x Sym^l2 -> Sym^(l1+l2) (ictd_irreps.py:1245-1261)."""
    c1, c2, cL = counts_list(l1), counts_list(l2), counts_list(l1 + l2)
    idx = {t: i for i, t in enumerate(cL)}
    M = np.zeros((len(cL), len(c1) * len(c2)))
    for i, a in enumerate(c1):
        for j, b in enumerate(c2):
            M[idx[(a[0] + b[0], a[1] + b[1], a[2] + b[2])], i * len(c2) + j] = 1.0
    return M


@lru_cache(maxsize=None)
def cg_tensor(l1: int, l2: int, l3: int) -> np.ndarray:
    """Raw coupling C[m1,m2,m3] in the ICTC basis (ictd_irreps.py:1264-1304)."""
    if not (abs(l1 - l2) <= l3 <= l1 + l2) or (l1 + l2 + l3) % 2:
        return np.zeros((2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1))
    B1, B2 = harmonic_basis(l1), harmonic_basis(l2)
    outer = np.einsum("im,jn->ijmn", B1, B2).reshape(B1.shape[0] * B2.shape[0], -1)
    c3 = projector(l1 + l2, l3) @ (poly_mult_matrix(l1, l2) @ outer)
    return c3.T.reshape(2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1)


def cg_component(l1: int, l2: int, l3: int) -> np.ndarray:
    """Component normalisation C * sqrt(2 l3 + 1) / ||C||_F (ictd_irreps.py:151-157)."""
    C = cg_tensor(l1, l2, l3)
    n = np.linalg.norm(C)
    return C * (math.sqrt(2 * l3 + 1) / n) if n > 1e-30 else C


# ---------------------------------------------------------------------------
# Direction harmonics  (ictd_irreps.py:939-985, 1153-1208)
# ---------------------------------------------------------------------------


@lru_cache(maxsize=None)
def direction_projection(l: int) -> np.ndarray:
    """G_l B_l (ictd_irreps.py:939-949)."""
    if l == 0:
        return np.ones((1, 1))
    return gram_gaussian(l) @ harmonic_basis(l)


def multinomials(l: int) -> np.ndarray:
    return np.array([math.factorial(l) / (math.factorial(a) * math.factorial(b) * math.factorial(c))
                     for a, b, c in counts_list(l)])


@lru_cache(maxsize=None)
def direction_scale(l: int) -> float:
    """Component (RMS 1 on the sphere) scale (ictd_irreps.py:952-985)."""
    if l == 0:
        return 1.0
    cl, co = counts_list(l), multinomials(l)
    S = np.zeros((len(cl), len(cl)))
    for i, (a, b, c) in enumerate(cl):
        for j, (a2, b2, c2) in enumerate(cl):
            S[i, j] = co[i] * co[j] * sphere_moment(a + a2, b + b2, c + c2)
    P = direction_projection(l)
    ms = np.trace(P.T @ S @ P) / (2 * l + 1)
    return float(1.0 / math.sqrt(max(ms, 1e-30)))


def direction_harmonics(n: torch.Tensor, lmax: int) -> List[torch.Tensor]:
    """Y_l(n) = (t_l(n) G_l B_l) s_l, list over l (ictd_irreps.py:1153-1208).  Differentiable."""
    out = [torch.ones(*n.shape[:-1], 1, dtype=n.dtype, device=n.device)]
    for l in range(1, lmax + 1):
        cl = counts_list(l)
        t = torch.stack([n[..., 0] ** a * n[..., 1] ** b * n[..., 2] ** c for a, b, c in cl], -1)
        t = t * torch.tensor(multinomials(l), dtype=n.dtype)
        P = torch.tensor(direction_projection(l), dtype=n.dtype)
        out.append((t @ P) * direction_scale(l))
    return out


# ---------------------------------------------------------------------------
# Path tables  (operators.py:206-207, ictd_irreps.py:116-148, 2335-2357, 2681-2711)
# ---------------------------------------------------------------------------


def natural_paths(input_lmax: int, edge_lmax: int, output_lmax: int) -> List[Tuple[int, int, int]]:
    """Natural-parity triangle paths, l1 outer, l2, l3 ascending (operators.py:206-207)."""
    return [(i, j, k) for i in range(input_lmax + 1) for j in range(edge_lmax + 1)
            for k in range(output_lmax + 1) if abs(i - j) <= k <= i + j and (i + j + k) % 2 == 0]


def path_tables(paths):
    """(scaled CG list, path offsets, counts by l3).

    Element path normalisation 1/sqrt(#paths sharing l3) with num_elements=1
    (ictd_irreps.py:116-148, 2359-2364); offsets are the running count of
    earlier paths with the same l3 in group order (ictd_irreps.py:2692-2705).
    """
    count: Dict[int, int] = {}
    for _, _, l3 in paths:
        count[l3] = count.get(l3, 0) + 1
    cgs, offsets, seen = [], [], {}
    for (l1, l2, l3) in paths:
        cgs.append(cg_component(l1, l2, l3) / math.sqrt(count[l3]))
        offsets.append(seen.get(l3, 0))
        seen[l3] = seen.get(l3, 0) + 1
    return cgs, offsets, count


# ---------------------------------------------------------------------------
# Edge TP  (ictd_irreps.py:2849-2971) and packed layouts (operators.py:283-308)
# ---------------------------------------------------------------------------


def edge_tp_blocks(x: Dict[int, torch.Tensor], Y: Dict[int, torch.Tensor], gates: torch.Tensor,
                   paths, weight: torch.Tensor | None = None, lmax_out: int | None = None):
    """Path-preserving edge TP.

    x[l1]: [E, C, 2l1+1]; Y[l2]: [E, 2l2+1]; gates [E, P, C]; weight [P, C] (default ones).
    Returns {l3: [E, count_l3 * C, 2l3+1]} with path p at channel block offset_p*C
    (ictd_irreps.py:2849-2928: y = (a (x) b) U, seg * w[p] * g[:, p]).
    """
    cgs, offsets, count = path_tables(paths)
    E, C = gates.shape[0], gates.shape[2]
    lmax_out = max(l3 for _, _, l3 in paths) if lmax_out is None else lmax_out
    blocks: Dict[int, list] = {l: [None] * count.get(l, 0) for l in range(lmax_out + 1)}
    for p, (l1, l2, l3) in enumerate(paths):
        cg = torch.tensor(cgs[p], dtype=gates.dtype)
        seg = torch.einsum("ecm,emk->eck", x[l1], torch.einsum("en,mnk->emk", Y[l2], cg))
        if weight is not None:
            seg = seg * weight[p].view(1, C, 1)
        seg = seg * gates[:, p, :].unsqueeze(-1)
        blocks[l3][offsets[p]] = seg          # channel block offsets[p]*C .. +C of out[l3]
    # offsets are the running count per l3, so the blocks tile out[l3] in order
    return {l: (torch.cat(b, 1) if b else torch.zeros(E, 0, 2 * l + 1, dtype=gates.dtype)) for l, b in blocks.items()}


def pack_ir_mul(blocks: Dict[int, torch.Tensor], lmax: int) -> torch.Tensor:
    """{l: [R, C, 2l+1]} -> [R, sum_l (2l+1) C] with [2l+1, C] per degree (operators.py:283-294)."""
    return torch.cat([blocks[l].transpose(1, 2).reshape(blocks[l].shape[0], -1) for l in range(lmax + 1)], -1)


def unpack_ir_mul(flat: torch.Tensor, C: int, lmax: int) -> Dict[int, torch.Tensor]:
    out, off = {}, 0
    for l in range(lmax + 1):
        w = (2 * l + 1) * C
        out[l] = flat[:, off:off + w].reshape(-1, 2 * l + 1, C).transpose(1, 2)
        off += w
    return out


def pack_output(out_blocks: Dict[int, torch.Tensor], counts: Dict[int, int], C: int) -> torch.Tensor:
    """{l: [R, count C, 2l+1]} -> [R, odim], each path slot [2l+1, C] (operators.py:296-308)."""
    parts = []
    for l in sorted(out_blocks):
        k = counts.get(l, 0)
        if k == 0:
            continue
        v = out_blocks[l]
        parts.append(v.reshape(v.shape[0], k, C, 2 * l + 1).transpose(2, 3).reshape(v.shape[0], -1))
    return torch.cat(parts, -1)


def harmonics_packed(Y: List[torch.Tensor]) -> torch.Tensor:
    return torch.cat(Y, -1)


def edge_tp_packed(features: torch.Tensor, harmonics: torch.Tensor, gates: torch.Tensor,
                   input_lmax: int, edge_lmax: int, output_lmax: int, C: int) -> torch.Tensor:
    """EdgeTensorProduct.forward semantics on packed ir_mul buffers (operators.py:310-340)."""
    paths = natural_paths(input_lmax, edge_lmax, output_lmax)
    E = features.shape[0]
    x = unpack_ir_mul(features, C, input_lmax)
    Y = {l: harmonics[:, l * l:(l + 1) ** 2] for l in range(edge_lmax + 1)}
    out = edge_tp_blocks(x, Y, gates.reshape(E, len(paths), C), paths)
    _, _, counts = path_tables(paths)
    return pack_output(out, counts, C)


def message_packed(features: torch.Tensor, harmonics: torch.Tensor, gates: torch.Tensor,
                   src: torch.Tensor, dst: torch.Tensor, mask: torch.Tensor | None,
                   input_lmax: int, edge_lmax: int, output_lmax: int, C: int) -> torch.Tensor:
    """PackedGraphMessage: gather x[src], edge TP, * mask, index_add into dst.

    fused_message.py:492-510 (_native) and operators.py:382-409.
    """
    edge = edge_tp_packed(features[src], harmonics, gates, input_lmax, edge_lmax, output_lmax, C)
    if mask is not None:
        edge = edge * mask.reshape(-1, 1)
    out = torch.zeros(features.shape[0], edge.shape[1], dtype=edge.dtype)
    return out.index_add(0, dst, edge)
