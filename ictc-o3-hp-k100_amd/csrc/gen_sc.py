"""Emit ``generated/ictc_sc.h``: straight-line symmetric-contraction polynomials.

The correlation-nu symmetric contraction of the reference
(ictc_o3/ops/_mace_symmetric_contraction.py:298-355, U from _mace_cg.py:118-190
with the ICTC bridge folded in, symmetric_contraction.py:50-96) is, per node n,
channel c and output component (L, m),

    out[L, m] = sum_nu sum_p W_nu^L[s_n, p, c] * sum_{i1..inu} U_nu^L[m, i1..inu, p] x_i1 ... x_inu .

Only the symmetric part of U in (i1..inu) contributes, so each (L, m) output
is a sparse polynomial in the NX = (LI+1)^2 input components whose
coefficients are linear in the per-species weights.  For every supported
(LI, LT, CORR) this script emits ``Sc<LI, LT, CORR>`` with device functions
working on per-lane registers (one lane = one channel):

  fwd     o[k]   = sum_mono mono(x) * (sum_{nu,p} coef * W)
  dx      d[i]   = d/dx_i of sum_k go[k] o[k]
  dw      dw[q]  = sum_k go[k] * d o[k] / d W_q           (q enumerates (L, nu, p))
  jvp     t[k]   = sum_i h_i d o[k] / d x_i
  hvp     d[i]   = sum_j h_j d^2 (go . o) / dx_i dx_j
  dwjvp   dw[q]  = sum_k go[k] * sum_i h_i d^2 o[k] / dW_q dx_i

Weights are read through a ``ScWeights`` table (one [S, P, C] array per (L, nu)).
"""
from __future__ import annotations

import itertools
import os
import sys

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(_HERE))

from ictc_o3.basis import e3nn_basis  # noqa: E402

ZERO = 1e-11
# (LI, LT) pairs compiled; every correlation 1..3.
CONFIGS = [(li, lt) for li in range(3) for lt in range(li + 1)] + [(3, 0), (3, 1), (3, 2)]


def f(v):
    return repr(float(v)) + "f"


def polynomial(li, lt, corr):
    """terms[k][mono] = [(L, nu, p, coef)] with k the packed output index, mono a sorted tuple."""
    nx = (li + 1) ** 2
    outs = []
    for L in range(lt + 1):
        for m in range(2 * L + 1):
            outs.append((L, m))
    terms = [dict() for _ in outs]
    counts = {}
    for L in range(lt + 1):
        for nu in range(1, corr + 1):
            U = e3nn_basis.mace_u_ictc(li, L, nu)
            if L == 0:
                U = U[None]
            P = U.shape[-1]
            counts[(L, nu)] = P
            for p in range(P):
                for m in range(2 * L + 1):
                    T = U[m, ..., p]
                    acc = {}
                    for idx in itertools.product(range(nx), repeat=nu):
                        v = T[idx]
                        if abs(v) > 1e-14:
                            key = tuple(sorted(idx))
                            acc[key] = acc.get(key, 0.0) + v
                    k = outs.index((L, m))
                    for key, v in acc.items():
                        if abs(v) > ZERO:
                            terms[k].setdefault(key, []).append((L, nu, p, v))
    return outs, terms, counts


def _weight_names(counts):
    q = []
    for (L, nu), P in sorted(counts.items()):
        for p in range(P):
            q.append((L, nu, p))
    return q


def _combo(entries):
    return " + ".join(f"{f(v)} * w{L}_{nu}_{p}" for L, nu, p, v in entries)


def _mono_expr(key):
    return " * ".join(f"x[{i}]" for i in key) if key else "1.f"


def _deriv(key):
    """[(i, multiplicity, remaining key)] of d/dx_i of the monomial."""
    out = []
    for i in sorted(set(key)):
        rest = list(key)
        rest.remove(i)
        out.append((i, key.count(i), tuple(rest)))
    return out


DW_BLOCK = 32   # weights per weight-gradient wave (kDwBlock in sc_kernels.h)


def sc_struct(li, lt, corr):
    outs, terms, counts = polynomial(li, lt, corr)
    nx, no = (li + 1) ** 2, len(outs)
    wq = _weight_names(counts)
    nq = len(wq)
    qindex = {w: i for i, w in enumerate(wq)}
    L = [f"template <> struct Sc<{li}, {lt}, {corr}> {{",
         f"  static constexpr int NX = {nx}, NO = {no}, NW = {nq};"]
    # weight counts table
    rows = []
    for Lo in range(4):
        rows.append("{" + ", ".join(str(counts.get((Lo, nu), 0)) for nu in (1, 2, 3)) + "}")
    L.append(f"  static constexpr int P[4][3] = {{{', '.join(rows)}}};")
    nterms = sum(len(e) for t in terms for e in t.values())
    L.append(f"  static constexpr int TERMS = {nterms};")

    def load_weights():
        # species row of each weight block (wave-uniform) + the lane's byte offset: SGPR-base loads
        s = ["    const int64_t sb = s;", "    const uint32_t off = sc_lane_offset(c);"]
        for (Lo, nu) in sorted({(Lo, nu) for (Lo, nu, p) in wq}):
            P = counts[(Lo, nu)]
            s.append(f"    const float* __restrict__ wb{Lo}_{nu} = t.w[{Lo}][{nu - 1}] + sb * {P} * C;")
        for (Lo, nu, p) in wq:
            s.append(f"    const float w{Lo}_{nu}_{p} = sc_load(wb{Lo}_{nu} + {p} * C, off);")
        return s

    # forward
    L.append("  __device__ __forceinline__ static void fwd(const float* __restrict__ x, const ScWeights& t, int s,"
             " int C, int c, float* __restrict__ o) {")
    L += load_weights()
    for k in range(no):
        expr = " + ".join(f"({_mono_expr(key)}) * ({_combo(e)})" for key, e in terms[k].items()) or "0.f"
        L.append(f"    o[{k}] = {expr};")
    L.append("  }")
    # dx: gradient of sum_k go[k] o[k]
    L.append("  __device__ __forceinline__ static void dx(const float* __restrict__ x, const ScWeights& t, int s,"
             " int C, int c, const float* __restrict__ go, float* __restrict__ d) {")
    L += load_weights()
    L.append(f"    float a[{nx}];")
    L.append(f"    for (int i = 0; i < {nx}; ++i) a[i] = 0.f;")
    mono_all = {}
    for k in range(no):
        for key, e in terms[k].items():
            mono_all.setdefault(key, []).append((k, e))
    for key, lst in mono_all.items():
        if not key:
            continue
        g = " + ".join(f"go[{k}] * ({_combo(e)})" for k, e in lst)
        L.append(f"    {{ const float g = {g};")
        for i, mult, rest in _deriv(key):
            L.append(f"      a[{i}] = fmaf(g, {float(mult)}f * ({_mono_expr(rest)}), a[{i}]);")
        L.append("    }")
    L.append(f"    for (int i = 0; i < {nx}; ++i) d[i] = a[i];")
    L.append("  }")
    # dw: per weight q, sum_k go[k] * coef * mono; emitted in blocks of DW_BLOCK weights
    # (dwb<B> accumulates weights B*DW_BLOCK ...) so one wave holds one block's accumulators.
    per_q = {q: [] for q in range(nq)}
    for k in range(no):
        for key, e in terms[k].items():
            for (Lo, nu, p, v) in e:
                per_q[qindex[(Lo, nu, p)]].append((k, key, v))
    nb = max(1, (nq + DW_BLOCK - 1) // DW_BLOCK)

    def by_monomial(b):
        """{mono key: {local q: [(k, coef)]}} for the weights of block b, in first-use order."""
        groups = {}
        for q in range(b * DW_BLOCK, min(nq, (b + 1) * DW_BLOCK)):
            for k, key, v in per_q[q]:
                groups.setdefault(key, {}).setdefault(q - b * DW_BLOCK, []).append((k, v))
        return groups

    def go_combo(lst):
        return " + ".join(f"{f(v)} * go[{k}]" for k, v in lst)

    # Each monomial is formed once and consumed at once (short live ranges).
    L.append(f"  static constexpr int NB = {nb};")
    L.append("  template <int B>")
    L.append("  __device__ __forceinline__ static void dwb(const float* __restrict__ x, const float* __restrict__ go,"
             " float* __restrict__ acc) {")
    for b in range(nb):
        L.append(f"    {'if' if b == 0 else 'else if'} constexpr (B == {b}) {{")
        for key, qs in by_monomial(b).items():
            L.append(f"      {{ const float m = {_mono_expr(key)};")
            for ql, lst in qs.items():
                L.append(f"        acc[{ql}] = fmaf(m, {go_combo(lst)}, acc[{ql}]);")
            L.append("      }")
        L.append("    }")
    L.append("  }")
    # jvp: directional derivative of o along h
    L.append("  __device__ __forceinline__ static void jvp(const float* __restrict__ x, const ScWeights& t, int s,"
             " int C, int c, const float* __restrict__ h, float* __restrict__ o) {")
    L += load_weights()
    for k in range(no):
        parts = []
        for key, e in terms[k].items():
            dparts = [f"{float(mult)}f * ({_mono_expr(rest)}) * h[{i}]" for i, mult, rest in _deriv(key)]
            if dparts:
                parts.append(f"({' + '.join(dparts)}) * ({_combo(e)})")
        L.append(f"    o[{k}] = {' + '.join(parts) or '0.f'};")
    L.append("  }")
    # hvp: d[i] = sum_j h_j d2(go.o)/dx_i dx_j
    L.append("  __device__ __forceinline__ static void hvp(const float* __restrict__ x, const ScWeights& t, int s,"
             " int C, int c, const float* __restrict__ go, const float* __restrict__ h, float* __restrict__ d) {")
    L += load_weights()
    L.append(f"    float a[{nx}];")
    L.append(f"    for (int i = 0; i < {nx}; ++i) a[i] = 0.f;")
    for key, lst in mono_all.items():
        if len(key) < 2:
            continue
        g = " + ".join(f"go[{k}] * ({_combo(e)})" for k, e in lst)
        L.append(f"    {{ const float g = {g};")
        for i, mi, rest in _deriv(key):
            # d/dx_i of mono = mi * rest ; then directional derivative of rest along h
            inner = [f"{float(mj)}f * ({_mono_expr(r2)}) * h[{j}]" for j, mj, r2 in _deriv(rest)]
            L.append(f"      a[{i}] = fmaf(g, {float(mi)}f * ({' + '.join(inner)}), a[{i}]);")
        L.append("    }")
    L.append(f"    for (int i = 0; i < {nx}; ++i) d[i] = a[i];")
    L.append("  }")
    # dwjvp: dw[q] = sum_k go[k] coef * (d mono . h), in the same weight blocks as dwb
    L.append("  template <int B>")
    L.append("  __device__ __forceinline__ static void dwjvpb(const float* __restrict__ x, const float* __restrict__ go,"
             " const float* __restrict__ h, float* __restrict__ acc) {")
    for b in range(nb):
        L.append(f"    {'if' if b == 0 else 'else if'} constexpr (B == {b}) {{")
        for key, qs in by_monomial(b).items():
            dparts = [f"{float(mult)}f * ({_mono_expr(rest)}) * h[{i}]" for i, mult, rest in _deriv(key)]
            if not dparts:
                continue
            L.append(f"      {{ const float m = {' + '.join(dparts)};")
            for ql, lst in qs.items():
                L.append(f"        acc[{ql}] = fmaf(m, {go_combo(lst)}, acc[{ql}]);")
            L.append("      }")
        L.append("    }")
    L.append("  }")
    # weight slot table: q -> (L, nu-1, p)
    L.append(f"  static constexpr int WQ[{max(nq, 1)}][3] = {{"
             + ", ".join(f"{{{Lo}, {nu - 1}, {p}}}" for Lo, nu, p in wq) + ("" if nq else "{0, 0, 0}") + "};")
    L.append("};")
    return "\n".join(L)


def generate(path):
    parts = ["// Generated by csrc/gen_sc.py from the frozen ICTC basis and the e3nn/MACE coupling. Do not edit.",
             "#pragma once", "#include <stdint.h>", "namespace ictc {",
             "struct ScWeights { const float* w[4][3]; };",
             "// Lane byte offset kept opaque so that its zero extension stays next to each load.",
             "__device__ __forceinline__ uint32_t sc_lane_offset(int c) {",
             "  uint32_t off = (uint32_t)c * 4u;",
             "  asm volatile(\"\" : \"+v\"(off));",
             "  return off;",
             "}",
             "__device__ __forceinline__ float sc_load(const float* __restrict__ row, uint32_t off) {",
             "  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(row) + off);",
             "}",
             "template <int LI, int LT, int CORR> struct Sc;"]
    cfgs = []
    for li, lt in CONFIGS:
        for corr in (1, 2, 3):
            parts.append(sc_struct(li, lt, corr))
            cfgs.append((li, lt, corr))
    parts.append("}  // namespace ictc")
    parts.append("#define ICTC_FOR_EACH_SC(X) " + " ".join(f"X({a},{b},{c})" for a, b, c in cfgs))
    text = "\n".join(parts) + "\n"
    os.makedirs(os.path.dirname(path), exist_ok=True)
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as fh:
            fh.write(text)
    return cfgs


if __name__ == "__main__":
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(_HERE, "generated", "ictc_sc.h")
    print(len(generate(out)), "SC configurations ->", out)
