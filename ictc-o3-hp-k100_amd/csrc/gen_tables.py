"""Emit ``generated/ictc_tables.h``: straight-line CG and harmonic code for gfx950.

Run at build time (``__graft_entry__.build()`` / ``csrc/build.py``).  The
reference JIT-compiles per-shape kernels with CG literals at first call
(ictc_o3/backends/k100/generated_cartesian_message.py:85-291,
native_jit.py:17-62); this build instead emits every qualified shape
(input, edge and output degree <= 3, natural-parity paths) ahead of time, so
there is no cold-start compiler in the product.

For each (LI, LE, LO) the header defines ``Tp<LI,LE,LO>`` with four device
functions operating on per-lane register arrays, indices in the packed
component order (component k of degree l sits at l*l + m):

  fwd   o[k]  += gw[p] * sum C_p[m1,m2,m3] x[m1] y[m2]      (o index: output slot)
  dx    dx[i] += sum_p gw[p] sum C_p y[m2] go[k]
  dy    dy[j] += sum_p gw[p] sum C_p x[m1] go[k]
  dg    dg[p]  = sum_k go[k] sum C_p x[m1] y[m2]
  dydg  dy and dg of the same x in one pass
  dxdydg dx, dy and dg in one pass, factorised through V_p[i][j] = sum_k C go[k]
  dydg_v, dx_v  the same factorisation for dy + dg alone and for dx alone

The sums are grouped so that the lane-varying operand meets the CG literal
first: B_jk = sum_i C x[i] costs one VALU op per nonzero, and the per-edge
harmonics y (wave-uniform, in SGPRs) enter once per (j, k) pair.  dydg
shares each B_jk between the two adjoints.

and ``Sh<L>`` with the component-normalised direction harmonics, their
Jacobian-transpose product (bwd), Jacobian product (jvp) and the
Hessian-vector product of sum_k g_k Y_k (hvp).
"""
from __future__ import annotations

import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(_HERE))

from ictc_o3.basis import tables  # noqa: E402

LMAX = 3
# Scheduling fence after each output slot of the contractions: without it the
# scheduler interleaves the independent B_jk products of many slots and the
# register demand of the degree-3 kernels doubles.
SB = ""


def f(v: float) -> str:
    return repr(float(v)) + "f"


def tp_struct(li, le, lo):
    paths = tables.natural_paths(li, le, lo)
    if not paths:
        return None
    T = tables.PathTable(paths, lmax_out=lo)
    NX, NY, P, NO = (li + 1) ** 2, (le + 1) ** 2, len(paths), T.out_components
    lines = [f"template <> struct Tp<{li}, {le}, {lo}> {{",
             f"  static constexpr int LI = {li}, LE = {le}, LO = {lo};",
             f"  static constexpr int NX = {NX}, NY = {NY}, P = {P}, NO = {NO};"]
    # entries: (p, xi, yj, ok, coef)
    ent = []
    for p, (l1, l2, l3) in enumerate(paths):
        for (m1, m2, m3, v) in T.nonzeros(p):
            ent.append((p, l1 * l1 + m1, l2 * l2 + m2, T.out_component(p, m3), v))
    lines.append(f"  static constexpr int NNZ = {len(ent)};")
    path_of = {}
    by_kj = {}    # output slot k -> edge component j -> [(i, coef)]
    for p, i, j, k, v in ent:
        path_of[k] = p
        by_kj.setdefault(k, {}).setdefault(j, []).append((i, v))

    def b_expr(x, terms):
        # B_jk = sum_i C x[i]: lane-varying operand times a literal, one VALU op per nonzero
        return " + ".join(f"{f(v)} * {x}[{i}]" for i, v in terms)

    def t_expr(x, y, js):
        return " + ".join(f"{y}[{j}] * ({b_expr(x, terms)})" for j, terms in sorted(js.items()))

    # forward: o[k] += gw[p] sum_j y[j] B_jk(x)
    lines.append("  __device__ __forceinline__ static void fwd(const float* __restrict__ x, const float* __restrict__ y,"
                 " const float* __restrict__ gw, float* __restrict__ o) {")
    by_out = {}
    for p, i, j, k, v in ent:
        by_out.setdefault((p, k), []).append((i, j, v))
    for (p, k), terms in sorted(by_out.items(), key=lambda t: t[0][1]):
        expr = " + ".join(f"{f(v)} * (x[{i}] * y[{j}])" for i, j, v in terms)
        lines.append(f"    o[{k}] = fmaf(gw[{p}], {expr}, o[{k}]);")
    lines.append("  }")
    # forward grouped like the adjoints (o[k] += gw[p] sum_j y[j] B_jk(x)): fewer VALU ops, more live
    # values; used where a single forward is the kernel's only contraction
    lines.append("  __device__ __forceinline__ static void fwd_b(const float* __restrict__ x, const float* __restrict__ y,"
                 " const float* __restrict__ gw, float* __restrict__ o) {")
    for k, js in sorted(by_kj.items()):
        lines.append(f"    o[{k}] = fmaf(gw[{path_of[k]}], {t_expr('x', 'y', js)}, o[{k}]);")
    lines.append("  }")
    # dx: d[i] += sum_j y[j] sum_p gw[p] sum_{k in p} C go[k]
    lines.append("  __device__ __forceinline__ static void dx(const float* __restrict__ y, const float* __restrict__ gw,"
                 " const float* __restrict__ go, float* __restrict__ d) {")
    by_ij = {}
    for p, i, j, k, v in ent:
        by_ij.setdefault(i, {}).setdefault(j, {}).setdefault(p, []).append((k, v))
    for i, js in sorted(by_ij.items()):
        parts = []
        for j, ps in sorted(js.items()):
            inner = " + ".join(f"gw[{p}] * ({' + '.join(f'{f(v)} * go[{k}]' for k, v in ks)})"
                               for p, ks in sorted(ps.items()))
            parts.append(f"y[{j}] * ({inner})")
        lines.append(f"    d[{i}] += {' + '.join(parts)};")
    lines.append("  }")
    # dy: d[j] += sum_k (gw[p] go[k]) B_jk(x)
    lines.append("  __device__ __forceinline__ static void dy(const float* __restrict__ x, const float* __restrict__ gw,"
                 " const float* __restrict__ go, float* __restrict__ d) {")
    for k, js in sorted(by_kj.items()):
        lines.append(f"    {{ const float w = gw[{path_of[k]}] * go[{k}];")
        for j, terms in sorted(js.items()):
            lines.append(f"      d[{j}] = fmaf(w, {b_expr('x', terms)}, d[{j}]);")
        lines.append(f"    }}{SB}")
    lines.append("  }")
    # dg: d[p] = sum_{k in p} go[k] sum_j y[j] B_jk(x)
    lines.append("  __device__ __forceinline__ static void dg(const float* __restrict__ x, const float* __restrict__ y,"
                 " const float* __restrict__ go, float* __restrict__ d) {")
    lines.append(f"#pragma unroll\n    for (int p = 0; p < {P}; ++p) d[p] = 0.f;")
    for k, js in sorted(by_kj.items()):
        lines.append(f"    d[{path_of[k]}] = fmaf(go[{k}], {t_expr('x', 'y', js)}, d[{path_of[k]}]);{SB}")
    lines.append("  }")
    # dy and dg of one x together: each B_jk(x) feeds both
    lines.append("  __device__ __forceinline__ static void dydg(const float* __restrict__ x, const float* __restrict__ y,"
                 " const float* __restrict__ gw, const float* __restrict__ go, float* __restrict__ dyv,"
                 " float* __restrict__ d) {")
    lines.append(f"#pragma unroll\n    for (int p = 0; p < {P}; ++p) d[p] = 0.f;")
    for k, js in sorted(by_kj.items()):
        p = path_of[k]
        lines.append(f"    {{ const float w = gw[{p}] * go[{k}]; float t = 0.f;")
        for j, terms in sorted(js.items()):
            lines.append(f"      {{ const float b = {b_expr('x', terms)}; dyv[{j}] = fmaf(w, b, dyv[{j}]);"
                         f" t = fmaf(y[{j}], b, t); }}")
        lines.append(f"      d[{p}] = fmaf(go[{k}], t, d[{p}]); }}{SB}")
    lines.append("  }")
    # dx, dy and dg together, factorised through V_p[i][j] = sum_{k in p} C go[k] (one op per nonzero):
    #   d[i]   += gw[p] sum_j V_p[i][j] y[j]
    #   dyv[j] += gw[p] sum_i V_p[i][j] x[i]
    #   dg[p]   = sum_j y[j] sum_i V_p[i][j] x[i]
    # path by path (V_p, its row sums and its column sums live only inside the path's block)
    by_pij = {}
    for p, i, j, k, v in ent:
        by_pij.setdefault(p, {}).setdefault((i, j), []).append((k, v))

    def factored(name, args, want_dx, want_dydg):
        lines.append(f"  __device__ __forceinline__ static void {name}({args}) {{")
        for p in range(P):
            pairs = by_pij.get(p, {})
            lines.append("    {")
            for (i, j), ks in sorted(pairs.items()):
                lines.append(f"      const float v{i}_{j} = {' + '.join(f'{f(v)} * go[{k}]' for k, v in ks)};")
            rows = {}
            cols = {}
            for (i, j) in sorted(pairs):
                rows.setdefault(i, []).append(j)
                cols.setdefault(j, []).append(i)
            if want_dx:
                for i, js in sorted(rows.items()):
                    lines.append(f"      d[{i}] = fmaf(gw[{p}], {' + '.join(f'v{i}_{j} * y[{j}]' for j in js)}, d[{i}]);")
            if want_dydg:
                tl = []
                for j, is_ in sorted(cols.items()):
                    lines.append(f"      const float t{j} = {' + '.join(f'v{i}_{j} * x[{i}]' for i in is_)};")
                    lines.append(f"      dyv[{j}] = fmaf(gw[{p}], t{j}, dyv[{j}]);")
                    tl.append(f"y[{j}] * t{j}")
                lines.append(f"      dg[{p}] = {' + '.join(tl) if tl else '0.f'};")
            lines.append(f"    }}{SB}")
        lines.append("  }")

    factored("dxdydg", "const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ gw, "
             "const float* __restrict__ go, float* __restrict__ d, float* __restrict__ dyv, float* __restrict__ dg",
             True, True)
    # dy and dg alone (x varies per edge, so nothing of dydg's B_jk(x) survives between edges)
    factored("dydg_v", "const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ gw, "
             "const float* __restrict__ go, float* __restrict__ dyv, float* __restrict__ dg", False, True)
    # dx alone
    factored("dx_v", "const float* __restrict__ y, const float* __restrict__ gw, const float* __restrict__ go, "
             "float* __restrict__ d", True, False)
    lines.append("};")
    return "\n".join(lines)


def tp_group_struct(li, le, lo, l1):
    """``TpG<LI,LE,LO,L1>``: the paths of ``Tp<LI,LE,LO>`` with input degree l1 only.

    Paths are enumerated l1 outer, so a group is the contiguous range
    P0 .. P0+PG-1 of path indices (and of gate rows).  Operands are the group's
    views: x[NXG] the degree-l1 block (component m1), gw[PG] the group's gates,
    o / go[NOG] the group's output slots, whose packed output components are
    SLOT[0..NOG) in ascending order.  Same term grouping as ``Tp``.
    """
    paths = tables.natural_paths(li, le, lo)
    group = [p for p, path in enumerate(paths) if path[0] == l1]
    if not group:
        return None
    T = tables.PathTable(paths, lmax_out=lo)
    p0, PG = group[0], len(group)
    assert group == list(range(p0, p0 + PG))
    slots = sorted({T.out_component(p, m3) for p in group for m3 in range(2 * paths[p][2] + 1)})
    local = {k: n for n, k in enumerate(slots)}
    ent = []
    for p in group:
        for (m1, m2, m3, v) in T.nonzeros(p):
            ent.append((p - p0, m1, paths[p][1] ** 2 + m2, local[T.out_component(p, m3)], v))
    NY = (le + 1) ** 2
    lines = [f"template <> struct TpG<{li}, {le}, {lo}, {l1}> {{",
             f"  static constexpr int LI = {li}, LE = {le}, LO = {lo}, L1 = {l1};",
             f"  static constexpr int NXG = {2 * l1 + 1}, X0 = {l1 * l1}, NY = {NY}, P0 = {p0}, PG = {PG}, "
             f"NOG = {len(slots)}, NO = {T.out_components};",
             f"  static constexpr int SLOT[{len(slots)}] = {{{', '.join(map(str, slots))}}};"]
    path_of, by_kj = {}, {}
    for p, i, j, k, v in ent:
        path_of[k] = p
        by_kj.setdefault(k, {}).setdefault(j, []).append((i, v))

    def b_expr(x, terms):
        return " + ".join(f"{f(v)} * {x}[{i}]" for i, v in terms)

    def t_expr(x, y, js):
        return " + ".join(f"{y}[{j}] * ({b_expr(x, terms)})" for j, terms in sorted(js.items()))

    lines.append("  __device__ __forceinline__ static void fwd_b(const float* __restrict__ x, const float* __restrict__ y,"
                 " const float* __restrict__ gw, float* __restrict__ o) {")
    for k, js in sorted(by_kj.items()):
        lines.append(f"    o[{k}] = fmaf(gw[{path_of[k]}], {t_expr('x', 'y', js)}, o[{k}]);")
    lines.append("  }")
    lines.append("  __device__ __forceinline__ static void dx(const float* __restrict__ y, const float* __restrict__ gw,"
                 " const float* __restrict__ go, float* __restrict__ d) {")
    by_ij = {}
    for p, i, j, k, v in ent:
        by_ij.setdefault(i, {}).setdefault(j, {}).setdefault(p, []).append((k, v))
    for i, js in sorted(by_ij.items()):
        parts = []
        for j, ps in sorted(js.items()):
            inner = " + ".join(f"gw[{p}] * ({' + '.join(f'{f(v)} * go[{k}]' for k, v in ks)})"
                               for p, ks in sorted(ps.items()))
            parts.append(f"y[{j}] * ({inner})")
        lines.append(f"    d[{i}] += {' + '.join(parts)};")
    lines.append("  }")
    lines.append("  __device__ __forceinline__ static void dydg(const float* __restrict__ x, const float* __restrict__ y,"
                 " const float* __restrict__ gw, const float* __restrict__ go, float* __restrict__ dyv,"
                 " float* __restrict__ d) {")
    lines.append(f"#pragma unroll\n    for (int p = 0; p < {PG}; ++p) d[p] = 0.f;")
    for k, js in sorted(by_kj.items()):
        p = path_of[k]
        lines.append(f"    {{ const float w = gw[{p}] * go[{k}]; float t = 0.f;")
        for j, terms in sorted(js.items()):
            lines.append(f"      {{ const float b = {b_expr('x', terms)}; dyv[{j}] = fmaf(w, b, dyv[{j}]);"
                         f" t = fmaf(y[{j}], b, t); }}")
        lines.append(f"      d[{p}] = fmaf(go[{k}], t, d[{p}]); }}")
    lines.append("  }")
    lines.append("  __device__ __forceinline__ static void dg(const float* __restrict__ x, const float* __restrict__ y,"
                 " const float* __restrict__ go, float* __restrict__ d) {")
    lines.append(f"#pragma unroll\n    for (int p = 0; p < {PG}; ++p) d[p] = 0.f;")
    for k, js in sorted(by_kj.items()):
        lines.append(f"    d[{path_of[k]}] = fmaf(go[{k}], {t_expr('x', 'y', js)}, d[{path_of[k]}]);")
    lines.append("  }")
    lines.append("};")
    return "\n".join(lines)


def sh_struct(L):
    N = (L + 1) ** 2
    lines = [f"template <> struct Sh<{L}> {{", f"  static constexpr int N = {N};",
             "  __device__ __forceinline__ static void fwd(float x, float y, float z, float* __restrict__ Y) {"]
    # power tables
    lines.append(f"    float px[{L + 1}], py[{L + 1}], pz[{L + 1}]; px[0] = py[0] = pz[0] = 1.f;")
    for k in range(1, L + 1):
        lines.append(f"    px[{k}] = px[{k - 1}] * x; py[{k}] = py[{k - 1}] * y; pz[{k}] = pz[{k - 1}] * z;")
    polys = {l: tables.harmonic_polynomials(l) for l in range(L + 1)}
    for l in range(L + 1):
        mono, coef = polys[l]
        for m in range(2 * l + 1):
            terms = [f"{f(coef[k, m])} * (px[{a}] * py[{b}] * pz[{c}])"
                     for k, (a, b, c) in enumerate(mono) if abs(coef[k, m]) > tables.ZERO]
            lines.append(f"    Y[{l * l + m}] = {' + '.join(terms) or '0.f'};")
    lines.append("  }")
    # backward: gradient of sum_m gY[m] Y[m] wrt (x,y,z)
    lines.append("  __device__ __forceinline__ static void bwd(float x, float y, float z, const float* __restrict__ g,"
                 " float& gx, float& gy, float& gz) {")
    lines.append(f"    float px[{L + 1}], py[{L + 1}], pz[{L + 1}]; px[0] = py[0] = pz[0] = 1.f;")
    for k in range(1, L + 1):
        lines.append(f"    px[{k}] = px[{k - 1}] * x; py[{k}] = py[{k - 1}] * y; pz[{k}] = pz[{k - 1}] * z;")
    lines.append("    float ax = 0.f, ay = 0.f, az = 0.f;")
    for l in range(1, L + 1):
        mono, coef = polys[l]
        for k, (a, b, c) in enumerate(mono):
            gterms = [f"{f(coef[k, m])} * g[{l * l + m}]" for m in range(2 * l + 1) if abs(coef[k, m]) > tables.ZERO]
            if not gterms:
                continue
            lines.append(f"    {{ const float s = {' + '.join(gterms)};")
            if a:
                lines.append(f"      ax = fmaf(s, {float(a)}f * (px[{a - 1}] * py[{b}] * pz[{c}]), ax);")
            if b:
                lines.append(f"      ay = fmaf(s, {float(b)}f * (px[{a}] * py[{b - 1}] * pz[{c}]), ay);")
            if c:
                lines.append(f"      az = fmaf(s, {float(c)}f * (px[{a}] * py[{b}] * pz[{c - 1}]), az);")
            lines.append("    }")
    lines.append("    gx = ax; gy = ay; gz = az;")
    lines.append("  }")
    # forward-mode product J h  (the cotangent derivative of bwd)
    lines.append("  __device__ __forceinline__ static void jvp(float x, float y, float z, float hx, float hy, float hz,"
                 " float* __restrict__ dY) {")
    lines.append(f"    float px[{L + 1}], py[{L + 1}], pz[{L + 1}]; px[0] = py[0] = pz[0] = 1.f;")
    for k in range(1, L + 1):
        lines.append(f"    px[{k}] = px[{k - 1}] * x; py[{k}] = py[{k - 1}] * y; pz[{k}] = pz[{k - 1}] * z;")
    lines.append("    dY[0] = 0.f;")
    for l in range(1, L + 1):
        mono, coef = polys[l]
        dmono = []
        for (a, b, c) in mono:
            t = []
            if a:
                t.append(f"{float(a)}f * (px[{a - 1}] * py[{b}] * pz[{c}]) * hx")
            if b:
                t.append(f"{float(b)}f * (px[{a}] * py[{b - 1}] * pz[{c}]) * hy")
            if c:
                t.append(f"{float(c)}f * (px[{a}] * py[{b}] * pz[{c - 1}]) * hz")
            dmono.append(" + ".join(t) or "0.f")
        for k in range(len(mono)):
            lines.append(f"    const float d{l}_{k} = {dmono[k]};")
        for m in range(2 * l + 1):
            terms = [f"{f(coef[k, m])} * d{l}_{k}" for k in range(len(mono)) if abs(coef[k, m]) > tables.ZERO]
            lines.append(f"    dY[{l * l + m}] = {' + '.join(terms) or '0.f'};")
    lines.append("  }")
    # Hessian-vector product of s(n) = sum_k g[k] Y_k(n)
    lines.append("  __device__ __forceinline__ static void hvp(float x, float y, float z, const float* __restrict__ g,"
                 " float hx, float hy, float hz, float& ox, float& oy, float& oz) {")
    lines.append(f"    float px[{L + 1}], py[{L + 1}], pz[{L + 1}]; px[0] = py[0] = pz[0] = 1.f;")
    for k in range(1, L + 1):
        lines.append(f"    px[{k}] = px[{k - 1}] * x; py[{k}] = py[{k - 1}] * y; pz[{k}] = pz[{k - 1}] * z;")
    lines.append("    float ax = 0.f, ay = 0.f, az = 0.f;")

    def mon(a, b, c):
        return f"(px[{a}] * py[{b}] * pz[{c}])"
    for l in range(2, L + 1):
        mono, coef = polys[l]
        for k, (a, b, c) in enumerate(mono):
            gterms = [f"{f(coef[k, m])} * g[{l * l + m}]" for m in range(2 * l + 1) if abs(coef[k, m]) > tables.ZERO]
            if not gterms:
                continue
            H = {}
            if a >= 2:
                H[("x", "x")] = f"{float(a * (a - 1))}f * {mon(a - 2, b, c)}"
            if b >= 2:
                H[("y", "y")] = f"{float(b * (b - 1))}f * {mon(a, b - 2, c)}"
            if c >= 2:
                H[("z", "z")] = f"{float(c * (c - 1))}f * {mon(a, b, c - 2)}"
            if a and b:
                H[("x", "y")] = f"{float(a * b)}f * {mon(a - 1, b - 1, c)}"
            if a and c:
                H[("x", "z")] = f"{float(a * c)}f * {mon(a - 1, b, c - 1)}"
            if b and c:
                H[("y", "z")] = f"{float(b * c)}f * {mon(a, b - 1, c - 1)}"
            if not H:
                continue
            lines.append(f"    {{ const float s = {' + '.join(gterms)};")
            for (u, v), expr in H.items():
                if u == v:
                    lines.append(f"      a{u} = fmaf(s * ({expr}), h{u}, a{u});")
                else:
                    lines.append(f"      {{ const float t = s * ({expr}); a{u} = fmaf(t, h{v}, a{u}); a{v} = fmaf(t, h{u}, a{v}); }}")
            lines.append("    }")
    lines.append("    ox = ax; oy = ay; oz = az;")
    lines.append("  }")
    lines.append("};")
    return "\n".join(lines)


def generate(path):
    parts = ["// Generated by csrc/gen_tables.py from the frozen ICTC basis. Do not edit.",
             "#pragma once", "namespace ictc {",
             "template <int LI, int LE, int LO> struct Tp;", "template <int L> struct Sh;"]
    configs = []
    for li in range(LMAX + 1):
        for le in range(LMAX + 1):
            for lo in range(LMAX + 1):
                s = tp_struct(li, le, lo)
                if s is not None:
                    parts.append(s)
                    configs.append((li, le, lo))
    parts.append("template <int LI, int LE, int LO, int L1> struct TpG;")
    for li, le, lo in configs:
        for l1 in range(li + 1):
            g = tp_group_struct(li, le, lo, l1)
            if g is not None:
                parts.append(g)
    for L in range(LMAX + 1):
        parts.append(sh_struct(L))
    parts.append("}  // namespace ictc")
    parts.append("#define ICTC_FOR_EACH_TP(X) " + " ".join(f"X({a},{b},{c})" for a, b, c in configs))
    text = "\n".join(parts) + "\n"
    os.makedirs(os.path.dirname(path), exist_ok=True)
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as fh:
            fh.write(text)
    return configs


if __name__ == "__main__":
    out = sys.argv[1] if len(sys.argv) > 1 else os.path.join(_HERE, "generated", "ictc_tables.h")
    print(len(generate(out)), "TP configurations ->", out)
