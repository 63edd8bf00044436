"""Edge geometry (vec, r, n, mask) with a deterministic CSR-gather adjoint to the positions.

Forward follows mace_ictc/models/pure_cartesian_ictd_layers.py:1288-1297
(vec = pos[dst] - pos[src] + shift, r = |vec|, n = vec / r.clamp(min=1e-8),
mask = r <= cutoff).  The adjoint replaces the two index-gather backwards
(scatter-adds into pos) with one kernel that sums, per node, the adjoints of its
incoming edges minus those of its outgoing edges in CSR order.  First
derivatives only.  Force-loss training differentiates the edge vectors twice
and uses ``edge_vectors``: the gather and its CSR adjoint are each other's
adjoints, so every derivative order stays deterministic and atomic-free.
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from ictc_o3 import _native as nat


def _c(t):
    return t if t.is_contiguous() else t.contiguous()


class _EdgeGeometry(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pos, shift, topo, cutoff):
        pos = _c(pos.detach())
        shift = None if shift is None else _c(shift.detach())
        E, N = topo.src.numel(), pos.shape[0]
        r = pos.new_empty(E)
        n = pos.new_empty(E, 3)
        mask = pos.new_empty(E)
        nat.call("ictc_edge_geometry_fwd", nat.ptr(pos), nat.ptr(shift), nat.ptr(topo.src), nat.ptr(topo.dst), N, E,
                 float(cutoff), nat.ptr(r), nat.ptr(n), nat.ptr(mask), nat.stream_of(pos))
        ctx.topo, ctx.nodes = topo, N
        ctx.mark_non_differentiable(mask)
        ctx.save_for_backward(r, n)
        return r, n, mask

    @staticmethod
    @once_differentiable
    def backward(ctx, dr, dn, _dmask):
        r, n = ctx.saved_tensors
        topo, N = ctx.topo, ctx.nodes
        E = r.numel()
        dr = None if dr is None else _c(dr)
        dn = None if dn is None else _c(dn)
        dpos = r.new_empty(N, 3)
        dshift = r.new_empty(E, 3) if ctx.needs_input_grad[1] else None
        src_csr = topo.by_src
        nat.call("ictc_edge_geometry_bwd", nat.ptr(r), nat.ptr(n), nat.ptr(dr), nat.ptr(dn), N, E,
                 nat.ptr(topo.by_dst.ptr), nat.ptr(topo.by_dst.order), nat.ptr(src_csr.ptr), nat.ptr(src_csr.order),
                 nat.ptr(dshift), nat.ptr(dpos), nat.stream_of(r))
        return (dpos if ctx.needs_input_grad[0] else None), dshift, None, None


def edge_geometry(pos: torch.Tensor, shift: torch.Tensor | None, topo, cutoff: float):
    """(r [E], n [E,3], mask [E]) for the edges of ``topo`` (a Topology over src/dst), float32."""
    if pos.dtype != torch.float32 or (shift is not None and shift.dtype != torch.float32):
        raise TypeError("edge_geometry runs in float32")
    if pos.dim() != 2 or pos.shape[1] != 3:
        raise ValueError("pos must be [N, 3]")
    if shift is not None and tuple(shift.shape) != (topo.src.numel(), 3):
        raise ValueError("shift must be [E, 3]")
    return _EdgeGeometry.apply(pos, shift, topo, float(cutoff))


class _EdgeHarmonics(torch.autograd.Function):
    """(r, Y, mask) of the edges in one kernel; the adjoint forms d vec per edge (harmonics adjoint folded with
    dr) and gathers it into dpos: the values of _EdgeGeometry followed by the harmonics op (bitwise), and their
    adjoint to FP32 rounding.  With
    uses = 2 the forward also returns r and Y a second time (views) for a second consumer: their cotangents
    reach the backward apart and the kernel adds them, where autograd would have launched the additions."""

    @staticmethod
    def forward(ctx, pos, shift, topo, cutoff, lmax, uses):
        pos = _c(pos.detach())
        shift = None if shift is None else _c(shift.detach())
        E, N = topo.src.numel(), pos.shape[0]
        r = pos.new_empty(E)
        n = pos.new_empty(E, 3)
        mask = pos.new_empty(E)
        Y = pos.new_empty(E, (lmax + 1) ** 2)
        nat.call("ictc_edge_harmonics_fwd", nat.ptr(pos), nat.ptr(shift), nat.ptr(topo.src), nat.ptr(topo.dst), N,
                 E, float(cutoff), lmax, nat.ptr(r), nat.ptr(n), nat.ptr(mask), nat.ptr(Y), nat.stream_of(pos))
        ctx.topo, ctx.nodes, ctx.lmax, ctx.uses = topo, N, lmax, uses
        ctx.mark_non_differentiable(mask)
        ctx.save_for_backward(r, n)
        if uses == 2:
            return r, r.view_as(r), Y, Y.view_as(Y), mask
        return r, Y, mask

    @staticmethod
    @once_differentiable
    def backward(ctx, *grads):
        if ctx.uses == 2:
            dr, dr2, dY, dY2, _dmask = grads
        else:
            (dr, dY, _dmask), dr2, dY2 = grads, None, None
        r, n = ctx.saved_tensors
        E = r.numel()
        dvec = r.new_empty(E, 3)
        cot = [None if g is None else _c(g) for g in (dr, dY, dr2, dY2)]
        # the kernel reads dY / dY2 as 16-byte vectors
        cot = [g if g is None or k in (0, 2) or g.data_ptr() % 16 == 0 else g.clone() for k, g in enumerate(cot)]
        nat.call("ictc_edge_harmonics_bwd", nat.ptr(r), nat.ptr(n), *[nat.ptr(g) for g in cot], E, ctx.lmax,
                 nat.ptr(dvec), nat.stream_of(r))
        dpos = _vector_adjoint(dvec, ctx.topo, ctx.nodes) if ctx.needs_input_grad[0] else None
        return dpos, (dvec if ctx.needs_input_grad[1] else None), None, None, None, None


def edge_harmonics(pos: torch.Tensor, shift: torch.Tensor | None, topo, cutoff: float, lmax: int, uses: int = 1):
    """(r [E], Y [E, (lmax+1)^2], mask [E]): edge_geometry followed by the packed direction harmonics of n, in one
    kernel, float32, first derivatives only (positions and shifts).  uses = 2 returns (r, r', Y, Y', mask) with
    r' and Y' the same values for a second consumer, whose cotangents the adjoint adds in its kernel."""
    if pos.dtype != torch.float32 or (shift is not None and shift.dtype != torch.float32):
        raise TypeError("edge_harmonics runs in float32")
    if pos.dim() != 2 or pos.shape[1] != 3:
        raise ValueError("pos must be [N, 3]")
    if shift is not None and tuple(shift.shape) != (topo.src.numel(), 3):
        raise ValueError("shift must be [E, 3]")
    if not 0 <= int(lmax) <= 3:
        raise ValueError("edge_harmonics: lmax outside 0..3")
    if uses not in (1, 2):
        raise ValueError("edge_harmonics: uses is 1 or 2")
    return _EdgeHarmonics.apply(pos, shift, topo, float(cutoff), int(lmax), int(uses))


def _vector_adjoint(dvec: torch.Tensor, topo, N: int) -> torch.Tensor:
    dvec = _c(dvec.detach())
    dpos = dvec.new_empty(N, 3)
    src_csr = topo.by_src
    nat.call("ictc_edge_vector_bwd", nat.ptr(dvec), N, dvec.shape[0], nat.ptr(topo.by_dst.ptr),
             nat.ptr(topo.by_dst.order), nat.ptr(src_csr.ptr), nat.ptr(src_csr.order), nat.ptr(dpos),
             nat.stream_of(dvec))
    return dpos


class _EdgeVectors(torch.autograd.Function):
    """vec = pos[dst] - pos[src] (+ shift); the adjoint is _EdgeVectorAdjoint."""

    @staticmethod
    def forward(ctx, pos, shift, topo):
        ctx.topo, ctx.nodes = topo, pos.shape[0]
        vec = pos.index_select(0, topo.dst) - pos.index_select(0, topo.src)
        return vec if shift is None else vec + shift

    @staticmethod
    def backward(ctx, dvec):
        dpos = _EdgeVectorAdjoint.apply(dvec, ctx.topo, ctx.nodes) if ctx.needs_input_grad[0] else None
        return dpos, (dvec if ctx.needs_input_grad[1] else None), None


class _EdgeVectorAdjoint(torch.autograd.Function):
    """dpos = sum_in dvec - sum_out dvec (CSR gather); the adjoint is _EdgeVectors without shift."""

    @staticmethod
    def forward(ctx, dvec, topo, N):
        ctx.topo = topo
        return _vector_adjoint(dvec, topo, N)

    @staticmethod
    def backward(ctx, h):
        return _EdgeVectors.apply(h, None, ctx.topo), None, None


def edge_vectors(pos: torch.Tensor, shift: torch.Tensor | None, topo) -> torch.Tensor:
    """vec [E, 3] = pos[dst] - pos[src] + shift for the edges of ``topo``, differentiable to any order."""
    if pos.dim() != 2 or pos.shape[1] != 3:
        raise ValueError("pos must be [N, 3]")
    if not pos.is_cuda or pos.dtype != torch.float32:
        raise TypeError("edge_vectors runs on float32 device tensors")
    return _EdgeVectors.apply(pos, shift, topo)


def shift_vectors(shifts: torch.Tensor, cell: torch.Tensor, batch: torch.Tensor | None,
                  src: torch.Tensor | None) -> torch.Tensor:
    """Cartesian image shifts [E, 3] = shifts [E, 3] (lattice coordinates) . cell of the edge's graph
    (cell [3, 3] or [G, 3, 3]; graph batch[src[e]] when G > 1), as (s0 c0j + s1 c1j) + s2 c2j with every
    operation rounded on its own, so an edge and its reverse get exactly negated shifts.  FP32 device
    tensors; not differentiable (the cell carries no gradient here)."""
    shifts = _c(shifts.detach())
    if shifts.dtype != torch.float32 or shifts.dim() != 2 or shifts.shape[1] != 3:
        raise ValueError("shift_vectors: shifts must be float32 [E, 3]")
    cells = _c(cell.detach().to(torch.float32).reshape(-1, 3, 3))
    E, G = shifts.shape[0], cells.shape[0]
    out = shifts.new_empty(E, 3)
    if G > 1:
        if batch is None or src is None:
            raise ValueError("shift_vectors: batch and src are needed with several cells")
        batch, src = _c(batch.long()), _c(src.long())
    nodes = batch.numel() if G > 1 else 0
    nat.call("ictc_shift_vectors", nat.ptr(shifts), E, nat.ptr(cells), G, nat.ptr(batch) if G > 1 else None,
             nat.ptr(src) if G > 1 else None, nodes, nat.ptr(out), nat.stream_of(shifts))
    return out


def _unit(order, v=None, r=None, n=None, gr=None, gn=None, h=None, outs=()):
    E = (v if v is not None else r).shape[0]
    nat.call("ictc_edge_unit", order, nat.ptr(v), nat.ptr(r), nat.ptr(n), nat.ptr(gr), nat.ptr(gn), nat.ptr(h), E,
             *[nat.ptr(t) for t in outs], *([None] * (3 - len(outs))), nat.stream_of(v if v is not None else r))


def _edge_unit_torch(vec):
    r = vec.norm(dim=1)
    return r, vec / r.clamp(min=1e-8).unsqueeze(-1)


class _EdgeUnit(torch.autograd.Function):
    """(r, n) = (|v|, v / max(|v|, 1e-8)) of edge vectors; the adjoint is _EdgeUnitAdjoint."""

    @staticmethod
    def forward(ctx, vec):
        v = _c(vec.detach())
        r, n = v.new_empty(v.shape[0]), torch.empty_like(v)
        _unit(0, v=v, outs=(r, n))
        ctx.save_for_backward(vec, r, n)
        return r, n

    @staticmethod
    def backward(ctx, gr, gn):
        vec, r, n = ctx.saved_tensors
        if gr is None and gn is None:
            return None
        return _EdgeUnitAdjoint.apply(vec, r, n, gr, gn)


class _EdgeUnitAdjoint(torch.autograd.Function):
    """gv(v, gr, gn) = gr n + (gn - (gn . n) n) / r, differentiable once more on ictc_edge_unit (order 2) and
    to higher orders through the composed torch form."""

    @staticmethod
    def forward(ctx, vec, r, n, gr, gn):
        grc = None if gr is None else _c(gr.detach())
        gnc = None if gn is None else _c(gn.detach())
        gv = torch.empty_like(n)
        _unit(1, r=r, n=n, gr=grc, gn=gnc, outs=(gv,))
        ctx.save_for_backward(vec, r, n, gr, gn)
        return gv

    @staticmethod
    def backward(ctx, h):
        vec, r, n, gr, gn = ctx.saved_tensors
        need_v, _, _, need_gr, need_gn = ctx.needs_input_grad
        if h is None:
            return None, None, None, None, None
        if torch.is_grad_enabled():
            return _edge_unit_adjoint_torch(vec, gr, gn, h, (need_v, need_gr, need_gn))
        dv = torch.empty_like(n) if need_v else None
        dgr = r.new_empty(r.shape[0]) if need_gr and gr is not None else None
        dgn = torch.empty_like(n) if need_gn and gn is not None else None
        _unit(2, r=r, n=n, gr=None if gr is None else _c(gr.detach()), gn=None if gn is None else _c(gn.detach()),
              h=_c(h), outs=(dv, dgr, dgn))
        return dv, None, None, dgr, dgn


def _edge_unit_adjoint_torch(vec, gr, gn, h, needs):
    """Derivative of the adjoint on the composed form, keeping the graph (third and higher orders)."""
    inputs = [t if t is not None and t.requires_grad else (None if t is None else t.detach().requires_grad_(True))
              for t in (vec, gr, gn)]
    v, g1, g2 = inputs
    with torch.enable_grad():
        r, n = _edge_unit_torch(v)
        outs = [(o, c) for o, c in ((r, g1), (n, g2)) if c is not None]
        (gv,) = torch.autograd.grad([o for o, _ in outs], v, [c for _, c in outs], create_graph=True)
        wanted = [t for t, need in zip(inputs, needs) if need and t is not None]
        got = iter(torch.autograd.grad(gv, wanted, h, create_graph=True, allow_unused=True))
    dv, dgr, dgn = (next(got) if need and t is not None else None for t, need in zip(inputs, needs))
    return dv, None, None, dgr, dgn


def edge_unit(vec: torch.Tensor):
    """(r [E], n [E, 3]) = (|vec|, vec / max(|vec|, 1e-8)) with first and second derivatives on ictc_edge_unit
    (float32 on the device); other inputs, and a third derivative, through the composed torch form."""
    if not (vec.is_cuda and vec.dtype == torch.float32 and vec.dim() == 2 and vec.shape[1] == 3):
        return _edge_unit_torch(vec)
    return _EdgeUnit.apply(vec)
