"""Autograd Functions over the per-edge TP and the CSR graph message kernels.

Both maps are multilinear in (features x, harmonics Y, gates g) and linear in
the upstream cotangent go.  Writing F(x, Y, g) for the forward and
A_x, A_Y, A_g for its first adjoints (each bilinear in the remaining operand
and go), the mixed second derivatives needed for force-loss training follow
from the same kernels with one operand swapped for its tangent
(the algebra of the reference's _second_raw, ops/fused_message.py:677-729,
and generated_message_second.py:78-204):

  d go  = F(hx, Y, g) + F(x, hY, g) + F(x, Y, hg)
  d x   = A_x(hY, g, go) + A_x(Y, hg, go)
  d Y   = A_Y(hx, g, go) + A_Y(x, hg, go)
  d g   = A_g(hx, Y, go) + A_g(x, hY, go)

Every term is itself an autograd Function, so derivatives of any order stay
on the HIP kernels (the reference recomputes third and higher orders through
a differentiable torch path, operators.py:85-103).
"""
from __future__ import annotations

import weakref
from dataclasses import dataclass
from typing import Optional

import torch

from ictc_o3 import _native as nat
from ictc_o3 import _timing
from ictc_o3.autograd import required_gradients
from torch.autograd.function import once_differentiable


@dataclass(frozen=True)
class TpSpec:
    """Static description of one natural-parity TP (degrees, channels, fixed weight)."""
    li: int
    le: int
    lo: int
    channels: int
    num_paths: int
    out_components: int
    weight: Optional[torch.Tensor] = None   # [P, C] fixed coefficients, None = unit

    @property
    def nx(self):
        return (self.li + 1) ** 2

    @property
    def ny(self):
        return (self.le + 1) ** 2


def make_spec(li, le, lo, channels, weight=None) -> TpSpec:
    P, NO = nat.tp_shape(li, le, lo)
    return TpSpec(li, le, lo, channels, P, NO, weight)


def _w(spec):
    return nat.ptr(spec.weight) if spec.weight is not None else None


def _c(t):
    return t if t.is_contiguous() else t.contiguous()


def _add(a, b):
    if a is None:
        return b
    if b is None:
        return a
    return a + b


# ---------------------------------------------------------------------------
# Per-edge TP
# ---------------------------------------------------------------------------


def _edge_fwd_raw(spec, x, sh, g):
    E = x.shape[0]
    out = x.new_empty(E, spec.out_components * spec.channels)
    nat.call("ictc_tp_fwd", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh), nat.ptr(g),
             _w(spec), E, nat.ptr(out), nat.stream_of(x))
    return out


def _group_ws(spec, E, dsh):
    """Workspace of the channel groups' partial harmonic gradients (None when not needed)."""
    if dsh is None:
        return None, 0
    nbytes = int(nat.lib().ictc_tp_workspace_bytes(spec.le, spec.channels, E))
    if nbytes <= 0:
        return None, 0
    return torch.empty(nbytes // 4, dtype=torch.float32, device=dsh.device), nbytes


def _edge_bwd_raw(spec, x, sh, g, go, need):
    E = x.shape[0]
    dx = torch.empty_like(x) if need[0] else None
    dsh = torch.empty_like(sh) if need[1] else None
    dg = torch.empty_like(g) if need[2] else None
    ws, ws_bytes = _group_ws(spec, E, dsh)
    nat.call("ictc_tp_bwd", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh), nat.ptr(g),
             _w(spec), nat.ptr(go), E, nat.ptr(dx), nat.ptr(dsh), nat.ptr(dg), nat.ptr(ws), ws_bytes,
             nat.stream_of(x))
    return dx, dsh, dg


def _tangents(tx, tsh, tg):
    return tuple(None if t is None else _c(t) for t in (tx, tsh, tg))


def _second_outputs(need, tx, tsh, tg):
    """Which of (dx, dsh, dg, dgo) have a contributing tangent (the others are None)."""
    nx, nsh, ng, ngo = need
    return (nx and (tsh is not None or tg is not None), nsh and (tx is not None or tg is not None),
            ng and (tx is not None or tsh is not None), ngo and any(t is not None for t in (tx, tsh, tg)))


def _edge_second_raw(spec, x, sh, g, go, tx, tsh, tg, need):
    """Fused mixed second derivative of the edge TP adjoint (one kernel); returns (dx, dsh, dg, dgo)."""
    E = x.shape[0]
    tx, tsh, tg = _tangents(tx, tsh, tg)
    wx, wsh, wg, wgo = _second_outputs(need, tx, tsh, tg)
    dx = torch.empty_like(x) if wx else None
    dsh = torch.empty_like(sh) if wsh else None
    dg = torch.empty_like(g) if wg else None
    dgo = torch.empty_like(go) if wgo else None
    if wx or wsh or wg or wgo:
        ws, ws_bytes = _group_ws(spec, E, dsh)
        nat.call("ictc_tp_second", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh), nat.ptr(g),
                 _w(spec), nat.ptr(go), nat.ptr(tx), nat.ptr(tsh), nat.ptr(tg), E, nat.ptr(dgo), nat.ptr(dx),
                 nat.ptr(dsh), nat.ptr(dg), nat.ptr(ws), ws_bytes, nat.stream_of(x))
    return dx, dsh, dg, dgo


class EdgeTP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, sh, g, spec):
        ctx.set_materialize_grads(False)
        ctx.spec = spec
        x, sh, g = _c(x), _c(sh), _c(g)
        ctx.save_for_backward(x, sh, g)
        return _edge_fwd_raw(spec, x, sh, g)

    @staticmethod
    def backward(ctx, go):
        if go is None:
            return None, None, None, None
        x, sh, g = ctx.saved_tensors
        need = required_gradients((x, sh, g), ctx.needs_input_grad[:3])
        if not any(need):
            return None, None, None, None
        dx, dsh, dg = EdgeTPAdjoint.apply(x, sh, g, _c(go), ctx.spec, need)
        return dx, dsh, dg, None


def edge_tp(x, sh, g, spec):
    return EdgeTP.apply(x, sh, g, spec)


def edge_adjoint(x, sh, g, go, spec, need):
    return EdgeTPAdjoint.apply(x, sh, g, go, spec, need)


class EdgeTPAdjoint(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, sh, g, go, spec, need):
        ctx.set_materialize_grads(False)
        ctx.spec = spec
        x, sh, g, go = _c(x), _c(sh), _c(g), _c(go)
        ctx.save_for_backward(x, sh, g, go)
        return _edge_bwd_raw(spec, x, sh, g, go, need)

    @staticmethod
    def backward(ctx, hx, hsh, hg):
        x, sh, g, go = ctx.saved_tensors
        spec = ctx.spec
        nx, nsh, ng, ngo = required_gradients((x, sh, g, go), ctx.needs_input_grad[:4])
        if not torch.is_grad_enabled():
            # the mixed second derivative itself is the last order asked for: one fused kernel
            dx, dsh, dg, dgo = _edge_second_raw(spec, x, sh, g, go, hx, hsh, hg, (nx, nsh, ng, ngo))
            return dx, dsh, dg, dgo, None, None
        # higher orders: compose differentiable first-order operators (multilinearity)
        dx = dsh = dg = dgo = None
        if ngo:
            if hx is not None:
                dgo = _add(dgo, edge_tp(hx, sh, g, spec))
            if hsh is not None:
                dgo = _add(dgo, edge_tp(x, hsh, g, spec))
            if hg is not None:
                dgo = _add(dgo, edge_tp(x, sh, hg, spec))
        if nx:
            if hsh is not None:
                dx = _add(dx, edge_adjoint(x, hsh, g, go, spec, (True, False, False))[0])
            if hg is not None:
                dx = _add(dx, edge_adjoint(x, sh, hg, go, spec, (True, False, False))[0])
        if nsh:
            if hx is not None:
                dsh = _add(dsh, edge_adjoint(hx, sh, g, go, spec, (False, True, False))[1])
            if hg is not None:
                dsh = _add(dsh, edge_adjoint(x, sh, hg, go, spec, (False, True, False))[1])
        if ng:
            if hx is not None:
                dg = _add(dg, edge_adjoint(hx, sh, g, go, spec, (False, False, True))[2])
            if hsh is not None:
                dg = _add(dg, edge_adjoint(x, hsh, g, go, spec, (False, False, True))[2])
        return dx, dsh, dg, dgo, None, None


# ---------------------------------------------------------------------------
# CSR topology and graph message
# ---------------------------------------------------------------------------


class Csr:
    """Stable key-sorted CSR of an edge list (int32 ptr [N+2] and order [E]).

    presorted=True: the keys are known to be in non-decreasing order and in
    range (a receiver-sorted neighbour list); only ptr is built and order is
    None (the identity)."""

    def __init__(self, keys: torch.Tensor, nodes: int, presorted: bool = False):
        E = keys.numel()
        self.nodes = nodes
        self.ptr = torch.empty(nodes + 2, dtype=torch.int32, device=keys.device)
        if presorted:
            self.order = None
            nat.call("ictc_csr_build", nat.ptr(keys), E, nodes, nat.ptr(self.ptr), None, None, 0,
                     nat.stream_of(keys))
            return
        self.order = torch.empty(max(E, 1), dtype=torch.int32, device=keys.device)
        ws_bytes = int(nat.lib().ictc_csr_workspace_bytes(E, nodes))
        if ws_bytes < 0:
            raise ValueError("graph too large for int32 CSR indices")
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=keys.device)
        nat.call("ictc_csr_build", nat.ptr(keys), E, nodes, nat.ptr(self.ptr), nat.ptr(self.order),
                 nat.ptr(ws), ws_bytes, nat.stream_of(keys))


    @classmethod
    def prebuilt(cls, ptr: torch.Tensor, order: torch.Tensor | None, nodes: int) -> "Csr":
        """A CSR whose ptr / order were built elsewhere (ictc_edge_pairs_src_csr's source order)."""
        csr = cls.__new__(cls)
        csr.nodes, csr.ptr, csr.order = nodes, ptr, order
        return csr


def morton_order(positions: torch.Tensor, spacing: float) -> torch.Tensor:
    """int32 [N] rows sorted (stably) by the Morton key of their grid cell floor(pos / spacing)."""
    pos = _c(positions.detach().float())
    N = pos.shape[0]
    order = torch.empty(max(N, 1), dtype=torch.int32, device=pos.device)
    ws_bytes = int(nat.lib().ictc_morton_workspace_bytes(N))
    if ws_bytes < 0:
        raise ValueError("too many rows for an int32 row order")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=pos.device)
    nat.call("ictc_morton_order", nat.ptr(pos), N, float(spacing), nat.ptr(order), nat.ptr(ws), ws_bytes,
             nat.stream_of(pos))
    return order[:N]


def _receiver_rows(positions: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    """The receiver passes' row order: ``rows`` (Morton) when consecutively numbered atoms lie, on average,
    over twice as far apart as consecutive ``rows``, else index order (0 .. N-1).

    A lattice or domain-ordered numbering lands near 1x (both orders step to a
    neighbour, measured within 2 % of each other on the receiver passes); a
    shuffled numbering lands near (box / neighbour spacing) x.  Decided on the
    device (no host sync): both candidates are row lists the kernels read the same way.
    """
    pos = _c(positions.detach().float())
    N = pos.shape[0]
    out = torch.empty(max(N, 1), dtype=torch.int32, device=pos.device)
    ws_bytes = int(nat.lib().ictc_receiver_rows_workspace_bytes(N))
    if ws_bytes < 0:
        raise ValueError("too many rows for an int32 row order")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=pos.device)
    nat.call("ictc_receiver_rows", nat.ptr(pos), N, nat.ptr(_c(rows)), nat.ptr(out), nat.ptr(ws), ws_bytes,
             nat.stream_of(pos))
    return out[:N]


def mark_receiver_sorted(dst: torch.Tensor, nodes: int) -> torch.Tensor:
    """Record that `dst` (as it is now) is in non-decreasing order with every id in [0, nodes): a Topology
    over it skips the receiver sort.  For edge lists built sorted (the neighbour list); an in-place change
    of `dst` (a new version) or another node count clears the mark."""
    dst._ictc_receiver_sorted = (dst._version, int(nodes))
    return dst


def receiver_sorted(dst: torch.Tensor, nodes: int) -> bool:
    return getattr(dst, "_ictc_receiver_sorted", None) == (dst._version, int(nodes))


class Topology:
    """Receiver-sorted CSR (forward, gate / harmonic adjoints) and source-sorted CSR (feature adjoint).

    ``positions`` (optional, [N,3]) sets a spatial (Morton) order in which the
    source-owned feature adjoint visits rows (``src_rows``), so that the
    receiver cotangent rows gathered by concurrent waves share the L2.  The
    receiver-owned passes use the same Morton order (``dst_rows``) only when
    the atom numbering is far less local than it (mean distance between
    consecutively numbered atoms over twice that of the Morton rows).  A numbering that is already
    spatial (a lattice, a domain-decomposed system) keeps index order, which
    streams the receiver-sorted gate rows sequentially; a scattered numbering
    (atoms shuffled, read from an unordered file) gets the Morton order, which
    keeps the gathered sender rows of concurrent waves in L2.  Results are
    bit-identical for any row order.
    """

    def __init__(self, src: torch.Tensor, dst: torch.Tensor, nodes: int, positions: torch.Tensor | None = None,
                 spacing: float = 2.0):
        self.src, self.dst, self.nodes = _c(src), _c(dst), nodes
        self.by_dst = Csr(self.dst, nodes, presorted=receiver_sorted(self.dst, nodes))
        self._by_src = None
        # the row orders are made at their first use (the message kernels), so that work enqueued right
        # after the topology (the edge pairing) reaches the GPU before their launches; they change no
        # result bit, only the visiting order
        self._rows_from = (positions.detach(), spacing) if positions is not None and nodes > 0 else None
        self._src_rows = self._dst_rows = None
        self._gate_rows = None    # int32 [E]: row of the shared radial gates each edge reads (pair_edges)
        self._gate_reps = None    # int32 [rows]: the edge whose length fills each gate row
        self._gate_input = None   # (lengths, their version, those of the gate rows): every layer reads them
        self._pending = None      # pairing launched, row count on its way to the host
        self._pairs_of = None

    def _make_rows(self):
        made, self._rows_from = self._rows_from, None
        if made is not None:
            positions, spacing = made
            self._src_rows = morton_order(positions, spacing)
            if self.nodes > 1:
                self._dst_rows = _receiver_rows(positions, self._src_rows)

    @property
    def src_rows(self):
        self._make_rows()
        return self._src_rows

    @src_rows.setter
    def src_rows(self, value):
        self._rows_from = None
        self._src_rows = value

    @property
    def dst_rows(self):
        self._make_rows()
        return self._dst_rows

    @dst_rows.setter
    def dst_rows(self, value):
        self._make_rows()
        self._dst_rows = value

    def _resolve(self):
        """Finish pair_edges: wait for the row count's copy (only that copy, not the whole stream) and keep
        the shared rows when some edge found its reverse."""
        pending, self._pending = self._pending, None
        if pending is None:
            return
        host, event, rows, reps, E, src_order = pending
        event.synchronize()
        n = int(host[0])
        if n < E:
            self._gate_rows, self._gate_reps = rows, reps[:n]
        if src_order is not None and int(host[1]) == 1 and self._by_src is None:
            # every edge paired one-to-one with its reverse: the source CSR shares the receiver CSR's ptr
            self._by_src = Csr.prebuilt(self.by_dst.ptr, src_order, self.nodes)

    @property
    def gate_rows(self):
        self._resolve()
        return self._gate_rows

    @gate_rows.setter
    def gate_rows(self, value):
        self._pending = None
        self._gate_rows = value

    @property
    def gate_reps(self):
        self._resolve()
        return self._gate_reps

    @gate_reps.setter
    def gate_reps(self, value):
        self._pending = None
        self._gate_reps = value

    def pair_edges(self, shifts: torch.Tensor | None):
        """Share one radial-gate row between every edge and its reverse (same length, bitwise).

        The reverse of (s -> d, shift S) is an edge (d -> s, shift -S); shifts
        [E, 3] are compared exactly (None = no periodic images).  Computed once
        per live shifts tensor and version.  The row count comes to the host by an asynchronous copy and
        is waited for (that copy only) at the first use of gate_rows / gate_reps, so the launches issued in
        between keep the GPU busy.
        Where no edge has a reverse, or the graph is past the pairing's index range (2^30 edges), the rows
        stay per edge (gate_rows None).
        """
        key = None if shifts is None else (shifts._version, tuple(shifts.shape))
        seen = self._pairs_of
        if seen is not None and (seen[0] is None if shifts is None else seen[0] is not None and seen[0]() is shifts) \
                and seen[1] == key:
            return
        E = self.src.numel()
        self._pending = None
        self._gate_rows = self._gate_reps = None
        self._gate_input = None
        ws_bytes = int(nat.lib().ictc_edge_pairs_workspace_bytes(E))
        # pairing is an optimisation: graphs past its index range keep one gate row per edge
        if E > 0 and ws_bytes >= 0 and self.nodes < (1 << 31) - 2:
            sh = None if shifts is None else _c(shifts.detach().to(torch.float32))
            if sh is not None and tuple(sh.shape) != (E, 3):
                raise ValueError("edge shifts must be [E, 3]")
            dev = self.src.device
            rows = torch.empty(E, dtype=torch.int32, device=dev)
            reps = torch.empty(E, dtype=torch.int32, device=dev)
            count = torch.zeros(2, dtype=torch.int32, device=dev)
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
            src_order = None
            if self._by_src is None and SOURCE_CSR_FROM_PAIRS:
                # the same reverse lookup also yields the source CSR of a symmetric list (no sort)
                src_order = torch.empty(E, dtype=torch.int32, device=dev)
                nat.call("ictc_edge_pairs_src_csr", nat.ptr(self.src), nat.ptr(self.dst), nat.ptr(sh), self.nodes,
                         E, nat.ptr(self.by_dst.ptr), nat.ptr(self.by_dst.order), nat.ptr(rows), nat.ptr(reps),
                         nat.ptr(count), nat.ptr(src_order), nat.ptr(count[1:]), nat.ptr(ws), ws_bytes,
                         nat.stream_of(self.src))
            else:
                nat.call("ictc_edge_pairs", nat.ptr(self.src), nat.ptr(self.dst), nat.ptr(sh), self.nodes, E,
                         nat.ptr(self.by_dst.ptr), nat.ptr(self.by_dst.order), nat.ptr(rows), nat.ptr(reps),
                         nat.ptr(count), nat.ptr(ws), ws_bytes, nat.stream_of(self.src))
            host = torch.empty(2, dtype=torch.int32, pin_memory=True)
            host.copy_(count, non_blocking=True)
            event = torch.cuda.Event()
            event.record(torch.cuda.current_stream(dev))
            self._pending = (host, event, rows, reps, E, src_order)
        self._pairs_of = (None if shifts is None else weakref.ref(shifts), key)

    def gate_input(self, r: torch.Tensor) -> torch.Tensor:
        """The edge lengths of the gate rows (r itself when the rows are per edge); the gather is kept for the
        same lengths (the same storage at an unchanged version), which every layer of a step reads."""
        if self.gate_reps is None:
            return r
        graph = torch.is_grad_enabled() and r.requires_grad
        memo = self._gate_input
        if not graph and memo is not None:
            held, version, out = memo   # held keeps the storage alive, so its address is not reused
            if (held.data_ptr() == r.data_ptr() and held.shape == r.shape and held.stride() == r.stride()
                    and held.dtype == r.dtype and held.device == r.device and held._version == version):
                return out
        out = r.index_select(0, self.gate_reps)
        if not graph:
            held = r.detach()   # shares r's version counter: an in-place change invalidates the memo
            self._gate_input = (held, held._version, out)
        return out

    @property
    def by_src(self):
        self._resolve()
        if self._by_src is None:
            self._by_src = Csr(self.src, self.nodes)
        return self._by_src


def _expand_gates(g, gate_rows):
    """Per-edge gate rows [E, ...] from rows shared through gate_rows (None = already per edge)."""
    return g if gate_rows is None else g.index_select(0, gate_rows)


def _msg_fwd_raw(spec, topo, x, sh, g, mask, gate_rows=None):
    N, E = x.shape[0], sh.shape[0]
    out = x.new_empty(N, spec.out_components * spec.channels)
    tok = _timing.begin(f"msg_fwd[{spec.li}{spec.le}{spec.lo}C{spec.channels}]")
    nat.call("ictc_msg_fwd", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh), nat.ptr(g),
             _w(spec), nat.ptr(mask), nat.ptr(topo.src), N, E, nat.ptr(topo.by_dst.ptr),
             nat.ptr(topo.by_dst.order), nat.ptr(topo.dst_rows), nat.ptr(out), nat.ptr(gate_rows),
             nat.stream_of(x))
    _timing.end(tok)
    return out


def _msg_bwd_raw(spec, topo, x, sh, g, mask, go, need, dg_into=None):
    """First adjoint (dx, dsh, dg); dg_into (contiguous, like g): the gate gradient is added to it in place
    (ictc_msg_bwd_accumulate) and returned as dg."""
    N, E = x.shape[0], sh.shape[0]
    dx = torch.empty_like(x) if need[0] else None
    dsh = torch.empty_like(sh) if need[1] else None
    dg = dg_into if dg_into is not None else torch.empty_like(g) if need[2] else None
    sp = topo.by_src if need[0] else None
    ws, ws_bytes = _group_ws(spec, E, dsh)
    nat.call("ictc_msg_bwd_accumulate" if dg_into is not None else "ictc_msg_bwd", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh), nat.ptr(g),
             _w(spec), nat.ptr(mask), nat.ptr(topo.src), nat.ptr(topo.dst), N, E,
             nat.ptr(topo.by_dst.ptr), nat.ptr(topo.by_dst.order),
             nat.ptr(sp.ptr) if sp else None, nat.ptr(sp.order) if sp else None, nat.ptr(topo.dst_rows),
             nat.ptr(topo.src_rows), nat.ptr(go),
             nat.ptr(dx), nat.ptr(dsh), nat.ptr(dg), nat.ptr(ws), ws_bytes, nat.stream_of(x))
    return dx, dsh, dg


def _msg_second_raw(spec, topo, x, sh, g, mask, go, tx, tsh, tg, need):
    """Fused mixed second derivative of the message adjoint; returns (dx, dsh, dg, dgo)."""
    N, E = x.shape[0], sh.shape[0]
    tx, tsh, tg = _tangents(tx, tsh, tg)
    wx, wsh, wg, wgo = _second_outputs(need, tx, tsh, tg)
    dx = torch.empty_like(x) if wx else None
    dsh = torch.empty_like(sh) if wsh else None
    dg = torch.empty_like(g) if wg else None
    dgo = torch.empty_like(go) if wgo else None
    if wx or wsh or wg or wgo:
        sp = topo.by_src if wx else None
        ws, ws_bytes = _group_ws(spec, E, dsh)
        nat.call("ictc_msg_second", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh), nat.ptr(g),
                 _w(spec), nat.ptr(mask), nat.ptr(topo.src), nat.ptr(topo.dst), N, E,
                 nat.ptr(topo.by_dst.ptr), nat.ptr(topo.by_dst.order),
                 nat.ptr(sp.ptr) if sp else None, nat.ptr(sp.order) if sp else None, nat.ptr(topo.dst_rows),
                 nat.ptr(topo.src_rows), nat.ptr(go), nat.ptr(tx), nat.ptr(tsh), nat.ptr(tg), nat.ptr(dgo),
                 nat.ptr(dx), nat.ptr(dsh), nat.ptr(dg), nat.ptr(ws), ws_bytes, nat.stream_of(x))
    return dx, dsh, dg, dgo


def _graph_task():
    """Id of the running backward pass (graph task); -1 outside one."""
    return torch._C._current_graph_task_id()


# Whether the mixed second derivative hands its gate gradient to the first-order message adjoint of the
# same backward pass (_GateLink) instead of returning it for autograd to add; False = autograd's own add.
LINK_GATE_GRADIENTS = True


class _GateLink:
    """Hands the gate gradient of a message's mixed second derivative to the first-order adjoint of the
    same message in the same backward pass.

    In a force-loss backward both passes differentiate the same gates g: the
    mixed second derivative of the force pass's adjoint (MessageAdjoint.backward,
    which runs first) and the first-order adjoint of the forward message
    (Message.backward, later, with the energy term's cotangent and what the
    second derivatives send into the forward graph).  Autograd would add the two
    [E, P*C] gradients with a separate tensor add; instead the second-order pass
    leaves its gradient here and the first-order kernel adds it in its own store
    (ictc_msg_bwd_accumulate; a + b = b + a in IEEE arithmetic, so the sum is
    bitwise autograd's).  The gradient is left only when the engine will still
    run the forward message's node in this pass (torch._C._will_engine_execute_node)
    and that node has not run yet; a callback at the end of the pass raises if
    it was not taken, so a gradient is never dropped silently.
    """
    __slots__ = ("node", "ran", "pending", "what", "enabled", "__weakref__")

    def __init__(self, node, what="message gate gradient of the mixed second derivative",
                 enabled=lambda: LINK_GATE_GRADIENTS):
        self.node = weakref.ref(node)
        self.ran = None          # graph task in which the forward node's backward last ran
        self.pending = None      # (graph task, held value)
        self.what = what
        self.enabled = enabled

    def can_hold(self):
        from torch.fx.experimental.proxy_tensor import get_proxy_mode
        if (not self.enabled() or torch.compiler.is_compiling() or get_proxy_mode() is not None
                or torch._C._are_functorch_transforms_active()
                or not hasattr(torch._C, "_will_engine_execute_node")):
            return False
        task, node = _graph_task(), self.node()
        if self.pending is not None and self.pending[0] != task:
            self.pending = None   # left by a backward pass that stopped early (its callback did not run)
        if task < 0 or node is None or self.ran == task or self.pending is not None:
            return False
        try:
            return bool(torch._C._will_engine_execute_node(node))
        except (RuntimeError, AttributeError, AssertionError):
            return False

    def hold(self, dg):
        task = _graph_task()
        self.pending = (task, dg)
        ref = weakref.ref(self)

        def check():
            link = ref()
            if link is not None and link.pending is not None and link.pending[0] == task:
                link.pending = None
                raise RuntimeError(f"{link.what} was not consumed")
        torch.autograd.Variable._execution_engine.queue_callback(check)

    def take(self):
        task = _graph_task()
        self.ran = task
        if self.pending is not None and self.pending[0] == task:
            dg, self.pending = self.pending[1], None
            return dg
        return None


class Message(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, sh, g, spec, topo, mask):
        ctx.set_materialize_grads(False)
        ctx.spec, ctx.topo, ctx.mask = spec, topo, mask
        ctx.link = _GateLink(ctx)
        x, sh, g = _c(x), _c(sh), _c(g)
        ctx.save_for_backward(x, sh, g)
        return _msg_fwd_raw(spec, topo, x, sh, g, mask)

    @staticmethod
    def backward(ctx, go):
        dg_in = ctx.link.take()   # gate gradient the mixed second derivative left for this pass
        if go is None:
            return None, None, dg_in, None, None, None
        x, sh, g = ctx.saved_tensors
        need = required_gradients((x, sh, g), ctx.needs_input_grad[:3])
        if not any(need):
            return None, None, dg_in, None, None, None
        if torch.is_grad_enabled():
            dx, dsh, dg = MessageAdjoint.apply(x, sh, g, _c(go), ctx.spec, ctx.topo, ctx.mask, need, ctx.link)
        elif dg_in is not None and need[2]:
            dx, dsh, dg = _msg_bwd_raw(ctx.spec, ctx.topo, x, sh, g, ctx.mask, _c(go), need, dg_into=dg_in)
            dg_in = None
        else:
            dx, dsh, dg = _msg_bwd_raw(ctx.spec, ctx.topo, x, sh, g, ctx.mask, _c(go), need)
        if dg_in is not None:
            dg = dg_in if dg is None else dg + dg_in
        return dx, dsh, dg, None, None, None


def _msg_bwd_tangent_raw(spec, topo, x, sh, g, gdot, mask, go, need, gate_rows=None):
    """First adjoint with the gate gradient contracted against gdot = d gates / dr: (dx, dsh, dr)."""
    N, E = x.shape[0], sh.shape[0]
    dx = torch.empty_like(x) if need[0] else None
    dsh = torch.empty_like(sh) if need[1] else None
    dr = sh.new_empty(E)
    sp = topo.by_src if need[0] else None
    nbytes = int(nat.lib().ictc_msg_bwd_tangent_workspace_bytes(spec.le, spec.channels, E))
    ws = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=x.device) if nbytes > 0 else None
    tok = _timing.begin(f"msg_bwd_tan[{spec.li}{spec.le}{spec.lo}C{spec.channels}]")
    nat.call("ictc_msg_bwd_tangent", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh), nat.ptr(g),
             _w(spec), nat.ptr(mask), nat.ptr(topo.src), nat.ptr(topo.dst), N, E,
             nat.ptr(topo.by_dst.ptr), nat.ptr(topo.by_dst.order),
             nat.ptr(sp.ptr) if sp else None, nat.ptr(sp.order) if sp else None, nat.ptr(topo.dst_rows),
             nat.ptr(topo.src_rows), nat.ptr(go), nat.ptr(gdot),
             nat.ptr(dx), nat.ptr(dsh), nat.ptr(dr), nat.ptr(ws), max(nbytes, 0), nat.ptr(gate_rows),
             nat.stream_of(x))
    _timing.end(tok)
    return dx, dsh, dr


class RadialMessage(torch.autograd.Function):
    """message(x, sh, radial_gates(r, fc)) for first-derivative (energy + forces) callers.

    The forward also writes d gates / dr (forward mode through the radial MLP), so
    a backward that needs no weight gradient forms dE/dr = sum dgates * d gates/dr
    inside the message adjoint: the gate gradient [E, P*C], its projection onto the
    hidden layer and the MLP adjoint are never run.  A backward that does need the
    weight gradients takes the ordinary route (message adjoint, then radial adjoint).
    With paired edges (Topology.pair_edges) the gates are evaluated once per
    gate row and read through topo.gate_rows.
    """

    @staticmethod
    def forward(ctx, x, sh, r, W1, W2, W3, W4, spec, topo, mask, cfg):
        from ictc_o3.ops.radial_mlp import radial_gates_tangent
        ctx.set_materialize_grads(False)
        ctx.inputs = (x, sh, r, W1, W2, W3, W4)
        ctx.spec, ctx.topo, ctx.mask, ctx.cfg = spec, topo, mask, cfg
        x, sh = _c(x), _c(sh)
        ctx.rows = topo.gate_rows
        gates, gdot = radial_gates_tangent(topo.gate_input(r), (W1, W2, W3, W4), *cfg)
        ctx.save_for_backward(x, sh, _c(r), *(_c(w) for w in (W1, W2, W3, W4)), gates, gdot)
        return _msg_fwd_raw(spec, topo, x, sh, gates, mask, ctx.rows)

    @staticmethod
    @once_differentiable
    def backward(ctx, go):
        from ictc_o3.ops.radial_mlp import radial_gates_adjoint
        if go is None:
            return (None,) * 11
        x, sh, r, W1, W2, W3, W4, gates, gdot = ctx.saved_tensors
        needs = required_gradients(ctx.inputs, ctx.needs_input_grad[:7])
        ctx.inputs = None
        spec, topo, mask = ctx.spec, ctx.topo, ctx.mask
        go = _c(go)
        dW = [None] * 4
        if any(needs[3:7]):
            gates = _expand_gates(gates, ctx.rows)
            dx, dsh, dg = _msg_bwd_raw(spec, topo, x, sh, gates, mask, go, (needs[0], needs[1], True))
            dr, dW = radial_gates_adjoint(r, (W1, W2, W3, W4), ctx.cfg, dg, (needs[2], *needs[3:7]))
        elif needs[2]:
            dx, dsh, dr = _msg_bwd_tangent_raw(spec, topo, x, sh, gates, gdot, mask, go, needs[:2], ctx.rows)
        elif needs[0] or needs[1]:
            gates = _expand_gates(gates, ctx.rows)
            dx, dsh, _ = _msg_bwd_raw(spec, topo, x, sh, gates, mask, go, (needs[0], needs[1], False))
            dr = None
        else:
            return (None,) * 11
        return (dx, dsh, dr, *dW, None, None, None, None)


# Where the fused radial-gate message (FusedRadialMessage) replaces the materialised-gate RadialMessage:
# "auto" = the compiled shapes with input degree 0 (cfg4 layer 0, P3 C64: 5.3 against 6.0 ms for the
# layer's radial gates + message forward + adjoint); with input degree 2 (P11) the three path-group
# launches of the adjoint measure slower than reading materialised gates (22.8 against 20.7 ms);
# "always" = every compiled shape; "never" = nowhere.
FUSED_GATES = "auto"

# Whether models that need second derivatives run the radial MLP's hidden layers on the fused kernels
# (ictc_o3.ops.radial_mlp.radial_hidden: forward, first adjoint and its derivative in one launch each)
# instead of composing them from per-layer Linear and SiLU operations.
FUSED_HIDDEN = True

# Whether callers of radial_message pair edges with their reverses (Topology.pair_edges) so that the
# radial gates are evaluated once per undirected edge; False keeps one gate row per directed edge.
PAIR_GATES = True
# pair_edges also builds the source CSR from the reverse lookup when the list is symmetric (no sort over src)
SOURCE_CSR_FROM_PAIRS = True


def _fused_weight(fc, W4, spec):
    """W4 folded with the path weight and split into the fused kernels' MFMA operand layout, cached on `fc`
    per (storage, version) of the weights (the reference's _folded_weights, streamed_gate_message.py:23-47)."""
    tpw = spec.weight
    key = (W4.data_ptr(), W4._version, str(W4.device),
           None if tpw is None else (tpw.data_ptr(), tpw._version))
    cached = getattr(fc, "_ictc_fused_w4", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    W = _c(W4.detach())
    nbytes = int(nat.lib().ictc_fused_weight_bytes(spec.num_paths, spec.channels))
    out = torch.empty(nbytes // 4, dtype=torch.float32, device=W.device)
    nat.call("ictc_fused_weight_split", nat.ptr(W), None if tpw is None else nat.ptr(_c(tpw.detach())),
             spec.num_paths, spec.channels, nat.ptr(out), nbytes, nat.stream_of(W))
    fc._ictc_fused_w4 = (key, out)
    return out


def _fused_ok(spec, x):
    if FUSED_GATES == "never" or (FUSED_GATES == "auto" and spec.li != 0):
        return False
    return (x.is_cuda and x.dtype == torch.float32
            and bool(nat.lib().ictc_fused_supported(spec.li, spec.le, spec.lo, spec.channels)))


# Whether the first layer's message (input degree 0, features a function of the species) runs in the species
# form (SpeciesRadialMessage) where the caller supplies the species table; False = FusedRadialMessage.
SPECIES_FORM = True
SPECIES_MAX = 4


def _species_ok(spec, x, xtab):
    return (SPECIES_FORM and xtab is not None and spec.li == 0 and spec.le == spec.lo and spec.le <= 2
            and x.is_cuda and x.dtype == torch.float32 and xtab.dtype == torch.float32
            and 1 <= xtab.shape[0] <= SPECIES_MAX and xtab.shape[1] == spec.channels)


class SpeciesRadialMessage(torch.autograd.Function):
    """message(x, sh, radial_gates(r, fc)) of input degree 0 for energy + forces, with x = xtab[species].

    The first layer's features depend on the species alone, so the message
    factorises through the radial MLP's hidden space: the edge pass sums
    m Y_lm h3 per receiver and source species, and one FP32 GEMM per output
    component projects those sums with W4 folded with the species rows of
    xtab (ictc_species_message_fwd).  The energy-and-forces adjoint projects
    the cotangent the same way and forms dharmonics and dr per edge against the
    hidden state h3 and its r tangent t3 (ictc_species_message_bwd).  h3 and t3
    have one row per gate row (Topology.pair_edges).  A backward that needs the
    feature or weight gradients takes the general route (gates rebuilt from
    h3, ordinary message and radial adjoints) with the full features x.
    The caller guarantees x[n] == xtab[species[n]] (up to rounding).
    """

    @staticmethod
    def forward(ctx, x, sh, r, W1, W2, W3, W4, spec, topo, mask, cfg, xtab, species):
        ctx.set_materialize_grads(False)
        ctx.inputs = (x, sh, r, W1, W2, W3, W4)
        ctx.spec, ctx.topo, ctx.mask, ctx.cfg = spec, topo, mask, cfg
        x, sh, rc = _c(x), _c(sh), _c(r.detach())
        Ws = [_c(w.detach()) for w in (W1, W2, W3, W4)]
        xtab, species = _c(xtab.detach()), _c(species)
        E, N, S = rc.shape[0], x.shape[0], xtab.shape[0]
        rg = _c(topo.gate_input(rc))
        ctx.rows = topo.gate_rows
        h3, t3 = rc.new_empty(rg.shape[0], 64), rc.new_empty(rg.shape[0], 64)
        nat.call("ictc_radial_mlp_tangent_fwd", nat.ptr(rg), rg.shape[0], 8, 64, float(cfg[0]), int(cfg[1]),
                 nat.ptr(Ws[0]), nat.ptr(Ws[1]), nat.ptr(Ws[2]), float(cfg[2]), nat.ptr(h3), nat.ptr(t3),
                 nat.stream_of(rc))
        out = x.new_empty(N, spec.out_components * spec.channels)
        ws, nbytes = _species_ws(spec, S, N, x.device)
        tok = _timing.begin(f"species_fwd[{spec.le}C{spec.channels}S{S}]")
        nat.call("ictc_species_message_fwd", spec.le, spec.lo, spec.channels, S, nat.ptr(xtab), nat.ptr(species),
                 nat.ptr(sh), nat.ptr(h3), nat.ptr(Ws[3]), _w(spec), nat.ptr(mask), nat.ptr(topo.src), N, E,
                 nat.ptr(topo.by_dst.ptr), nat.ptr(topo.by_dst.order), nat.ptr(topo.dst_rows), nat.ptr(ctx.rows),
                 nat.ptr(out), nat.ptr(ws), nbytes, nat.stream_of(x))
        _timing.end(tok)
        ctx.save_for_backward(x, sh, rc, *Ws, h3, t3, xtab, species)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, go):
        from ictc_o3.ops.radial_mlp import gate_projection, radial_gates_adjoint
        if go is None:
            return (None,) * 13
        x, sh, r, W1, W2, W3, W4, h3, t3, xtab, species = ctx.saved_tensors
        needs = required_gradients(ctx.inputs, ctx.needs_input_grad[:7])
        ctx.inputs = None
        spec, topo, mask = ctx.spec, ctx.topo, ctx.mask
        go = _c(go)
        rest = (None,) * 6
        if needs[0] or any(needs[3:7]):
            gates = _expand_gates(gate_projection(h3, W4), ctx.rows)   # unweighted: the kernels apply the path weight
            dx, dsh, dg = _msg_bwd_raw(spec, topo, x, sh, gates, mask, go, (needs[0], needs[1], True))
            dr, dW = radial_gates_adjoint(r, (W1, W2, W3, W4), ctx.cfg, dg, (needs[2], *needs[3:7]))
            return (dx, dsh, dr, *dW, *rest)
        if not (needs[1] or needs[2]):
            return (None,) * 13
        N, E, S = x.shape[0], sh.shape[0], xtab.shape[0]
        dsh, dr = torch.empty_like(sh), sh.new_empty(E)
        ws, nbytes = _species_ws(spec, S, N, x.device)
        tok = _timing.begin(f"species_bwd[{spec.le}C{spec.channels}S{S}]")
        nat.call("ictc_species_message_bwd", spec.le, spec.lo, spec.channels, S, nat.ptr(xtab), nat.ptr(species),
                 nat.ptr(sh), nat.ptr(h3), nat.ptr(t3), nat.ptr(W4), _w(spec), nat.ptr(mask), nat.ptr(topo.src),
                 N, E, nat.ptr(topo.by_dst.ptr), nat.ptr(topo.by_dst.order), nat.ptr(topo.dst_rows),
                 nat.ptr(ctx.rows), nat.ptr(go), nat.ptr(dsh), nat.ptr(dr), nat.ptr(ws), nbytes, nat.stream_of(x))
        _timing.end(tok)
        return (None, dsh if needs[1] else None, dr if needs[2] else None, None, None, None, None, *rest)


def _species_ws(spec, S, N, device):
    nbytes = int(nat.lib().ictc_species_message_workspace_bytes(spec.le, S, spec.channels, N))
    if nbytes < 0:
        raise ValueError("species message: unsupported shape")
    return torch.empty(max(nbytes, 256) // 4, dtype=torch.float32, device=device), nbytes


class FusedRadialMessage(torch.autograd.Function):
    """message(x, sh, radial_gates(r, fc)) for energy + forces without materialised gates.

    The forward writes the MLP's last hidden activation h3 and its r tangent
    t3 = d h3 / dr ([E, 64] each) and the message kernels project the gates
    (and, in the adjoint, their r tangents) per edge tile from them
    (streamed_gate_message.py:87-223).  h3 and t3 have one row per gate row
    of the topology (Topology.pair_edges).  A backward that needs weight
    gradients rebuilds the gates [E, P*C] from h3 and takes the ordinary
    message and radial adjoints.
    """

    @staticmethod
    def forward(ctx, x, sh, r, W1, W2, W3, W4, spec, topo, mask, cfg, w4s):
        ctx.set_materialize_grads(False)
        ctx.inputs = (x, sh, r, W1, W2, W3, W4)
        ctx.spec, ctx.topo, ctx.mask, ctx.cfg, ctx.w4s = spec, topo, mask, cfg, w4s
        x, sh, rc = _c(x), _c(sh), _c(r.detach())
        Ws = [_c(w.detach()) for w in (W1, W2, W3, W4)]
        E = rc.shape[0]
        rg = _c(topo.gate_input(rc))     # one row per edge pair
        ctx.rows = topo.gate_rows
        h3, t3 = rc.new_empty(rg.shape[0], 64), rc.new_empty(rg.shape[0], 64)
        nat.call("ictc_radial_mlp_tangent_fwd", nat.ptr(rg), rg.shape[0], 8, 64, float(cfg[0]), int(cfg[1]),
                 nat.ptr(Ws[0]), nat.ptr(Ws[1]), nat.ptr(Ws[2]), float(cfg[2]), nat.ptr(h3), nat.ptr(t3),
                 nat.stream_of(rc))
        N = x.shape[0]
        out = x.new_empty(N, spec.out_components * spec.channels)
        nat.call("ictc_msg_fused_fwd", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh),
                 nat.ptr(h3), nat.ptr(w4s), nat.ptr(mask), nat.ptr(topo.src), N, E, nat.ptr(topo.by_dst.ptr),
                 nat.ptr(topo.by_dst.order), nat.ptr(topo.dst_rows), nat.ptr(out), nat.ptr(ctx.rows),
                 nat.stream_of(x))
        ctx.save_for_backward(x, sh, rc, *Ws, h3, t3)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, go):
        from ictc_o3.ops.radial_mlp import gate_projection, radial_gates_adjoint
        if go is None:
            return (None,) * 12
        x, sh, r, W1, W2, W3, W4, h3, t3 = ctx.saved_tensors
        needs = required_gradients(ctx.inputs, ctx.needs_input_grad[:7])
        ctx.inputs = None
        spec, topo, mask = ctx.spec, ctx.topo, ctx.mask
        go = _c(go)
        if any(needs[3:7]):
            gates = _expand_gates(gate_projection(h3, W4), ctx.rows)   # unweighted: the kernels apply the path weight
            dx, dsh, dg = _msg_bwd_raw(spec, topo, x, sh, gates, mask, go, (needs[0], needs[1], True))
            dr, dW = radial_gates_adjoint(r, (W1, W2, W3, W4), ctx.cfg, dg, (needs[2], *needs[3:7]))
            return (dx, dsh, dr, *dW, None, None, None, None, None)
        if not any(needs[:3]):
            return (None,) * 12
        N, E = x.shape[0], sh.shape[0]
        dx = torch.empty_like(x) if needs[0] else None
        dsh = torch.empty_like(sh) if needs[1] else None
        dr = sh.new_empty(E)
        sp = topo.by_src if needs[0] else None
        nat.call("ictc_msg_fused_bwd_tangent", spec.li, spec.le, spec.lo, spec.channels, nat.ptr(x), nat.ptr(sh),
                 nat.ptr(h3), nat.ptr(t3), nat.ptr(ctx.w4s), nat.ptr(mask), nat.ptr(topo.src), nat.ptr(topo.dst),
                 N, E, nat.ptr(topo.by_dst.ptr), nat.ptr(topo.by_dst.order),
                 nat.ptr(sp.ptr) if sp else None, nat.ptr(sp.order) if sp else None, nat.ptr(topo.dst_rows),
                 nat.ptr(topo.src_rows), nat.ptr(go), nat.ptr(dx), nat.ptr(dsh), nat.ptr(dr),
                 nat.ptr(ctx.rows), nat.stream_of(x))
        return (dx, dsh, dr if needs[2] else None, None, None, None, None, None, None, None, None, None)


def radial_message(x, sh, r, fc, spec, topo, mask, cfg, basis_scale=1.0, species=None):
    """message() with the fused radial gates of `fc` (SpeciesRadialMessage where the caller passes
    species = (xtab, node species) with x == xtab[node species] and the shape allows it, else
    FusedRadialMessage where the library compiles the shape, else RadialMessage); cfg = (cutoff, poly_p,
    silu_scale); basis_scale multiplies the radial basis (folded into the first Linear's weight)."""
    W = [m.weight for m in fc if isinstance(m, torch.nn.Linear)]
    if basis_scale != 1.0:
        W[0] = W[0] * basis_scale
    cfg = (float(cfg[0]), int(cfg[1]), float(cfg[2]))
    if species is not None and _species_ok(spec, x, species[0]):
        return SpeciesRadialMessage.apply(x, sh, r, *W, spec, topo, mask, cfg, species[0], species[1])
    if _fused_ok(spec, x):
        w4s = _fused_weight(fc, W[-1], spec)
        return FusedRadialMessage.apply(x, sh, r, *W, spec, topo, mask, cfg, w4s)
    return RadialMessage.apply(x, sh, r, *W, spec, topo, mask, cfg)


def message(x, sh, g, spec, topo, mask=None):
    return Message.apply(x, sh, g, spec, topo, mask)


def message_adjoint(x, sh, g, go, spec, topo, mask, need):
    return MessageAdjoint.apply(x, sh, g, go, spec, topo, mask, need)


class MessageAdjoint(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, sh, g, go, spec, topo, mask, need, link=None):
        ctx.set_materialize_grads(False)
        ctx.spec, ctx.topo, ctx.mask, ctx.link = spec, topo, mask, link
        x, sh, g, go = _c(x), _c(sh), _c(g), _c(go)
        ctx.save_for_backward(x, sh, g, go)
        return _msg_bwd_raw(spec, topo, x, sh, g, mask, go, need)

    @staticmethod
    def backward(ctx, hx, hsh, hg):
        x, sh, g, go = ctx.saved_tensors
        spec, topo, mask = ctx.spec, ctx.topo, ctx.mask
        nx, nsh, ng, ngo = required_gradients((x, sh, g, go), ctx.needs_input_grad[:4])
        if not torch.is_grad_enabled():
            # the mixed second derivative itself is the last order asked for: fused kernels
            dx, dsh, dg, dgo = _msg_second_raw(spec, topo, x, sh, g, mask, go, hx, hsh, hg, (nx, nsh, ng, ngo))
            if dg is not None and ctx.link is not None and ctx.link.can_hold():
                ctx.link.hold(dg)   # added by the forward message's first-order adjoint later in this pass
                dg = None
            return dx, dsh, dg, dgo, None, None, None, None, None
        # higher orders: compose differentiable first-order operators (multilinearity)
        dx = dsh = dg = dgo = None
        if ngo:
            if hx is not None:
                dgo = _add(dgo, message(hx, sh, g, spec, topo, mask))
            if hsh is not None:
                dgo = _add(dgo, message(x, hsh, g, spec, topo, mask))
            if hg is not None:
                dgo = _add(dgo, message(x, sh, hg, spec, topo, mask))
        if nx:
            if hsh is not None:
                dx = _add(dx, message_adjoint(x, hsh, g, go, spec, topo, mask, (True, False, False))[0])
            if hg is not None:
                dx = _add(dx, message_adjoint(x, sh, hg, go, spec, topo, mask, (True, False, False))[0])
        if nsh:
            if hx is not None:
                dsh = _add(dsh, message_adjoint(hx, sh, g, go, spec, topo, mask, (False, True, False))[1])
            if hg is not None:
                dsh = _add(dsh, message_adjoint(x, sh, hg, go, spec, topo, mask, (False, True, False))[1])
        if ng:
            if hx is not None:
                dg = _add(dg, message_adjoint(hx, sh, g, go, spec, topo, mask, (False, False, True))[2])
            if hsh is not None:
                dg = _add(dg, message_adjoint(x, hsh, g, go, spec, topo, mask, (False, False, True))[2])
        return dx, dsh, dg, dgo, None, None, None, None, None
