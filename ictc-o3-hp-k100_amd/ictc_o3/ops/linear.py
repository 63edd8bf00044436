"""Channel-mixing linears on the packed component-major layout.

These are the only GEMM-shaped maps of the model (north-star: the MFMA
site).  Shapes (C channels, N nodes):
  degree_linear  out[n, l*l+m, :] = scale * W_l @ x[n, l*l+m, :]            (linear_up, product linear)
  path_linear    out[n, l*l+m, :] = scale * W_l @ concat_k msg[n, l, k, m, :] (message_linear / avg_num_neighbors)
  species_linear out[n, :] = W[s_n] @ x[n, :]                               (element-conditioned self-connection)
The composable forms below are FP32 GEMMs through the ROCm BLAS library (TF32
off) whose weight gradients over the tall row dimension run on the
split-reduction kernel (``edge_linear``); they stay differentiable to any order; ``degree_linear_fast`` /
``path_linear_fast`` run the same maps on the hand-written MFMA kernel
(``ictc_packed_linear``) for first-derivative callers (energy + forces).
"""
from __future__ import annotations

from typing import Dict, List

import torch
from torch.autograd.function import once_differentiable

from ictc_o3.ops.radial_mlp import edge_linear


def degree_linear(x: torch.Tensor, weights: List[torch.Tensor], C: int, lmax: int, scale: float = 1.0):
    N = x.shape[0]
    # one split (its adjoint is a single concatenation) rather than per-degree
    # slices, whose adjoints each materialise a zero-filled full-width gradient
    blocks = torch.split(x, [(2 * l + 1) * C for l in range(lmax + 1)], 1)
    parts = []
    for l in range(lmax + 1):
        blk = blocks[l].reshape(N * (2 * l + 1), C)
        w = weights[l] if scale == 1.0 else weights[l] * scale
        parts.append(edge_linear(blk, w).reshape(N, (2 * l + 1) * C))
    return torch.cat(parts, 1)


def path_linear(m: torch.Tensor, weights: List[torch.Tensor], counts: Dict[int, int], C: int, lmax: int,
                scale: float = 1.0):
    N = m.shape[0]
    sizes = [counts.get(l, 0) * (2 * l + 1) * C for l in range(lmax + 1)]
    tail = m.shape[1] - sum(sizes)
    blocks = torch.split(m, sizes + [tail] if tail else sizes, 1)
    parts = []
    for l in range(lmax + 1):
        k, w = counts.get(l, 0), 2 * l + 1
        blk = blocks[l].reshape(N, k, w, C).transpose(1, 2).reshape(N * w, k * C)
        parts.append(edge_linear(blk, weights[l] * scale).reshape(N, w * C))
    return torch.cat(parts, 1)


def species_linear(x: torch.Tensor, weight: torch.Tensor, species: torch.Tensor):
    """out[n] = weight[species[n]] @ x[n], weight [S, Cout, Cin] (layers.py:21-87).

    Square float32 maps of 64 or 128 channels on the device run on ictc_species_linear over species-sorted
    node tiles (each node's product only, differentiable to any order; nodes whose species is outside
    [0, S) get zero rows); otherwise all species products in one GEMM, then a select."""
    S, Co, Ci = weight.shape
    if (x.is_cuda and x.dtype == torch.float32 and weight.dtype == torch.float32 and Co == Ci and Ci in (64, 128)
            and x.dim() == 2 and x.shape[1] == Ci and species.dtype == torch.int64 and x.shape[0] < 2 ** 31):
        order = species_order(species, S)
        return _SpeciesLinear.apply(x, weight, order, False)
    allp = edge_linear(x, weight.reshape(S * Co, Ci)).reshape(x.shape[0], S, Co)
    return allp.gather(1, species.view(-1, 1, 1).expand(-1, 1, Co)).squeeze(1)


class SpeciesOrder:
    """Nodes in species order: perm [N] int32 node ids sorted by species (stable), off [S + 2] int32 with
    species s at sorted rows off[s] .. off[s + 1] and the nodes of species outside [0, S) last."""

    def __init__(self, species: torch.Tensor, S: int):
        from ictc_o3.ops.tensor_product import Csr
        csr = Csr(species.contiguous(), S)   # ictc_csr_build: stable radix sort over the species bits
        self.perm, self.off = csr.order, csr.ptr
        self.S, self.N = S, species.shape[0]


_order_memo = None


def species_order(species: torch.Tensor, S: int) -> SpeciesOrder:
    """SpeciesOrder of this species tensor, kept while the same unmodified tensor is passed again (both
    layers of a step and their backward share one sort)."""
    global _order_memo
    key = (species.data_ptr(), species._version, species.shape[0], S, species.device)
    if _order_memo is not None and _order_memo[0] == key and _order_memo[1] is species:
        return _order_memo[2]
    order = SpeciesOrder(species, S)
    _order_memo = (key, species, order)
    return order


def _rows_ok(t: torch.Tensor) -> torch.Tensor:
    """t with unit column stride and a row pitch and base the kernels read as 16-byte runs."""
    if t.stride(1) != 1 or t.stride(0) % 4 or t.data_ptr() % 16:
        return t.contiguous()
    return t


def _species_apply(x: torch.Tensor, W: torch.Tensor, order: SpeciesOrder, trans: bool) -> torch.Tensor:
    x, W = _rows_ok(x.detach()), W.detach().contiguous()
    out = x.new_empty(x.shape[0], W.shape[1])
    nat.call("ictc_species_linear", nat.ptr(x), x.stride(0), x.shape[0], x.shape[1], nat.ptr(W), order.S,
             nat.ptr(order.perm), nat.ptr(order.off), 1 if trans else 0, nat.ptr(out), out.stride(0),
             nat.stream_of(x))
    return out


def _species_outer_raw(a: torch.Tensor, b: torch.Tensor, order: SpeciesOrder) -> torch.Tensor:
    a, b = _rows_ok(a.detach()), _rows_ok(b.detach())
    N, C, S = a.shape[0], a.shape[1], order.S
    rows = max(128, ((N + 255) // 256 + 31) // 32 * 32)   # about 256 row tiles per species set
    ws_bytes = int(nat.lib().ictc_species_outer_workspace_bytes(N, C, S, rows))
    ws = torch.empty(max(ws_bytes, 16) // 4, dtype=torch.float32, device=a.device)
    out = a.new_empty(S, C, C)
    nat.call("ictc_species_outer", nat.ptr(a), a.stride(0), nat.ptr(b), b.stride(0), N, C, S, nat.ptr(order.perm),
             nat.ptr(order.off), rows, nat.ptr(out), nat.ptr(ws), ws_bytes, nat.stream_of(a))
    return out


class _SpeciesLinear(torch.autograd.Function):
    """y[n] = W[s_n] x[n] (trans: W[s_n]^T x[n]); the input adjoint is the other map, the weight gradient
    the per-species outer products (_SpeciesOuter)."""

    @staticmethod
    def forward(ctx, x, W, order, trans):
        ctx.order, ctx.trans = order, trans
        ctx.save_for_backward(x, W)
        return _species_apply(x, W, order, trans)

    @staticmethod
    def backward(ctx, g):
        x, W = ctx.saved_tensors
        needs = ctx.needs_input_grad
        if g is None or not (needs[0] or needs[1]):
            return None, None, None, None
        dx = _SpeciesLinear.apply(g, W, ctx.order, not ctx.trans) if needs[0] else None
        dW = None
        if needs[1]:
            dW = _SpeciesOuter.apply(x, g, ctx.order) if ctx.trans else _SpeciesOuter.apply(g, x, ctx.order)
        return dx, dW, None, None


class _SpeciesOuter(torch.autograd.Function):
    """out[s] = sum over the nodes n of species s of a[n] b[n]^T; adjoints a[n] <- H[s] b[n] and
    b[n] <- H[s]^T a[n] (the species linear and its transpose)."""

    @staticmethod
    def forward(ctx, a, b, order):
        ctx.order = order
        ctx.save_for_backward(a, b)
        return _species_outer_raw(a, b, order)

    @staticmethod
    def backward(ctx, H):
        a, b = ctx.saved_tensors
        if H is None:
            return None, None, None
        da = _SpeciesLinear.apply(b, H, ctx.order, False) if ctx.needs_input_grad[0] else None
        db = _SpeciesLinear.apply(a, H, ctx.order, True) if ctx.needs_input_grad[1] else None
        return da, db, None


class _SpeciesRows(torch.autograd.Function):
    """rows[n] = table[species[n]] (table [S, C]); the table gradient one_hot^T . drows runs on the
    split-reduction kernel in a fixed order (an index_select adjoint would add rows with atomics)."""

    @staticmethod
    def forward(ctx, table, species):
        ctx.save_for_backward(species)
        ctx.S = table.shape[0]
        return table.index_select(0, species)

    @staticmethod
    def backward(ctx, drows):
        from ictc_o3.ops.radial_mlp import _WeightGrad
        (species,) = ctx.saved_tensors
        if drows is None or not ctx.needs_input_grad[0]:
            return None, None
        onehot = torch.nn.functional.one_hot(species, ctx.S).to(drows.dtype)
        return _WeightGrad.apply(onehot, drows), None


def species_rows(table: torch.Tensor, species: torch.Tensor) -> torch.Tensor:
    """table[species] with a deterministic table gradient (node embedding, backbone.py:1016-1020)."""
    return _SpeciesRows.apply(table, species)


class _GraphSum(torch.autograd.Function):
    """out[b] = sum_{batch[n] == b} values[n] in FP64 (ictc_graph_sum: fixed order, no atomics); the adjoint
    is the gather grad[batch], differentiable to any order."""

    @staticmethod
    def forward(ctx, values, batch, graphs, batch_sorted):
        from ictc_o3 import _native as nat
        if values.dtype != torch.float32 or batch.dtype != torch.int64:
            raise TypeError("graph_sum: values must be float32 and batch int64")
        if values.shape != batch.shape:
            raise ValueError("graph_sum: values and batch must have the same shape [N]")
        values = values if values.is_contiguous() else values.contiguous()
        batch = batch if batch.is_contiguous() else batch.contiguous()
        out = torch.empty(graphs, dtype=torch.float64, device=values.device)
        nat.call("ictc_graph_sum", nat.ptr(values), nat.ptr(batch), values.numel(), graphs,
                 1 if batch_sorted else 0, nat.ptr(out),
                 nat.stream_of(values))
        ctx.save_for_backward(batch)
        ctx.dtype = values.dtype
        return out

    @staticmethod
    def backward(ctx, grad):
        (batch,) = ctx.saved_tensors
        return grad.index_select(0, batch).to(ctx.dtype), None, None, None


def graph_sum(values: torch.Tensor, batch: torch.Tensor, graphs: int, batch_sorted: bool = False) -> torch.Tensor:
    """Per-graph FP64 sums of float32 per-atom values (batch int64 graph ids in [0, graphs)).
    batch_sorted=True promises ascending ids (each graph's atoms contiguous) and makes the cost O(N + graphs)."""
    return _GraphSum.apply(values, batch, int(graphs), bool(batch_sorted))


def channel_linear(features: torch.Tensor, weight: torch.Tensor, bias=None):
    """[*, Cin, m] x [Cout, Cin] -> [*, Cout, m] (operators.py:609-628)."""
    angular = features.movedim(-2, -1).contiguous()
    out = torch.nn.functional.linear(angular.reshape(-1, weight.shape[1]), weight, bias)
    return out.reshape(*angular.shape[:-1], weight.shape[0]).movedim(-1, -2)


# ---------------------------------------------------------------------------
# MFMA kernel path (first derivatives): one launch per linear, reading the
# path-major degree blocks in place.
# ---------------------------------------------------------------------------
import ctypes

from ictc_o3 import _native as nat


_operand_cache = {}   # id(base) -> (weakref to base, {view key: contiguous operand})


def _weight_operand(w, transpose=False):
    """w (or w.t()) detached and contiguous, as the packed kernel reads it.  A non-contiguous view (the
    product linear's transposed blocks) or a transpose (the input adjoint) costs a copy launch; the copy is
    kept per live base tensor, view geometry and version counter (an optimizer step bumps the version), so
    a model whose weights do not change between steps makes it once."""
    import weakref
    v = w.detach().t() if transpose else w.detach()
    if v.is_contiguous():
        return v
    base = w._base if w._base is not None else w
    key = (v.storage_offset(), tuple(v.shape), tuple(v.stride()), w._version, v.dtype, v.device)
    entry = _operand_cache.get(id(base))
    if entry is None or entry[0]() is not base:
        if len(_operand_cache) > 256:
            for k in [k for k, (ref, _) in _operand_cache.items() if ref() is None]:
                del _operand_cache[k]
        entry = (weakref.ref(base), {})
        _operand_cache[id(base)] = entry
    views = entry[1]
    out = views.get(key)
    if out is None:
        if len(views) > 64:
            views.clear()
        out = v.contiguous()
        views[key] = out
    return out


def _packed_call(x, Ci, Co, lmax, pin, in_off, pout, out_off, weights, scales, out_cols):
    N = x.shape[0]
    out = x.new_empty(N, out_cols)
    L = lmax + 1
    ip, op = (ctypes.c_int * L)(*pin), (ctypes.c_int * L)(*pout)
    io, oo = (ctypes.c_int64 * L)(*in_off), (ctypes.c_int64 * L)(*out_off)
    ws = (ctypes.c_void_p * L)(*[w.data_ptr() for w in weights])
    sc = (ctypes.c_float * L)(*scales)
    nat.call("ictc_packed_linear", lmax, Ci, Co, nat.ptr(x), x.stride(0), ip, io, nat.ptr(out), out.stride(0), op,
             oo, ws, sc, N, nat.stream_of(x))
    return out


class _PackedLinear(torch.autograd.Function):
    """out = packed linear of x (first derivatives; weight gradients by einsum when required)."""

    @staticmethod
    def forward(ctx, x, layout, *weights):
        lmax, Ci, Co, pin, in_off, out_off, scales, in_cols = layout
        ctx.layout = layout
        ctx.inputs = (x, *weights)
        x = x if x.is_contiguous() else x.contiguous()
        ws = [_weight_operand(w) for w in weights]
        ctx.save_for_backward(x, *ws)
        return _packed_call(x, Ci, Co, lmax, pin, in_off, [1] * (lmax + 1), out_off, ws, scales,
                            (lmax + 1) ** 2 * Co)

    @staticmethod
    def backward(ctx, dout):
        from ictc_o3.autograd import required_gradients
        if torch.is_grad_enabled():
            raise RuntimeError("the MFMA linear path is first-order; build the model with second_order=True")
        x, *ws = ctx.saved_tensors
        needs = required_gradients(ctx.inputs, ctx.needs_input_grad[:1] + ctx.needs_input_grad[2:])
        ctx.inputs = None
        dx, dws = _packed_adjoint(x, ws, ctx.layout, dout, needs)
        return (dx, None, *dws)


def _packed_adjoint(x, ws, layout, dout, needs):
    """Input adjoint (needs[0]) and weight gradients (needs[1:]) of the packed linear for cotangent dout."""
    lmax, Ci, Co, pin, in_off, out_off, scales, in_cols = layout
    dout = dout if dout.is_contiguous() else dout.contiguous()
    dx = None
    if needs[0]:
        wt = [_weight_operand(w, transpose=True) for w in ws]
        dx = _packed_call(dout, Co, Ci, lmax, [1] * (lmax + 1), out_off, pin, in_off, wt, scales, in_cols)
    dws = []
    N = x.shape[0]
    for l, (w, need) in enumerate(zip(ws, needs[1:])):
        if not need:
            dws.append(None)
            continue
        k, m = pin[l], 2 * l + 1
        xin = x[:, in_off[l]:in_off[l] + k * m * Ci].reshape(N, k, m, Ci).transpose(1, 2).reshape(N * m, k * Ci)
        dl = dout[:, out_off[l]:out_off[l] + m * Co].reshape(N * m, Co)
        # dW[o, (k, c)] = sum_{n, m} dl[n, m, o] x[n, k, m, c] on the split-reduction kernel
        from ictc_o3.ops.radial_mlp import weight_grad
        dws.append(scales[l] * weight_grad(dl, xin))
    return dx, dws


class _LayerEntry(torch.autograd.Function):
    """(degree linear of h, h[:, :C] as a contiguous [N, C] copy) for first-order callers.

    The scalar columns of a layer's input feed the self connection and the
    previous layer's energy readout; taken as slices, each slice's backward
    would zero-fill a full [N, (L+1)^2 C] gradient and autograd would add the
    full tensors.  Here the backward forms the linear's input adjoint and adds
    the scalar columns' (small) gradient into its first C columns in place.
    """

    @staticmethod
    def forward(ctx, h, layout, C, *weights):
        lmax, Ci, Co, pin, in_off, out_off, scales, in_cols = layout
        ctx.layout, ctx.C = layout, C
        ctx.inputs = (h, *weights)
        x = h if h.is_contiguous() else h.contiguous()
        ws = [_weight_operand(w) for w in weights]
        ctx.save_for_backward(x, *ws)
        y = _packed_call(x, Ci, Co, lmax, pin, in_off, [1] * (lmax + 1), out_off, ws, scales, (lmax + 1) ** 2 * Co)
        return y, x[:, :C].contiguous()

    @staticmethod
    def backward(ctx, dy, ds):
        from ictc_o3.autograd import required_gradients
        if torch.is_grad_enabled():
            raise RuntimeError("the MFMA linear path is first-order; build the model with second_order=True")
        x, *ws = ctx.saved_tensors
        needs = required_gradients(ctx.inputs, ctx.needs_input_grad[:1] + ctx.needs_input_grad[3:])
        ctx.inputs = None
        if dy is None:
            dy = torch.zeros(x.shape[0], (ctx.layout[0] + 1) ** 2 * ctx.layout[2], dtype=x.dtype, device=x.device)
        dx, dws = _packed_adjoint(x, ws, ctx.layout, dy, needs)
        if dx is not None and ds is not None:
            dx[:, :ctx.C] += ds      # dx is this backward's own fresh tensor
        return (dx, None, None, *dws)


def layer_entry_fast(h, weights, C, lmax):
    """(degree_linear(h), h[:, :C]) on the MFMA kernel with a fused input adjoint (first derivatives only)."""
    if not _fast_ok(h, weights, C) or h.shape[1] == C:
        return None
    Co = weights[0].shape[0]
    layout = (lmax, C, Co, [1] * (lmax + 1), [l * l * C for l in range(lmax + 1)],
              [l * l * Co for l in range(lmax + 1)], [1.0] * (lmax + 1), (lmax + 1) ** 2 * C)
    return _LayerEntry.apply(h, layout, C, *weights[:lmax + 1])


class _AddScalars(torch.autograd.Function):
    """out[:, :C] += s in place on a fresh tensor no backward saves; the gradient passes through without
    the full-size clone an in-place slice update records (first-order callers)."""

    @staticmethod
    def forward(ctx, out, s):
        C = s.shape[1]
        out[:, :C] += s
        ctx.mark_dirty(out)
        ctx.C = C
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, g):
        return g, (None if g is None else g[:, :ctx.C].contiguous())


def add_scalars_(out, s):
    return _AddScalars.apply(out, s)


class _AddScalarsAny(torch.autograd.Function):
    """out[:, :C] += s in place on a fresh tensor, differentiable to any order: the gradient passes through
    and s's is the contiguous take of its first C columns (_TakeScalars), where an in-place slice update
    records a full-size clone and, differentiated again, a zero-filled as_strided gradient."""

    @staticmethod
    def forward(ctx, out, s):
        C = s.shape[1]
        out[:, :C] += s
        ctx.mark_dirty(out)
        ctx.C = C
        return out

    @staticmethod
    def backward(ctx, g):
        if g is None:
            return None, None
        return g, _TakeScalars.apply(g, ctx.C)


class _TakeScalars(torch.autograd.Function):
    """x[:, :C] as a contiguous [N, C] tensor; the adjoint writes the (small) gradient into the first C
    columns of a zero [N, W] tensor (_PadScalars), whose adjoint is this take again."""

    @staticmethod
    def forward(ctx, x, C):
        ctx.W, ctx.C = x.shape[1], C
        return x[:, :C].contiguous()

    @staticmethod
    def backward(ctx, g):
        return (None if g is None else _PadScalars.apply(g, ctx.W)), None


class _PadScalars(torch.autograd.Function):
    @staticmethod
    def forward(ctx, s, W):
        ctx.C = s.shape[1]
        out = s.new_zeros(s.shape[0], W)
        out[:, :ctx.C] = s
        return out

    @staticmethod
    def backward(ctx, g):
        return (None if g is None else _TakeScalars.apply(g, ctx.C)), None


def add_scalars_any_(out, s):
    """out[:, :C] += s (C = s.shape[1]) in place on a fresh tensor nothing else holds, any derivative order."""
    return _AddScalarsAny.apply(out, s)


def take_scalars(x, C):
    """x[:, :C] as a contiguous copy with a single-node adjoint (any derivative order); x itself when it has
    only C columns."""
    return x if x.shape[1] == C else _TakeScalars.apply(x, C)


def _fast_ok(x, weights, C):
    return (x.is_cuda and x.dtype == torch.float32 and C % 16 == 0 and len(weights) <= 4
            and all(w.numel() > 0 and w.dtype == torch.float32 for w in weights))


class _PackedLinearAny(torch.autograd.Function):
    """The packed linear, differentiable to any order (second-order callers: force-loss training).

    layout = (lmax, Ci, Co, pin, in_off, pout, out_off, scales, out_cols): degree l maps pin[l] input paths
    of Ci channels to pout[l] output paths of Co channels with W_l [pout Co, pin Ci].  The input adjoint
    is the same map with W_l^T (itself a _PackedLinearAny, so its derivative is this map again); the
    weight gradient dW_l = scale_l * dout_l^T x_l over the (node, component) rows runs on the
    split-reduction kernel (_WeightGrad, differentiable in both operands).  One launch per map instead
    of one GEMM per degree, and no split / concatenation of the packed rows.
    """

    @staticmethod
    def forward(ctx, x, layout, *weights):
        lmax, Ci, Co, pin, in_off, pout, out_off, scales, out_cols = layout
        ctx.layout = layout
        x = x if x.is_contiguous() else x.contiguous()
        ctx.save_for_backward(x, *weights)
        ws = [_weight_operand(w) for w in weights]
        return _packed_call(x, Ci, Co, lmax, pin, in_off, pout, out_off, ws, scales, out_cols)

    @staticmethod
    def backward(ctx, dout):
        from ictc_o3.autograd import required_gradients
        from ictc_o3.ops.radial_mlp import _WeightGrad
        x, *ws = ctx.saved_tensors
        lmax, Ci, Co, pin, in_off, pout, out_off, scales, out_cols = ctx.layout
        needs = required_gradients((x, *ws), ctx.needs_input_grad[:1] + ctx.needs_input_grad[2:])
        if dout is None or not any(needs):
            return (None, None) + (None,) * len(ws)
        dout = dout if dout.is_contiguous() else dout.contiguous()
        dx = None
        if needs[0]:
            layout_t = (lmax, Co, Ci, pout, out_off, pin, in_off, scales, x.shape[1])
            dx = _PackedLinearAny.apply(dout, layout_t, *[w.t() for w in ws])
        N, dws = x.shape[0], []
        direct = not torch.is_grad_enabled() and x.is_cuda and x.dtype == dout.dtype == torch.float32
        for l, need in enumerate(needs[1:]):
            if not need:
                dws.append(None)
                continue
            m = 2 * l + 1
            if direct:
                # no graph to build: the kernel reads the (node, component) rows of both blocks in place
                dws.append(scales[l] * _degree_weight_grad(dout, out_off[l], pout[l], Co, x, in_off[l], pin[l],
                                                           Ci, m))
                continue
            xin = x[:, in_off[l]:in_off[l] + pin[l] * m * Ci].reshape(N, pin[l], m, Ci).transpose(1, 2) \
                .reshape(N * m, pin[l] * Ci)
            dl = dout[:, out_off[l]:out_off[l] + pout[l] * m * Co].reshape(N, pout[l], m, Co).transpose(1, 2) \
                .reshape(N * m, pout[l] * Co)
            dws.append(scales[l] * _WeightGrad.apply(dl, xin))
        return (dx, None, *dws)


def _degree_weight_grad(dout, out_off, pout, Co, x, in_off, pin, Ci, m):
    """dout_l^T x_l [pout Co, pin Ci] over the (node, component) rows of one degree's packed blocks
    (ictc_gemm_tn_grouped), without rearranging them into [N m, paths C] copies."""
    N = x.shape[0]
    M, K = pout * Co, pin * Ci
    out = x.new_empty(M, K)
    ws_bytes = int(nat.lib().ictc_gemm_tn_workspace_bytes(N * m, M, K))
    if ws_bytes < 0:
        raise ValueError("degree weight gradient: unsupported shape")
    ws = torch.empty(max(ws_bytes, 16) // 4, dtype=torch.float32, device=x.device)
    nat.call("ictc_gemm_tn_grouped", ctypes.c_void_p(dout.data_ptr() + 4 * out_off), dout.stride(0), Co, Co, m * Co,
             ctypes.c_void_p(x.data_ptr() + 4 * in_off), x.stride(0), Ci, Ci, m * Ci, N, m, M, K, nat.ptr(out),
             nat.ptr(ws), ws_bytes, nat.stream_of(x))
    return out


def degree_linear_any(x, weights, C, lmax, scale=1.0):
    """degree_linear on the packed kernel, differentiable to any order (composable form where it does
    not apply)."""
    if not _fast_ok(x, weights, C) or weights[0].shape[0] % 16:
        return degree_linear(x, weights, C, lmax, scale)
    Co = weights[0].shape[0]
    layout = (lmax, C, Co, [1] * (lmax + 1), [l * l * C for l in range(lmax + 1)], [1] * (lmax + 1),
              [l * l * Co for l in range(lmax + 1)], [float(scale)] * (lmax + 1), (lmax + 1) ** 2 * Co)
    return _PackedLinearAny.apply(x, layout, *weights[:lmax + 1])


def path_linear_any(m, weights, counts, C, lmax, scale=1.0):
    """path_linear on the packed kernel, differentiable to any order (composable form where it does not
    apply)."""
    if not _fast_ok(m, weights, C) or weights[0].shape[0] % 16 or any(counts.get(l, 0) == 0 for l in range(lmax + 1)):
        return path_linear(m, weights, counts, C, lmax, scale)
    Co = weights[0].shape[0]
    pin, in_off, off = [], [], 0
    for l in range(lmax + 1):
        pin.append(counts[l])
        in_off.append(off)
        off += counts[l] * (2 * l + 1) * C
    if off != m.shape[1]:
        return path_linear(m, weights, counts, C, lmax, scale)
    layout = (lmax, C, Co, pin, in_off, [1] * (lmax + 1), [l * l * Co for l in range(lmax + 1)],
              [float(scale)] * (lmax + 1), (lmax + 1) ** 2 * Co)
    return _PackedLinearAny.apply(m, layout, *weights[:lmax + 1])


def degree_linear_fast(x, weights, C, lmax, scale=1.0):
    """degree_linear on the MFMA kernel (first derivatives only)."""
    if not _fast_ok(x, weights, C):
        return degree_linear(x, weights, C, lmax, scale)
    Co = weights[0].shape[0]
    layout = (lmax, C, Co, [1] * (lmax + 1), [l * l * C for l in range(lmax + 1)],
              [l * l * Co for l in range(lmax + 1)], [float(scale)] * (lmax + 1), (lmax + 1) ** 2 * C)
    return _PackedLinear.apply(x, layout, *weights[:lmax + 1])


def path_linear_fast(m, weights, counts, C, lmax, scale=1.0):
    """path_linear on the MFMA kernel (first derivatives only)."""
    if not _fast_ok(m, weights, C) or any(counts.get(l, 0) == 0 for l in range(lmax + 1)):
        return path_linear(m, weights, counts, C, lmax, scale)
    Co = weights[0].shape[0]
    pin, in_off, off = [], [], 0
    for l in range(lmax + 1):
        pin.append(counts[l])
        in_off.append(off)
        off += counts[l] * (2 * l + 1) * C
    layout = (lmax, C, Co, pin, in_off, [l * l * Co for l in range(lmax + 1)], [float(scale)] * (lmax + 1), off)
    return _PackedLinear.apply(m, layout, *weights[:lmax + 1])
