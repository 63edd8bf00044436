"""Radial MLP of the interaction blocks with a fused HIP kernel for its hidden layers.

fc = Linear(8,64) -> SiLU*s -> Linear(64,64) -> SiLU*s -> Linear(64,64) -> SiLU*s -> Linear(64, P*C)
on the radial basis of the edge lengths (mace_ictc/models/mace/layers.py:826-835,
radial_basis.py:11-92).  ``radial_gates`` runs the radial basis, the three
hidden layers and the 64 -> P*C gate projection in one MFMA kernel (the hidden
activations stay on chip); its adjoint runs the
projection's hidden-layer adjoint on a second split-bf16 kernel and fuses the
hidden-layer backward down to d/dr.  It supports first derivatives (forces,
first-order parameter gradients).  Callers that need second derivatives
(force-loss training) use ``radial_mlp_lengths``: the hidden layers through
``radial_hidden`` (forward, first adjoint and its derivative on fused kernels,
higher orders composed from torch operations) and the gate projection as an
``edge_linear``.  ``radial_mlp`` is the fully composable form on a given radial
basis.  The Linears take their weight gradients dW = dy^T x from a
split-reduction MFMA kernel (``ictc_gemm_tn``) instead of a library GEMM that
tiles only the small output.
"""
from __future__ import annotations

import ctypes
import math

import torch
from torch.autograd.function import once_differentiable

from ictc_o3 import _native as nat
from ictc_o3 import _timing


def _c(t):
    return t if t.is_contiguous() else t.contiguous()


def gate_projection(h: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """h [E, 64] . W^T ([M, 64], M a multiple of 16) on the split-bf16 MFMA kernel (FP32-level accuracy)."""
    E, M = h.shape[0], W.shape[0]
    if h.dim() != 2 or h.shape[1] != 64 or W.shape[1] != 64 or M % 16:
        raise ValueError("gate projection needs h [E, 64] and W [M, 64] with M a multiple of 16")
    h, W = _c(h), _c(W)
    out = h.new_empty(E, M)
    nat.call("ictc_gate_gemm_fwd", nat.ptr(h), E, 64, nat.ptr(W), M, nat.ptr(out), nat.stream_of(h))
    return out


def gate_projection_adjoint(dg: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """dg [E, M] . W ([M, 64]) on the split-bf16 MFMA kernel when M is a multiple of 64 up to 768."""
    E, M = dg.shape[0], W.shape[0]
    if dg.dim() != 2 or dg.shape[1] != M or W.shape[1] != 64:
        raise ValueError("gate adjoint needs dg [E, M] and W [M, 64]")
    if M % 64:
        return gemm_nt(dg, W.t())   # outside the split-bf16 kernel's column blocks: FP32 MFMA
    dg, W = _c(dg), _c(W)
    out = dg.new_empty(E, 64)
    # column blocks of at most 768 gates (the kernel's register budget), accumulated in column order
    for c0 in range(0, M, 768):
        mc = min(768, M - c0)
        nat.call("ictc_gate_gemm_bwd_strided", ctypes.c_void_p(dg.data_ptr() + 4 * c0), M, E, mc,
                 ctypes.c_void_p(W.data_ptr() + 4 * c0 * 64), 64, nat.ptr(out), int(c0 > 0), nat.stream_of(dg))
    return out


_TN_MIN_ROWS = 16384   # below this the library GEMM's output tiling is enough


def gemm_nt(x: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """x [M, K] . W^T ([N, K]) on the FP32-MFMA channel-linear kernel (ictc_gemm_nt)."""
    if x.stride(-1) != 1:
        x = x.contiguous()
    W = _c(W.detach())
    M, K, N = x.shape[0], x.shape[1], W.shape[0]
    out = x.new_empty(M, N)
    nat.call("ictc_gemm_nt", nat.ptr(x), M, K, x.stride(0), nat.ptr(W), N, K, nat.ptr(out), N, 0,
             nat.stream_of(x))
    return out


def _own_gemm(x: torch.Tensor) -> bool:
    return x.is_cuda and x.dtype == torch.float32 and x.dim() == 2


def _gemm_tn(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a [K, M], b [K, N] -> a^T b [M, N] on the split-reduction MFMA kernel (deterministic)."""
    a, b = _c(a.detach()), _c(b.detach())
    K, M = a.shape
    N = b.shape[1]
    out = a.new_empty(M, N)
    ws_bytes = int(nat.lib().ictc_gemm_tn_workspace_bytes(K, M, N))
    if ws_bytes < 0:
        raise ValueError("gemm_tn: unsupported shape")
    ws = torch.empty(max(ws_bytes, 16) // 4, dtype=torch.float32, device=a.device)
    nat.call("ictc_gemm_tn", nat.ptr(a), K, M, M, nat.ptr(b), N, N, nat.ptr(out), nat.ptr(ws), ws_bytes,
             nat.stream_of(a))
    return out


def weight_grad(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a^T b over rows on the split-reduction kernel (FP32 MFMA up to 16 output tiles of 64 x 64,
    split-bf16 MFMA beyond; chunk partials added in a fixed order, so the result is bitwise repeatable)."""
    if a.is_cuda and a.dtype == torch.float32 and b.dtype == torch.float32:
        return _gemm_tn(a, b)
    return a.t() @ b


class _WeightGrad(torch.autograd.Function):
    """a^T b over edge rows (a weight gradient); differentiable in a and b."""

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return weight_grad(a, b)

    @staticmethod
    def backward(ctx, h):
        a, b = ctx.saved_tensors
        if _own_gemm(a) and _own_gemm(b):
            h = _c(h)
            da = _EdgeLinear.apply(b, h) if ctx.needs_input_grad[0] else None        # b h^T
            db = _EdgeLinearT.apply(a, h) if ctx.needs_input_grad[1] else None       # a h
            return da, db
        da = b @ h.t() if ctx.needs_input_grad[0] else None
        db = a @ h if ctx.needs_input_grad[1] else None
        return da, db


class _EdgeLinear(torch.autograd.Function):
    """y = x W^T over edge rows; the weight gradient runs on the split-reduction kernel."""

    @staticmethod
    def forward(ctx, x, W):
        ctx.save_for_backward(x, W)
        ctx.inputs = (x, W)
        if x.is_cuda and x.shape[0] >= _TN_MIN_ROWS and x.shape[1] == 64 and W.shape[0] % 16 == 0:
            return gate_projection(x, W)   # split-bf16 MFMA, FP32-level accuracy (hidden layers and projection)
        if _own_gemm(x):
            return gemm_nt(x, W)
        return x @ W.t()

    @staticmethod
    def backward(ctx, g):
        from ictc_o3.autograd import required_gradients
        x, W = ctx.saved_tensors
        needs = required_gradients(ctx.inputs, ctx.needs_input_grad) if ctx.inputs else ctx.needs_input_grad
        ctx.inputs = None
        dx = _EdgeLinearT.apply(g, W) if needs[0] else None
        dW = _WeightGrad.apply(g, x) if needs[1] else None
        return dx, dW


class _EdgeLinearT(torch.autograd.Function):
    """z = u W over edge rows (the input adjoint of _EdgeLinear), differentiable in u and W."""

    @staticmethod
    def forward(ctx, u, W):
        ctx.save_for_backward(u, W)
        ctx.inputs = (u, W)
        M = W.shape[0]
        if u.is_cuda and u.shape[0] >= _TN_MIN_ROWS and W.shape[1] == 64 and M % 64 == 0:
            return gate_projection_adjoint(u, W)   # split-bf16 MFMA, FP32-level accuracy
        if _own_gemm(u):
            return gemm_nt(u, W.t())
        return u @ W

    @staticmethod
    def backward(ctx, h):
        from ictc_o3.autograd import required_gradients
        u, W = ctx.saved_tensors
        needs = required_gradients(ctx.inputs, ctx.needs_input_grad) if ctx.inputs else ctx.needs_input_grad
        ctx.inputs = None
        du = _EdgeLinear.apply(h, W) if needs[0] else None
        dW = _WeightGrad.apply(u, h) if needs[1] else None
        return du, dW


def edge_linear(x: torch.Tensor, W: torch.Tensor) -> torch.Tensor:
    """x [E, in] . W^T ([out, in], nn.Linear layout) with weight gradients on the split-reduction kernel.

    Same values as torch.nn.functional.linear without bias; every derivative
    order is supported (the adjoints are built from the same two operators).
    """
    if x.dim() != 2 or W.dim() != 2 or x.shape[1] != W.shape[1]:
        raise ValueError("edge_linear needs x [E, in] and W [out, in]")
    return _EdgeLinear.apply(x, W)


def radial_mlp(radial: torch.Tensor, fc: torch.nn.Sequential) -> torch.Tensor:
    """fc(radial) with its bias-free Linears as edge_linear (the composable, any-order path)."""
    h = radial
    for m in fc:
        if isinstance(m, torch.nn.Linear) and m.bias is None:
            h = edge_linear(h, m.weight)
        else:
            h = m(h)
    return h


class _RadialGates(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, W1, W2, W3, W4, cutoff, poly_p, scale):
        ctx.inputs = (r, W1, W2, W3, W4) if r.requires_grad or W1.requires_grad else None
        r = _c(r)
        W1, W2, W3, W4 = (_c(w.detach()) for w in (W1, W2, W3, W4))
        E, M = r.shape[0], W4.shape[0]
        # MLP and projection in one kernel: the hidden activation never goes to HBM
        gates = r.new_empty(E, M)
        ws_bytes = int(nat.lib().ictc_radial_gates_workspace_bytes(M))
        ws = torch.empty(max(ws_bytes, 16) // 4, dtype=torch.float32, device=r.device)
        nat.call("ictc_radial_gates_fwd", nat.ptr(r), E, 8, 64, float(cutoff), int(poly_p), nat.ptr(W1),
                 nat.ptr(W2), nat.ptr(W3), nat.ptr(W4), M, float(scale), nat.ptr(gates), nat.ptr(ws), ws_bytes,
                 nat.stream_of(r))
        ctx.cfg = (cutoff, poly_p, scale)
        ctx.save_for_backward(r, W1, W2, W3, W4)
        return gates

    @staticmethod
    @once_differentiable
    def backward(ctx, dg):
        r, W1, W2, W3, W4 = ctx.saved_tensors
        from ictc_o3.autograd import required_gradients
        needs = required_gradients(ctx.inputs, ctx.needs_input_grad[:5]) if ctx.inputs else ctx.needs_input_grad[:5]
        ctx.inputs = None
        dr, dW = radial_gates_adjoint(r, (W1, W2, W3, W4), ctx.cfg, _c(dg), needs)
        return (dr, *dW, None, None, None)


def radial_gates_adjoint(r, weights, cfg, dg, needs):
    """Adjoint of the fused radial gates for cotangent dg [E, M]: (dr or None, [dW1..dW4 or None])."""
    W1, W2, W3, W4 = weights
    cutoff, poly_p, scale = cfg
    E = r.shape[0]
    need_w = any(needs[1:5])
    da3 = gate_projection_adjoint(dg, W4)
    dr = r.new_empty(E)
    extra = [r.new_empty(E, 64) for _ in range(5)] if need_w else [None] * 5   # dz1, dz2, dz3, a1, a2
    nat.call("ictc_radial_mlp_bwd", nat.ptr(r), E, 8, 64, float(cutoff), int(poly_p), nat.ptr(W1), nat.ptr(W2),
             nat.ptr(W3), float(scale), nat.ptr(da3), nat.ptr(dr), *[nat.ptr(t) for t in extra],
             nat.stream_of(r))
    dW = [None] * 4
    if need_w:
        from ictc_o3.ops.activation import _radial
        dz1, dz2, dz3, a1, a2 = extra
        a3 = r.new_empty(E, 64)   # recomputed: the forward kept it on chip
        nat.call("ictc_radial_mlp_fwd", nat.ptr(r), E, 8, 64, float(cutoff), int(poly_p), nat.ptr(W1),
                 nat.ptr(W2), nat.ptr(W3), float(scale), nat.ptr(a3), nat.stream_of(r))
        R = _radial(0, r, None, None, 8, cutoff, poly_p)
        dW = [weight_grad(dz1, R), weight_grad(dz2, a1), weight_grad(dz3, a2), weight_grad(dg, a3)]
    return (dr if needs[0] else None), [d if n else None for d, n in zip(dW, needs[1:5])]


def radial_gates_tangent(r, weights, cutoff, poly_p, scale):
    """Fused radial gates [E, M] and their derivative along r, d gates / dr [E, M] (no autograd)."""
    W1, W2, W3, W4 = (_c(w.detach()) for w in weights)
    r = _c(r.detach())
    E, M = r.shape[0], W4.shape[0]
    gates, gdot = r.new_empty(E, M), r.new_empty(E, M)
    ws_bytes = int(nat.lib().ictc_radial_gates_workspace_bytes(M))
    ws = torch.empty(max(ws_bytes, 16) // 4, dtype=torch.float32, device=r.device)
    tok = _timing.begin(f"gates_tan[M{M}]")
    nat.call("ictc_radial_gates_tangent_fwd", nat.ptr(r), E, 8, 64, float(cutoff), int(poly_p), nat.ptr(W1),
             nat.ptr(W2), nat.ptr(W3), nat.ptr(W4), M, float(scale), nat.ptr(gates), nat.ptr(gdot), nat.ptr(ws),
             ws_bytes, nat.stream_of(r))
    _timing.end(tok)
    return gates, gdot


def fused_supported(fc: torch.nn.Sequential) -> bool:
    """True when fc is Linear(8,64), act, Linear(64,64), act, Linear(64,64), act, Linear(64, M) without biases."""
    lin = [m for m in fc if isinstance(m, torch.nn.Linear)]
    if len(lin) != 4 or any(m.bias is not None for m in lin):
        return False
    return (tuple(lin[0].weight.shape) == (64, 8) and tuple(lin[1].weight.shape) == (64, 64)
            and tuple(lin[2].weight.shape) == (64, 64) and lin[3].weight.shape[1] == 64
            and lin[3].weight.shape[0] % 16 == 0)


def radial_gates(r: torch.Tensor, fc: torch.nn.Sequential, cutoff: float, poly_p: int, scale: float,
                 basis_scale: float = 1.0):
    """[E] edge lengths -> [E, P*C] gates through the fused kernel (first derivatives only).

    basis_scale multiplies the radial basis (the historical sqrt(num_basis) norm,
    radial_basis.py:87-91); it is folded into the first Linear's weight."""
    lin = [m for m in fc if isinstance(m, torch.nn.Linear)]
    W1 = lin[0].weight if basis_scale == 1.0 else lin[0].weight * basis_scale
    return _RadialGates.apply(r, W1, lin[1].weight, lin[2].weight, lin[3].weight, float(cutoff),
                              int(poly_p), float(scale))


# ---- hidden layers with first and second derivatives on the fused kernels ----------------------------------

class EdgeLengths:
    """Radial input of an interaction block that runs fc's hidden layers on the fused kernels to second order
    (radial_hidden) instead of taking a materialised radial basis; the lengths themselves are the block's r."""
    __slots__ = ()


def hidden_supported(fc: torch.nn.Sequential, r: torch.Tensor) -> bool:
    return fused_supported(fc) and r.is_cuda and r.dtype == torch.float32


def radial_mlp_lengths(r: torch.Tensor, fc: torch.nn.Sequential, cutoff: float, poly_p: int, scale: float,
                       basis_scale: float = 1.0) -> torch.Tensor:
    """fc(radial_embedding(r) * basis_scale) with the hidden layers on the fused kernels (radial_hidden) and
    the gate projection as edge_linear; differentiable to any order (second order on the fused kernels)."""
    lin = [m for m in fc if isinstance(m, torch.nn.Linear)]
    W1 = lin[0].weight if basis_scale == 1.0 else lin[0].weight * basis_scale
    h3 = radial_hidden(r, W1, lin[1].weight, lin[2].weight, cutoff, poly_p, scale)
    return edge_linear(h3, lin[3].weight)


def radial_hidden(r, W1, W2, W3, cutoff: float, poly_p: int, scale: float) -> torch.Tensor:
    """h3 [E, 64] = s silu(W3 s silu(W2 s silu(W1 R(r)))) with R the Bessel x polynomial-cutoff basis
    (8 functions, radial_basis.py:11-92): the forward, the first adjoint and its derivative (the force-loss
    second derivative) on the fused kernels; third and higher orders on composed torch operations."""
    if r.dim() != 1 or tuple(W1.shape) != (64, 8) or tuple(W2.shape) != (64, 64) or tuple(W3.shape) != (64, 64):
        raise ValueError("radial_hidden needs r [E] and weights [64, 8], [64, 64], [64, 64]")
    return _Hidden.apply(r, W1, W2, W3, float(cutoff), int(poly_p), float(scale))


def _hidden_torch(r, W1, W2, W3, cutoff, poly_p, scale):
    """The same function on plain torch operations (any derivative order)."""
    rr = r.unsqueeze(-1)
    k = torch.arange(1, 9, device=r.device, dtype=r.dtype)
    u = rr / cutoff
    p = poly_p
    env = (1.0 - 0.5 * (p + 1) * (p + 2) * u ** p + p * (p + 2) * u ** (p + 1) - 0.5 * p * (p + 1) * u ** (p + 2))
    env = env * (rr < cutoff).to(r.dtype)
    h = math.sqrt(2.0 / cutoff) * torch.sin(k * math.pi * rr / cutoff) / rr.clamp(min=1e-12) * env
    for W in (W1, W2, W3):
        h = torch.nn.functional.silu(h @ W.t()) * scale
    return h


def _hidden_weight_grads(rows, needs):
    """d W1..W3 from the kernel's weight-gradient rows: (z1, b), (z2, a1), (z3, a2) pairs over the same rows."""
    z1, b, z2, a1, z3, a2 = rows
    return [weight_grad(z1, b) if needs[0] else None, weight_grad(z2, a1) if needs[1] else None,
            weight_grad(z3, a2) if needs[2] else None]


def _hidden_adjoint(r, Ws, cfg, u, needs):
    """First adjoint for cotangent u [E, 64]: (dr or None, [dW1, dW2, dW3] or None entries)."""
    cutoff, poly_p, scale = cfg
    r, u = _c(r.detach()), _c(u.detach())
    W1, W2, W3 = (_c(w.detach()) for w in Ws)
    E = r.shape[0]
    need_w = any(needs[1:4])
    dr = r.new_empty(E)
    extra = [r.new_empty(E, 64) for _ in range(5)] if need_w else [None] * 5   # dz1, dz2, dz3, a1, a2
    nat.call("ictc_radial_mlp_bwd", nat.ptr(r), E, 8, 64, float(cutoff), int(poly_p), nat.ptr(W1), nat.ptr(W2),
             nat.ptr(W3), float(scale), nat.ptr(u), nat.ptr(dr), *[nat.ptr(t) for t in extra], nat.stream_of(r))
    dW = [None] * 3
    if need_w:
        from ictc_o3.ops.activation import _radial
        dz1, dz2, dz3, a1, a2 = extra
        R = _radial(0, r, None, None, 8, cutoff, poly_p)
        dW = _hidden_weight_grads((dz1, R, dz2, a1, dz3, a2), needs[1:4])
    return (dr if needs[0] else None), dW


# Whether the derivative of the hidden layers' first adjoint (the force pass) hands its cotangent to the
# forward node's first adjoint in the same backward pass, so that one kernel launch returns the sum of both
# (ictc_radial_mlp_bwd2 with v); False = two launches added by autograd.
LINK_HIDDEN = True


def _hidden_second(r, Ws, cfg, u, rho, v, needs, want_du=False):
    """ictc_radial_mlp_bwd2 for inputs (r, W1, W2, W3): (dr, [dW1, dW2, dW3]) of rho . d<u, a3>/dr, plus the
    first adjoint for cotangent v (nullable) on a3, and d u = rho t3 when want_du (else None)."""
    cutoff, poly_p, scale = cfg
    rc, uc, rh = _c(r.detach()), _c(u.detach()), _c(rho.detach())
    vc = None if v is None else _c(v.detach())
    W1, W2, W3 = (_c(w.detach()) for w in Ws)
    E = rc.shape[0]
    need_w = any(needs[1:4])
    d_r = rc.new_empty(E)
    rows = [rc.new_empty(2 * E, 64) for _ in range(5)] + [rc.new_empty(2 * E, 8)] if need_w else [None] * 6
    z3, a2, z2, a1, z1, b = rows
    d_u = rc.new_empty(E, 64) if want_du else None
    nat.call("ictc_radial_mlp_bwd2", nat.ptr(rc), E, 8, 64, float(cutoff), int(poly_p), nat.ptr(W1), nat.ptr(W2),
             nat.ptr(W3), float(scale), nat.ptr(uc), nat.ptr(rh), nat.ptr(vc), nat.ptr(d_r), nat.ptr(d_u),
             *[nat.ptr(t) for t in rows], nat.stream_of(rc))
    dW = _hidden_weight_grads((z1, b, z2, a1, z3, a2), needs[1:4]) if need_w else [None] * 3
    return (d_r if needs[0] else None), dW, d_u


def _hidden_tangent_cotangent(r, Ws, cfg, u, rho):
    """d u = rho t3 alone (ictc_radial_mlp_bwd2 without dr)."""
    cutoff, poly_p, scale = cfg
    rc, uc, rh = _c(r.detach()), _c(u.detach()), _c(rho.detach())
    W1, W2, W3 = (_c(w.detach()) for w in Ws)
    d_u = rc.new_empty(rc.shape[0], 64)
    nat.call("ictc_radial_mlp_bwd2", nat.ptr(rc), rc.shape[0], 8, 64, float(cutoff), int(poly_p), nat.ptr(W1),
             nat.ptr(W2), nat.ptr(W3), float(scale), nat.ptr(uc), nat.ptr(rh), None, None, nat.ptr(d_u),
             *([None] * 6), nat.stream_of(rc))
    return d_u


class _Hidden(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, W1, W2, W3, cutoff, poly_p, scale):
        from ictc_o3.ops.tensor_product import _GateLink
        ctx.cfg = (cutoff, poly_p, scale)
        ctx.link = _GateLink(ctx, "cotangent of the radial MLP's second derivative", lambda: LINK_HIDDEN)
        rc = _c(r.detach())
        Ws = [_c(w.detach()) for w in (W1, W2, W3)]
        h3 = rc.new_empty(rc.shape[0], 64)
        nat.call("ictc_radial_mlp_fwd", nat.ptr(rc), rc.shape[0], 8, 64, float(cutoff), int(poly_p),
                 nat.ptr(Ws[0]), nat.ptr(Ws[1]), nat.ptr(Ws[2]), float(scale), nat.ptr(h3), nat.stream_of(rc))
        ctx.save_for_backward(r, W1, W2, W3)
        return h3

    @staticmethod
    def backward(ctx, u):
        from ictc_o3.autograd import required_gradients
        held = ctx.link.take()   # (u of the force pass, rho) the second derivative left for this pass
        r, W1, W2, W3 = ctx.saved_tensors
        # asked of the engine for every pass (a retained graph runs the same route each time)
        needs = required_gradients((r, W1, W2, W3), ctx.needs_input_grad[:4])
        if not any(needs):
            return (None,) * 7
        if held is not None:
            dr, dW, _ = _hidden_second(r, (W1, W2, W3), ctx.cfg, held[0], held[1], u, needs)
            return (dr, *dW, None, None, None)
        if u is None:
            return (None,) * 7
        if torch.is_grad_enabled():
            # differentiable adjoint (the force pass of a force-loss step)
            out = _HiddenAdjoint.apply(r, W1, W2, W3, u, ctx.cfg, tuple(needs), ctx.link)
            return (*out, None, None, None)
        dr, dW = _hidden_adjoint(r, (W1, W2, W3), ctx.cfg, u, needs)
        return (dr, *dW, None, None, None)


class _HiddenAdjoint(torch.autograd.Function):
    """(dr, dW1, dW2, dW3) of radial_hidden for cotangent u, differentiable once more on the fused kernel
    (ictc_radial_mlp_bwd2: cotangents on dr only); cotangents on the weight gradients, or a backward that
    itself builds a graph, go through _hidden_torch.  When the forward node's first adjoint runs later in
    the same pass, the r and weight parts are left to it (one launch for both derivatives)."""

    @staticmethod
    def forward(ctx, r, W1, W2, W3, u, cfg, needs, link):
        ctx.cfg, ctx.link = cfg, link
        ctx.save_for_backward(r, W1, W2, W3, u)
        dr, dW = _hidden_adjoint(r, (W1, W2, W3), cfg, u, needs)
        return dr, *dW

    @staticmethod
    def backward(ctx, hr, h1, h2, h3):
        from ictc_o3.autograd import required_gradients
        r, W1, W2, W3, u = ctx.saved_tensors
        needs = required_gradients((r, W1, W2, W3, u), ctx.needs_input_grad[:5])
        none = (None,) * 8
        if not any(needs) or (hr is None and h1 is None and h2 is None and h3 is None):
            return none
        if torch.is_grad_enabled() or h1 is not None or h2 is not None or h3 is not None:
            return (*_hidden_adjoint_torch(ctx.cfg, (r, W1, W2, W3, u), (hr, h1, h2, h3), needs), None, None, None)
        Ws = (W1, W2, W3)
        if any(needs[:4]) and ctx.link.can_hold():
            ctx.link.hold((u, hr))
            d_u = _hidden_tangent_cotangent(r, Ws, ctx.cfg, u, hr) if needs[4] else None
            return (None, None, None, None, d_u, None, None, None)
        if not any(needs[:4]):
            return (None, None, None, None, _hidden_tangent_cotangent(r, Ws, ctx.cfg, u, hr), None, None, None)
        dr, dW, d_u = _hidden_second(r, Ws, ctx.cfg, u, hr, None, needs, want_du=needs[4])
        return (dr, *dW, d_u, None, None, None)


def _hidden_adjoint_torch(cfg, saved, cotangents, needs):
    """Derivative of the first adjoint on composed torch operations (any order)."""
    create = torch.is_grad_enabled()
    # building a graph: differentiate the saved tensors themselves, so the result stays connected to theirs
    inputs = [t if create and t.requires_grad else t.detach().requires_grad_(True) for t in saved]
    r, W1, W2, W3, u = inputs
    with torch.enable_grad():
        h = _hidden_torch(r, W1, W2, W3, *cfg)
        first = torch.autograd.grad(h, (r, W1, W2, W3), u, create_graph=True, allow_unused=True)
        outs = [(f, c) for f, c in zip(first, cotangents) if f is not None and c is not None]
        wanted = [t for t, n in zip(inputs, needs) if n]
        got = torch.autograd.grad([f for f, _ in outs], wanted, [c for _, c in outs], create_graph=create,
                                  allow_unused=True)
    it = iter(got)
    return tuple(next(it) if n else None for n in needs)
