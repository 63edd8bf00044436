"""Direction harmonics on the HIP kernels, with first and mixed second derivatives.

Y(n) packed [E, (lmax+1)^2] (ictc_o3/basis/ictd_irreps.py:1153-1208).  The
adjoint J^T gY, its cotangent derivative J h and its direction derivative
Hess(gY . Y) h are each one kernel; that covers force-loss training
(derivatives up to second order of the harmonic map, as the reference's
harmonic _Adjoint, ops/generated_direction_harmonics.py:112-149).
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from ictc_o3 import _native as nat


def _c(t):
    return t if t.is_contiguous() else t.contiguous()


def _fwd_raw(n, lmax):
    out = n.new_empty(n.shape[0], (lmax + 1) ** 2)
    nat.call("ictc_sh_fwd", nat.ptr(n), n.shape[0], lmax, nat.ptr(out), nat.stream_of(n))
    return out


class Harmonics(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, lmax):
        ctx.set_materialize_grads(False)
        n = _c(n)
        ctx.lmax = lmax
        ctx.save_for_backward(n)
        return _fwd_raw(n, lmax)

    @staticmethod
    def backward(ctx, gY):
        if gY is None or not ctx.needs_input_grad[0]:
            return None, None
        (n,) = ctx.saved_tensors
        return HarmonicsAdjoint.apply(n, _c(gY), ctx.lmax), None


class HarmonicsAdjoint(torch.autograd.Function):
    @staticmethod
    def forward(ctx, n, gY, lmax):
        ctx.set_materialize_grads(False)
        ctx.lmax = lmax
        ctx.save_for_backward(n, gY)
        out = torch.empty_like(n)
        nat.call("ictc_sh_bwd", nat.ptr(n), nat.ptr(gY), n.shape[0], lmax, nat.ptr(out), nat.stream_of(n))
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, h):
        if h is None:
            return None, None, None
        n, gY = ctx.saved_tensors
        h = _c(h)
        dn = dgY = None
        if ctx.needs_input_grad[1]:
            dgY = n.new_empty(n.shape[0], (ctx.lmax + 1) ** 2)
            nat.call("ictc_sh_jvp", nat.ptr(n), nat.ptr(h), n.shape[0], ctx.lmax, nat.ptr(dgY), nat.stream_of(n))
        if ctx.needs_input_grad[0]:
            dn = torch.empty_like(n)
            nat.call("ictc_sh_hvp", nat.ptr(n), nat.ptr(gY), nat.ptr(h), n.shape[0], ctx.lmax, nat.ptr(dn),
                     nat.stream_of(n))
        return dn, dgY, None


def harmonics_packed(n: torch.Tensor, lmax: int) -> torch.Tensor:
    """[E,3] directions -> [E,(lmax+1)^2] packed harmonics (differentiable to second order)."""
    return Harmonics.apply(n, lmax)
