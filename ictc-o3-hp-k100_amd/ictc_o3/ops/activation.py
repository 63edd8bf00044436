"""Normalized SiLU and the radial basis on HIP kernels, with first and second derivatives.

normalized_silu(x, s) = s * x * sigmoid(x)     (operators.py:631-636, fused_activation.py,
                                                 backends/k100/hip_activation.py:11-36)
radial_embedding(r)   = sqrt(2/rc) sin(k pi r / rc) / r * env(r / rc) * [r < rc],  k = 1..K
                        with the MACE polynomial envelope of order p
                        (mace_ictc/models/radial_basis.py:11-92, sqrt_num_basis_norm=False)
"""
from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from ictc_o3 import _native as nat


def _c(t):
    return t if t.is_contiguous() else t.contiguous()


def _silu(mode, x, g, h, s):
    out = torch.empty_like(x)
    nat.call("ictc_silu", mode, nat.ptr(x), nat.ptr(g), nat.ptr(h), float(s), x.numel(), nat.ptr(out),
             nat.stream_of(x))
    return out


class _Silu(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, s):
        x = _c(x)
        ctx.s = s
        ctx.save_for_backward(x)
        return _silu(0, x, None, None, s)

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        return _SiluAdjoint.apply(x, _c(g), ctx.s), None


class _SiluAdjoint(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, g, s):
        ctx.s = s
        ctx.save_for_backward(x, g)
        return _silu(1, x, g, None, s)

    @staticmethod
    @once_differentiable
    def backward(ctx, h):
        x, g = ctx.saved_tensors
        h = _c(h)
        dx = _silu(2, x, g, h, ctx.s) if ctx.needs_input_grad[0] else None
        dg = _silu(1, x, h, None, ctx.s) if ctx.needs_input_grad[1] else None
        return dx, dg, None


def normalized_silu(features: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    if features.device.type != "cuda" or features.dtype != torch.float32:
        raise ValueError("normalized_silu requires FP32 tensors on a ROCm device")
    return _Silu.apply(features, float(scale))


def _radial(order, r, g, h, K, rc, p):
    E = r.shape[0]
    out = r.new_empty(E, K) if order in (0, 3) else r.new_empty(E)
    nat.call("ictc_radial", order, nat.ptr(r), nat.ptr(g), nat.ptr(h), E, K, float(rc), int(p), nat.ptr(out),
             nat.stream_of(r))
    return out


class _Radial(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, K, rc, p):
        r = _c(r)
        ctx.cfg = (K, rc, p)
        ctx.save_for_backward(r)
        return _radial(0, r, None, None, K, rc, p)

    @staticmethod
    def backward(ctx, g):
        (r,) = ctx.saved_tensors
        return _RadialAdjoint.apply(r, _c(g), *ctx.cfg), None, None, None


class _RadialAdjoint(torch.autograd.Function):
    @staticmethod
    def forward(ctx, r, g, K, rc, p):
        ctx.cfg = (K, rc, p)
        ctx.save_for_backward(r, g)
        return _radial(1, r, g, None, K, rc, p)

    @staticmethod
    @once_differentiable
    def backward(ctx, h):
        r, g = ctx.saved_tensors
        h = _c(h)
        dr = _radial(2, r, g, h, *ctx.cfg) if ctx.needs_input_grad[0] else None
        dg = _radial(3, r, None, h, *ctx.cfg) if ctx.needs_input_grad[1] else None
        return dr, dg, None, None, None


def radial_embedding(r: torch.Tensor, cutoff: float, num_basis: int = 8, poly_p: int = 5) -> torch.Tensor:
    """[E] edge lengths -> [E, num_basis] radial features (differentiable to second order)."""
    return _Radial.apply(r, int(num_basis), float(cutoff), int(poly_p))
