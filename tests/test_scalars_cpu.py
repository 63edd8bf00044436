"""Scalar-column take and in-place add of the model's layer input/output (CPU, float64): values and
derivatives to third order against the slice forms they replace."""
import torch
from torch.autograd import gradcheck, gradgradcheck

from ictc_o3.ops.linear import add_scalars_any_, take_scalars


def test_take_scalars_matches_slice_to_third_order():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(5, 12, dtype=torch.float64, generator=g, requires_grad=True)
    assert torch.equal(take_scalars(x, 4), x[:, :4])
    assert take_scalars(x, 12) is x
    f = lambda x: take_scalars(x * x, 4) ** 2
    assert gradcheck(f, (x,))
    assert gradgradcheck(f, (x,))
    # third order: derivative of a second-derivative quantity against the slice form
    def third(fn):
        y = fn(x)
        (d1,) = torch.autograd.grad(y.sum(), x, create_graph=True)
        (d2,) = torch.autograd.grad((d1 * d1).sum(), x, create_graph=True)
        (d3,) = torch.autograd.grad((d2 ** 2).sum(), x)
        return d3
    ref = third(lambda x: (x * x)[:, :4] ** 2)
    assert torch.allclose(third(f), ref, rtol=1e-12, atol=1e-12)


def test_add_scalars_matches_slice_add_to_third_order():
    g = torch.Generator().manual_seed(4)
    a = torch.randn(6, 9, dtype=torch.float64, generator=g, requires_grad=True)
    s = torch.randn(6, 3, dtype=torch.float64, generator=g, requires_grad=True)

    def new(a, s):
        return add_scalars_any_(torch.sin(a), s * s) ** 2

    def old(a, s):
        out = torch.sin(a)
        out[:, :3] += s * s
        return out ** 2

    assert torch.equal(new(a, s), old(a, s))
    assert gradcheck(new, (a, s))
    assert gradgradcheck(new, (a, s))

    def third(fn):
        y = fn(a, s)
        da, ds = torch.autograd.grad(y.sum(), (a, s), create_graph=True)
        d2a, d2s = torch.autograd.grad((da ** 2).sum() + (ds ** 3).sum(), (a, s), create_graph=True)
        return torch.autograd.grad((d2a ** 2).sum() + (d2s ** 2).sum(), (a, s))

    for x, y in zip(third(new), third(old)):
        assert torch.allclose(x, y, rtol=1e-12, atol=1e-12)
