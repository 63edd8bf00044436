"""GPU parity of the MFMA packed channel linears (degree and path-preserving) vs float64 torch.

Forward, input adjoint and weight gradients within 1e-5 relative (max-norm),
for channel counts 16/64/128, degrees 0..3 and 1..4 paths per degree, with
the composable torch forms as the reference semantics (the same maps the
model's ChannelLinear / PathPreservingLinear / product linear compute).
"""
import pytest
import torch

from helpers import rel_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("C,lmax,N", [(16, 0, 33), (64, 2, 1000), (128, 3, 257), (32, 1, 64)])
def test_degree_linear(device, C, lmax, N):
    from ictc_o3.ops.linear import degree_linear, degree_linear_fast
    g = torch.Generator().manual_seed(C + lmax)
    x = torch.randn(N, (lmax + 1) ** 2 * C, generator=g, dtype=torch.float64)
    Ws = [torch.randn(C, C, generator=g, dtype=torch.float64) / C ** 0.5 for _ in range(lmax + 1)]
    go = torch.randn(N, (lmax + 1) ** 2 * C, generator=g, dtype=torch.float64)
    xr = x.clone().requires_grad_(True)
    Wr = [w.clone().requires_grad_(True) for w in Ws]
    ref = degree_linear(xr, Wr, C, lmax, 0.7)
    ref.backward(go)
    xd = x.float().to(device).requires_grad_(True)
    Wd = [w.float().to(device).requires_grad_(True) for w in Ws]
    out = degree_linear_fast(xd, Wd, C, lmax, 0.7)
    assert rel_err(out, ref) < 1e-5
    out.backward(go.float().to(device))
    assert rel_err(xd.grad, xr.grad) < 1e-5
    for a, b in zip(Wd, Wr):
        assert rel_err(a.grad, b.grad) < 1e-5


@pytest.mark.parametrize("C,lmax,counts,N", [(64, 2, {0: 3, 1: 4, 2: 4}, 700), (16, 1, {0: 1, 1: 2}, 50),
                                             (128, 3, {0: 3, 1: 5, 2: 5, 3: 4}, 129)])
def test_path_linear(device, C, lmax, counts, N):
    from ictc_o3.ops.linear import path_linear, path_linear_fast
    g = torch.Generator().manual_seed(C * 7 + lmax)
    width = sum(counts[l] * (2 * l + 1) for l in range(lmax + 1)) * C
    m = torch.randn(N, width, generator=g, dtype=torch.float64)
    Ws = [torch.randn(C, counts[l] * C, generator=g, dtype=torch.float64) / (counts[l] * C) ** 0.5
          for l in range(lmax + 1)]
    go = torch.randn(N, (lmax + 1) ** 2 * C, generator=g, dtype=torch.float64)
    mr = m.clone().requires_grad_(True)
    Wr = [w.clone().requires_grad_(True) for w in Ws]
    ref = path_linear(mr, Wr, counts, C, lmax, 1 / 42.0)
    ref.backward(go)
    md = m.float().to(device).requires_grad_(True)
    Wd = [w.float().to(device).requires_grad_(True) for w in Ws]
    out = path_linear_fast(md, Wd, counts, C, lmax, 1 / 42.0)
    assert rel_err(out, ref) < 1e-5
    out.backward(go.float().to(device))
    assert rel_err(md.grad, mr.grad) < 1e-5
    for a, b in zip(Wd, Wr):
        assert rel_err(a.grad, b.grad) < 1e-5


def test_fast_linear_refuses_second_order(device):
    from ictc_o3.ops.linear import degree_linear_fast
    x = torch.randn(20, 64, device=device, requires_grad=True)
    W = [torch.randn(64, 64, device=device, requires_grad=True)]
    out = degree_linear_fast(x, W, 64, 0)
    (gx,) = torch.autograd.grad(out.sum(), x, create_graph=False)
    assert gx.shape == x.shape
    out = degree_linear_fast(x, W, 64, 0)
    with pytest.raises(RuntimeError):
        torch.autograd.grad(out.square().sum(), x, create_graph=True)
