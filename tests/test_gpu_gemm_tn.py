"""GPU checks of the split-reduction weight-gradient kernel (out = a^T b over edge rows) and of
edge_linear, the radial-MLP linear whose weight gradients use it.

Kernel: float64 reference, elementwise bound 1e-5 * (|a|^T |b|) (FP32 sums of
a few hundred terms per chunk, then of the chunk sums), on ragged shapes whose
widths end inside a 64-column tile and inside a 16-row slab, k = 0 (zeros),
strided operands, and bitwise repeatability.  edge_linear: values, first and
second derivatives equal torch.nn.functional.linear's to 1e-5 relative at an
edge count that takes the kernel path.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _tn(device, a, b):
    from ictc_o3.ops.radial_mlp import _gemm_tn
    return _gemm_tn(a.to(device), b.to(device)).double().cpu()


@pytest.mark.parametrize("K,M,N", [(100003, 64, 64), (50001, 70, 8), (20000, 2176, 64), (17, 5, 3), (424000, 64, 64),
                                   (1000, 512, 130)])
def test_gemm_tn_accuracy(device, K, M, N):
    g = torch.Generator().manual_seed(K + M + N)
    a = torch.randn(K, M, generator=g)
    b = torch.randn(K, N, generator=g)
    ref = a.double().t() @ b.double()
    bound = a.double().abs().t() @ b.double().abs()
    got = _tn(device, a, b)
    assert got.shape == (M, N)
    err = ((got - ref).abs() / bound).max()
    assert float(err) < 1e-5, float(err)


def test_gemm_tn_empty_and_strided(device):
    from ictc_o3 import _native as nat
    from ictc_o3.ops.radial_mlp import _gemm_tn
    z = _gemm_tn(torch.empty(0, 9, device=device), torch.empty(0, 4, device=device))
    assert z.shape == (9, 4) and bool((z == 0).all())
    g = torch.Generator().manual_seed(4)
    big = torch.randn(30000, 100, generator=g)
    a, b = big[:, 3:40], big[:, 50:61]          # row pitch 100 for both operands
    ref = a.double().t() @ b.double()
    bound = a.double().abs().t() @ b.double().abs()
    dbig = big.to(device)
    M, N, K = 37, 11, 30000
    out = torch.empty(M, N, device=device)
    ws_bytes = int(nat.lib().ictc_gemm_tn_workspace_bytes(K, M, N))
    ws = torch.empty(ws_bytes // 4, device=device)
    nat.call("ictc_gemm_tn", nat.ptr(dbig[:, 3:]), K, M, 100, nat.ptr(dbig[:, 50:]), N, 100, nat.ptr(out),
             nat.ptr(ws), ws_bytes, nat.stream_of(dbig))
    assert float(((out.double().cpu() - ref).abs() / bound).max()) < 1e-5
    with pytest.raises(ValueError):
        nat.call("ictc_gemm_tn", nat.ptr(dbig), K, M, 100, nat.ptr(dbig), N, 100, nat.ptr(out), nat.ptr(ws), 4,
                 nat.stream_of(dbig))


def test_gemm_tn_deterministic(device):
    g = torch.Generator().manual_seed(9)
    a = torch.randn(200000, 64, generator=g).to(device)
    b = torch.randn(200000, 64, generator=g).to(device)
    from ictc_o3.ops.radial_mlp import _gemm_tn
    r0 = _gemm_tn(a, b)
    for _ in range(3):
        assert torch.equal(_gemm_tn(a, b), r0)


def test_edge_linear_derivatives(device):
    """Values, gradients and double-backward (force-loss style) against F.linear, E = 40000 (kernel path)."""
    from ictc_o3.ops.radial_mlp import edge_linear, _TN_MIN_ROWS
    import torch.nn.functional as F
    E = 40000
    assert E >= _TN_MIN_ROWS
    g = torch.Generator().manual_seed(12)
    x0 = torch.randn(E, 64, generator=g).to(device)
    W1_0 = (torch.randn(64, 64, generator=g) / 8).to(device)
    W2_0 = (torch.randn(192, 64, generator=g) / 8).to(device)   # the split-bf16 projection and adjoint kernels
    t = torch.randn(E, 192, generator=g).to(device)

    def run(lin):
        x = x0.clone().requires_grad_(True)
        W1, W2 = W1_0.clone().requires_grad_(True), W2_0.clone().requires_grad_(True)
        h = torch.tanh(lin(x, W1))
        y = lin(h, W2)
        e = (y * t).sum()
        gx, = torch.autograd.grad(e, x, create_graph=True)
        loss = (gx ** 2).sum() + 0.1 * e
        loss.backward()
        return y.detach(), gx.detach(), W1.grad, W2.grad, x.grad

    ours = run(edge_linear)
    ref = run(lambda a, w: F.linear(a, w))
    for o, r in zip(ours, ref):
        rel = float((o - r).norm() / r.norm())
        assert rel < 1e-5, rel
