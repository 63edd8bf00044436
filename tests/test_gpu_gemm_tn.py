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
                                   (1000, 512, 130), (300001, 64, 16), (40000, 130, 1)])
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


def _grouped(device, a, b, groups, rg, a_cg, a_ldc, b_cg, b_ldc, M, N, a_off=0, b_off=0):
    """ictc_gemm_tn_grouped on row-major a, b with (group, member) rows: element (g, i, c) at
    g * stride(0) + i * (cg) + (c // cg) * ldc + c % cg, after an offset."""
    import ctypes
    from ictc_o3 import _native as nat
    a, b = a.to(device), b.to(device)
    out = torch.empty(M, N, device=device)
    ws_bytes = int(nat.lib().ictc_gemm_tn_workspace_bytes(groups * rg, M, N))
    ws = torch.empty(max(ws_bytes, 16) // 4, device=device)
    nat.call("ictc_gemm_tn_grouped", ctypes.c_void_p(a.data_ptr() + 4 * a_off), a.stride(0), a_cg, a_cg, a_ldc,
             ctypes.c_void_p(b.data_ptr() + 4 * b_off), b.stride(0), b_cg, b_cg, b_ldc, groups, rg, M, N,
             nat.ptr(out), nat.ptr(ws), ws_bytes, nat.stream_of(a))
    return out.double().cpu()


def _blocks(x, groups, rg, cg, blocks, off):
    """The [groups * rg, blocks * cg] operand a grouped call reads from x (rows (g, i), columns (block, c))."""
    v = x[:, off:off + blocks * rg * cg].reshape(groups, blocks, rg, cg).transpose(1, 2)
    return v.reshape(groups * rg, blocks * cg).double()


@pytest.mark.parametrize("groups,rg,pa,pb,C", [(5000, 3, 1, 1, 64), (777, 5, 3, 1, 48), (3001, 1, 2, 5, 32),
                                               (1200, 7, 1, 3, 128), (0, 3, 2, 2, 16), (900, 2, 2, 1, 16)])
def test_gemm_tn_grouped(device, groups, rg, pa, pb, C):
    """ictc_gemm_tn_grouped against a float64 product of the rearranged blocks (the per-degree weight
    gradient of a packed linear), elementwise bound 1e-5 * (|a|^T |b|); no groups writes zeros."""
    g = torch.Generator().manual_seed(groups + rg + C)
    a = torch.randn(groups, pa * rg * C + 13, generator=g)
    b = torch.randn(groups, pb * rg * C + 7, generator=g)
    A, B = _blocks(a, groups, rg, C, pa, 13), _blocks(b, groups, rg, C, pb, 7)
    got = _grouped(device, a, b, groups, rg, C, rg * C, C, rg * C, pa * C, pb * C, a_off=13, b_off=7)
    ref = A.t() @ B
    bound = A.abs().t() @ B.abs()
    assert got.shape == ref.shape
    if groups == 0:
        assert bool((got == 0).all())
    else:
        assert float(((got - ref).abs() / bound.clamp(min=1e-30)).max()) < 1e-5
    # bitwise repeatable
    assert torch.equal(got, _grouped(device, a, b, groups, rg, C, rg * C, C, rg * C, pa * C, pb * C, a_off=13,
                                     b_off=7))


def test_gemm_tn_grouped_rejects_bad_sizes(device):
    import ctypes
    from ictc_o3 import _native as nat
    x = torch.zeros(4, 64, device=device)
    with pytest.raises(ValueError):
        nat.call("ictc_gemm_tn_grouped", nat.ptr(x), 64, 16, 0, 16, nat.ptr(x), 64, 16, 16, 16, 4, 1, 16, 16,
                 nat.ptr(x), nat.ptr(x), 256, nat.stream_of(x))
    with pytest.raises(ValueError):
        nat.call("ictc_gemm_tn_grouped", nat.ptr(x), 64, 16, 16, 16, nat.ptr(x), 64, 16, 16, 16, 1 << 30, 4, 16, 16,
                 nat.ptr(x), nat.ptr(x), 256, nat.stream_of(x))
