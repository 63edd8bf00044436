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


@pytest.mark.parametrize("M,K,N,lda,acc", [(1000, 64, 1, 64, 0), (131, 8, 64, 8, 0), (517, 128, 1280, 200, 0),
                                           (64, 2176, 64, 2176, 1), (3, 5, 7, 9, 1), (8192, 16, 64, 16, 0)])
def test_gemm_nt_against_float64(device, M, K, N, lda, acc):
    """ictc_gemm_nt: c (+)= a . b^T with row pitches, odd sizes, thin readout shapes (FP32-MFMA sums, 1e-5)."""
    from ictc_o3 import _native as nat
    g = torch.Generator().manual_seed(M + K + N)
    a = torch.randn(M, lda, generator=g, dtype=torch.float64)
    b = torch.randn(N, K, generator=g, dtype=torch.float64)
    c0 = torch.randn(M, N, generator=g, dtype=torch.float64)
    ref = a[:, :K] @ b.t() + (c0 if acc else 0)
    ad, bd, cd = a.float().to(device), b.float().to(device), c0.float().to(device)
    nat.call("ictc_gemm_nt", nat.ptr(ad), M, K, lda, nat.ptr(bd), N, K, nat.ptr(cd), N, acc,
             torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.synchronize()
    assert rel_err(cd, ref) < 1e-5


def test_graph_sum_exact_and_repeatable(device):
    from ictc_o3.ops.linear import graph_sum
    g = torch.Generator().manual_seed(4)
    v = torch.randn(50000, generator=g)
    batch = torch.randint(0, 37, (50000,), generator=g)
    ref = torch.zeros(37, dtype=torch.float64).index_add(0, batch, v.double())
    vd = v.to(device).requires_grad_(True)
    out = graph_sum(vd, batch.to(device), 37)
    assert out.dtype == torch.float64 and float((out.cpu() - ref).abs().max()) < 1e-9
    assert torch.equal(out, graph_sum(vd, batch.to(device), 37))
    w = torch.randn(37, generator=g, dtype=torch.float64)
    (gv,) = torch.autograd.grad((out * w.to(device)).sum(), vd)
    assert torch.equal(gv.cpu(), w[batch].float())
    # contiguous-per-graph batch (the collate order) through the binary-searched form, with empty graphs
    sb, order = torch.sort(batch[batch % 5 != 3], stable=True)
    sv = v[batch % 5 != 3][order]
    ref = torch.zeros(37, dtype=torch.float64).index_add(0, sb, sv.double())
    got = graph_sum(sv.to(device), sb.to(device), 37, batch_sorted=True)
    assert float((got.cpu() - ref).abs().max()) < 1e-9
    assert torch.equal(got, graph_sum(sv.to(device), sb.to(device), 37))
    assert torch.equal(got[3::5].cpu(), torch.zeros_like(got[3::5].cpu()))
    with pytest.raises(TypeError):
        graph_sum(sv.double().to(device), sb.to(device), 37)


@pytest.mark.parametrize("kind,C,lmax,N", [("degree", 64, 2, 300), ("path", 128, 2, 129), ("degree", 32, 3, 77)])
def test_packed_linear_any_order(device, kind, C, lmax, N):
    """The any-order packed linear (second-order callers): output, first derivatives and the derivative of
    a first-derivative quantity (double backward through the adjoint and the weight gradients) vs float64
    autograd of the composable form."""
    from ictc_o3.ops.linear import degree_linear, degree_linear_any, path_linear, path_linear_any
    g = torch.Generator().manual_seed(C + lmax + N)
    counts = {0: 3, 1: 4, 2: 4, 3: 2}
    if kind == "degree":
        width_in = (lmax + 1) ** 2 * C
        Ws = [torch.randn(C, C, generator=g, dtype=torch.float64) / C ** 0.5 for _ in range(lmax + 1)]
        ref_fn = lambda x, W: degree_linear(x, W, C, lmax, 0.7)
        fn = lambda x, W: degree_linear_any(x, W, C, lmax, 0.7)
    else:
        width_in = sum(counts[l] * (2 * l + 1) for l in range(lmax + 1)) * C
        Ws = [torch.randn(C, counts[l] * C, generator=g, dtype=torch.float64) / (counts[l] * C) ** 0.5
              for l in range(lmax + 1)]
        ref_fn = lambda x, W: path_linear(x, W, counts, C, lmax, 1 / 42.0)
        fn = lambda x, W: path_linear_any(x, W, counts, C, lmax, 1 / 42.0)
    x = torch.randn(N, width_in, generator=g, dtype=torch.float64)
    go = torch.randn(N, (lmax + 1) ** 2 * C, generator=g, dtype=torch.float64)
    v = torch.randn(N, width_in, generator=g, dtype=torch.float64)

    def run(f, xs, Wl):
        xs = xs.clone().requires_grad_(True)
        Wl = [w.clone().requires_grad_(True) for w in Wl]
        out = f(xs, Wl)
        dx, *dW = torch.autograd.grad(out, [xs] + Wl, go.to(out), create_graph=True)
        # a scalar of the first derivatives, differentiated again (the force-loss pattern)
        s = (dx * v.to(dx)).sum() + sum((d ** 2).sum() for d in dW)
        gg = torch.autograd.grad(s, [xs] + Wl, allow_unused=True)
        return out, [dx] + dW, gg

    def plain(f, xs, Wl):
        # a backward that builds no graph: the weight gradients read the packed blocks in place
        # (ictc_gemm_tn_grouped)
        xs = xs.clone().requires_grad_(True)
        Wl = [w.clone().requires_grad_(True) for w in Wl]
        out = f(xs, Wl)
        return torch.autograd.grad(out, [xs] + Wl, go.to(out))

    out0, d0, gg0 = run(ref_fn, x, Ws)
    out1, d1, gg1 = run(fn, x.float().to(device), [w.float().to(device) for w in Ws])
    assert rel_err(out1, out0) < 1e-5
    for a, b in zip(d1, d0):
        assert rel_err(a, b) < 1e-5
    for a, b in zip(gg1, gg0):
        if b is None:
            continue
        assert rel_err(a, b) < 1e-5
    for a, b in zip(plain(fn, x.float().to(device), [w.float().to(device) for w in Ws]), d0):
        assert rel_err(a, b) < 1e-5


def _species_ref(x, W, s):
    """float64 out[n] = W[s_n] x[n], one masked product per species (zero rows outside [0, S))."""
    out = torch.zeros(x.shape[0], W.shape[1], dtype=x.dtype)
    for k in range(W.shape[0]):
        m = s == k
        out = out.index_put((m.nonzero().squeeze(1),), x[m] @ W[k].t())
    return out


@pytest.mark.parametrize("C,S,N,sp_mode", [(64, 3, 1000, "uniform"), (128, 10, 517, "uniform"), (16, 1, 33, "uniform"),
                                           (32, 4, 4096, "uniform"), (128, 10, 8192, "uniform"),
                                           (64, 3, 40000, "uniform"), (128, 6, 700, "gaps"), (64, 4, 300, "one")])
def test_species_linear(device, C, S, N, sp_mode):
    """species_linear (out[n] = W[species[n]] x[n]): values, first derivatives (input and weights) and the
    derivative of a first-derivative quantity against float64 autograd of the indexed product, 1e-5.
    64 and 128 channels run on the species-sorted tile kernels (8192 nodes: the force-loss training batch;
    40000: row tiles longer than 128 in the weight gradient); "gaps" leaves species without nodes and puts
    ids outside [0, S) (zero rows), "one" gives every node the same species."""
    from ictc_o3.ops.linear import species_linear
    g = torch.Generator().manual_seed(C + S + N)
    x64 = torch.randn(N, C, generator=g, dtype=torch.float64)
    W64 = torch.randn(S, C, C, generator=g, dtype=torch.float64) / C ** 0.5
    if sp_mode == "gaps":
        sp = torch.tensor([0, 2, 5, S, -1, S + 3])[torch.randint(0, 6, (N,), generator=g)]
    elif sp_mode == "one":
        sp = torch.full((N,), S - 1, dtype=torch.int64)
    else:
        sp = torch.randint(0, S, (N,), generator=g)
    go = torch.randn(N, C, generator=g, dtype=torch.float64)
    v = torch.randn(N, C, generator=g, dtype=torch.float64)

    def run(f, x, W, s):
        x = x.clone().requires_grad_(True)
        W = W.clone().requires_grad_(True)
        out = f(x, W, s)
        dx, dW = torch.autograd.grad(out, (x, W), go.to(out), create_graph=True)
        gg = torch.autograd.grad((dx * v.to(dx)).sum() + (dW ** 2).sum(), (x, W))
        return [out, dx, dW, *gg]

    ref = run(_species_ref, x64, W64, sp)
    got = run(species_linear, x64.float().to(device), W64.float().to(device), sp.to(device))
    for a, b in zip(got, ref):
        assert rel_err(a, b) < 1e-5


def test_species_linear_column_slice(device):
    """A column slice of a wider row (pitch 3C) read in place gives the same values and input gradient as its
    contiguous copy; a second call with the same species tensor reuses its sort."""
    from ictc_o3.ops import linear as lin
    C, S, N = 128, 10, 2000
    g = torch.Generator().manual_seed(7)
    wide = torch.randn(N, 3 * C, generator=g).to(device)
    W = (torch.randn(S, C, C, generator=g) / C ** 0.5).to(device)
    sp = torch.randint(0, S, (N,), generator=g).to(device)
    xs = wide[:, C:2 * C].requires_grad_(False)
    a = lin.species_linear(xs, W, sp)
    order = lin.species_order(sp, S)
    b = lin.species_linear(xs.contiguous(), W, sp)
    assert lin.species_order(sp, S) is order
    assert torch.equal(a, b)
    ref = _species_ref(xs.double().cpu(), W.double().cpu(), sp.cpu())
    assert rel_err(a, ref) < 1e-5


def test_species_linear_edge_cases(device):
    """No nodes; every species id outside [0, S) (zero rows, zero weight gradient); and the weight gradient
    through the C ABI with 256-row tiles (eight LDS stages per tile) against the float64 per-species sums."""
    import ctypes
    from ictc_o3 import _native as nat
    from ictc_o3.ops import linear as lin
    C, S = 64, 4
    W = (torch.randn(S, C, C) / C ** 0.5).to(device).requires_grad_(True)
    x0 = torch.zeros(0, C, device=device, requires_grad=True)
    y0 = lin.species_linear(x0, W, torch.zeros(0, dtype=torch.int64, device=device))
    assert y0.shape == (0, C)
    x = torch.randn(50, C, device=device, requires_grad=True)
    bad = torch.tensor([S, -1, S + 7] * 16 + [S, -2], device=device)
    y = lin.species_linear(x, W, bad)
    assert torch.equal(y, torch.zeros_like(y))
    dx, dW = torch.autograd.grad(y.sum(), (x, W))
    assert torch.equal(dx, torch.zeros_like(dx)) and torch.equal(dW, torch.zeros_like(dW))
    g = torch.Generator().manual_seed(11)
    N, C, S = 3000, 128, 3
    a64 = torch.randn(N, C, generator=g, dtype=torch.float64)
    b64 = torch.randn(N, C, generator=g, dtype=torch.float64)
    sp = torch.randint(0, S, (N,), generator=g)
    order = lin.species_order(sp.to(device), S)
    a, b = a64.float().to(device), b64.float().to(device)
    rows = 256
    nb = int(nat.lib().ictc_species_outer_workspace_bytes(N, C, S, rows))
    ws = torch.empty(nb // 4, device=device)
    out = torch.empty(S, C, C, device=device)
    nat.call("ictc_species_outer", nat.ptr(a), C, nat.ptr(b), C, N, C, S, nat.ptr(order.perm), nat.ptr(order.off),
             rows, nat.ptr(out), nat.ptr(ws), nb, nat.stream_of(a))
    ref = torch.stack([a64[sp == s].t() @ b64[sp == s] for s in range(S)])
    assert rel_err(out, ref) < 1e-5
