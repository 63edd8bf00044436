"""GPU parity of the edge-geometry op (r, n, mask and the CSR-gather adjoint to positions).

Compared with the float64 restatement model_oracle.edge_geometry under torch
autograd: r and n within 2e-6 relative (fp32 rounding of vec), position / shift gradients within 1e-5
relative (max-norm); mask bit-exact away from the cutoff.  The oracle's own
gradient is pinned by finite differences (test_geometry_oracle_gradcheck), and
translation invariance (sum over nodes of dpos = 0) checks the gather signs.
"""
import pytest
import torch

import model_oracle as mo
from helpers import rel_err

pytestmark = pytest.mark.gpu


def _case(N, E, seed, sort):
    g = torch.Generator().manual_seed(seed)
    pos = (torch.rand(N, 3, generator=g, dtype=torch.float64) * 6.0).float().double()   # fp32-representable
    src = torch.randint(0, N, (E,), generator=g)
    dst = torch.randint(0, N, (E,), generator=g)
    keep = src != dst
    src, dst = src[keep], dst[keep]
    if sort:
        o = torch.argsort(dst, stable=True)
        src, dst = src[o], dst[o]
    shift = torch.randn(src.numel(), 3, generator=g, dtype=torch.float64).float().double()
    return pos, src, dst, shift


@pytest.mark.parametrize("N,E,seed,sort,with_shift", [(200, 4000, 1, True, True), (57, 900, 2, False, True),
                                                      (40, 300, 3, True, False), (7, 0, 4, True, True),
                                                      (1000, 20000, 5, False, False)])
def test_edge_geometry(device, N, E, seed, sort, with_shift):
    from ictc_o3.ops.geometry import edge_geometry
    from ictc_o3.ops.tensor_product import Topology
    pos, src, dst, shift = _case(N, E, seed, sort)
    E = src.numel()
    g = torch.Generator().manual_seed(seed + 100)
    gr = torch.randn(E, generator=g, dtype=torch.float64)
    gn = torch.randn(E, 3, generator=g, dtype=torch.float64)

    p64 = pos.clone().requires_grad_(True)
    s64 = shift.clone().requires_grad_(True)
    r, n, m = mo.edge_geometry(p64, src, dst, s64 if with_shift else torch.zeros_like(shift), 4.5)
    if E:
        torch.autograd.backward([r, n], [gr, gn])

    pd = pos.float().to(device).requires_grad_(True)
    sd = shift.float().to(device).requires_grad_(True) if with_shift else None
    topo = Topology(src.to(device), dst.to(device), N)
    r2, n2, m2 = edge_geometry(pd, sd, topo, 4.5)
    if E:
        assert rel_err(r2, r) < 2e-6 and rel_err(n2, n) < 2e-6
        far = (r - 4.5).abs() > 1e-4
        assert torch.equal(m2.cpu()[far].double(), m[far])
        torch.autograd.backward([r2, n2], [gr.float().to(device), gn.float().to(device)])
        assert rel_err(pd.grad, p64.grad) < 1e-5
        assert pd.grad.double().sum(0).abs().max().item() < 1e-4 * pd.grad.abs().max().item()
        if with_shift:
            assert rel_err(sd.grad, s64.grad) < 1e-5
        # deterministic: a second adjoint is bitwise equal
        first = pd.grad.clone()
        pd.grad = None
        r3, n3, _ = edge_geometry(pd, sd, topo, 4.5)
        torch.autograd.backward([r3, n3], [gr.float().to(device), gn.float().to(device)])
        assert torch.equal(first, pd.grad)


@pytest.mark.parametrize("N,E,seed", [(200, 4000, 11), (31, 200, 12), (1000, 30000, 13)])
def test_edge_vectors_second_order(device, N, E, seed):
    """edge_vectors through a force-loss style double backward equals float64 gathers; repeatable bitwise."""
    from ictc_o3.ops.geometry import edge_vectors
    from ictc_o3.ops.tensor_product import Topology
    pos, src, dst, shift = _case(N, E, seed, True)
    E = src.numel()
    g = torch.Generator().manual_seed(seed + 7)
    t = torch.randn(N, 3, generator=g, dtype=torch.float64)

    def run(p, s, vec_fn):
        vec = vec_fn(p, s)
        e = (vec.norm(dim=1) ** 3).sum() + (vec[:, 0] * vec[:, 1]).sum()
        gp, = torch.autograd.grad(e, p, create_graph=True)
        loss = (gp * t.to(gp)).sum() + 0.5 * e
        loss.backward()
        return vec.detach(), gp.detach(), p.grad, s.grad

    p64, s64 = pos.clone().requires_grad_(True), shift.clone().requires_grad_(True)
    ref = run(p64, s64, lambda p, s: p[dst] - p[src] + s)
    topo = Topology(src.to(device), dst.to(device), N)
    outs = []
    for _ in range(2):
        pd = pos.float().to(device).requires_grad_(True)
        sd = shift.float().to(device).requires_grad_(True)
        outs.append(run(pd, sd, lambda p, s: edge_vectors(p, s, topo)))
    for o, r in zip(outs[0], ref):
        if r.numel():
            assert rel_err(o, r) < 1e-5
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("cells,E,seed", [(1, 5000, 7), (3, 4000, 8), (1, 0, 9)])
def test_shift_vectors(device, cells, E, seed):
    """ictc_shift_vectors against the same three products and two sums rounded one by one on the host
    (bitwise), exact oddness in the shift (an edge and its reverse), graph selection through batch[src],
    and NaN rows for an out-of-range source."""
    from ictc_o3.ops.geometry import shift_vectors
    g = torch.Generator().manual_seed(seed)
    N = 50
    sh = torch.randint(-2, 3, (E, 3), generator=g).float()
    cell = (torch.randn(cells, 3, 3, generator=g) * 4.0).float()
    batch = torch.randint(0, cells, (N,), generator=g)
    src = torch.randint(0, N, (E,), generator=g)
    c = cell[batch[src]] if cells > 1 else cell[0].expand(E, 3, 3)
    want = (sh[:, 0:1] * c[:, 0, :] + sh[:, 1:2] * c[:, 1, :]) + sh[:, 2:3] * c[:, 2, :]
    got = shift_vectors(sh.to(device), cell.to(device), batch.to(device), src.to(device)).cpu()
    assert torch.equal(got, want)
    neg = shift_vectors((-sh).to(device), cell.to(device), batch.to(device), src.to(device)).cpu()
    assert torch.equal(neg, -got)
    if cells > 1 and E:
        bad = src.clone()
        bad[3] = N + 5
        out = shift_vectors(sh.to(device), cell.to(device), batch.to(device), bad.to(device)).cpu()
        assert torch.isnan(out[3]).all() and torch.equal(out[torch.arange(E) != 3], got[torch.arange(E) != 3])


@pytest.mark.parametrize("lmax", [0, 1, 2, 3])
@pytest.mark.parametrize("N,E,seed,sort,with_shift,cot", [(200, 4000, 21, True, True, "both"),
                                                         (57, 900, 22, False, True, "dY"),
                                                         (300, 5000, 23, True, False, "dr"),
                                                         (7, 0, 24, True, True, "both")])
def test_edge_harmonics_matches_geometry_then_harmonics(device, lmax, N, E, seed, sort, with_shift, cot):
    """The one-pass geometry + harmonics op gives bitwise the values (r, Y, mask) of edge_geometry followed by
    harmonics_packed (whose parity the tests above and the harmonics tests hold), and their position / shift
    adjoints to FP32 rounding (1e-6 of the largest entry: the compiler may fuse a product into a
    multiply-add differently in the one-pass adjoint kernel and in the two separate ones)."""
    from ictc_o3.ops.geometry import edge_geometry, edge_harmonics
    from ictc_o3.ops.harmonics import harmonics_packed
    from ictc_o3.ops.tensor_product import Topology
    pos, src, dst, shift = _case(N, E, seed, sort)
    E = src.numel()
    topo = Topology(src.to(device), dst.to(device), N)
    g = torch.Generator().manual_seed(seed + 7)
    gr = torch.randn(E, generator=g).to(device)
    gY = torch.randn(E, (lmax + 1) ** 2, generator=g).to(device)
    outs = []
    for fused in (True, False):
        pd = pos.float().to(device).requires_grad_(True)
        sd = shift.float().to(device).requires_grad_(True) if with_shift else None
        if fused:
            r, Y, m = edge_harmonics(pd, sd, topo, 4.5, lmax)
        else:
            r, n, m = edge_geometry(pd, sd, topo, 4.5)
            Y = harmonics_packed(n, lmax)
        if E:
            ts, gs = ([r] if cot != "dY" else []) + ([Y] if cot != "dr" else []), \
                ([gr] if cot != "dY" else []) + ([gY] if cot != "dr" else [])
            torch.autograd.backward(ts, gs)
        outs.append((r.detach(), Y.detach(), m, None if pd.grad is None else pd.grad.clone(),
                     None if sd is None or sd.grad is None else sd.grad.clone()))
    for k, (a, b) in enumerate(zip(*outs)):
        assert (a is None) == (b is None)
        if a is None:
            continue
        if k < 3:
            assert torch.equal(a, b)
        elif a.numel():
            assert (a - b).abs().max().item() <= 1e-6 * b.abs().max().item()


@pytest.mark.parametrize("lmax", [1, 2])
@pytest.mark.parametrize("cot", ["both", "first_only", "second_only", "mixed"])
def test_edge_harmonics_two_consumers(device, lmax, cot):
    """uses = 2: the second (r, Y) outputs' cotangents are added in the adjoint kernel; dpos and dshift are
    bitwise those of one consumer fed with the fp32 sums (what autograd's addition would form)."""
    from ictc_o3.ops.geometry import edge_harmonics
    from ictc_o3.ops.tensor_product import Topology
    N, E, seed = 300, 6000, 31
    pos, src, dst, shift = _case(N, E, seed, True)
    E = src.numel()
    topo = Topology(src.to(device), dst.to(device), N)
    g = torch.Generator().manual_seed(seed)
    ga, gb = torch.randn(E, generator=g).to(device), torch.randn(E, generator=g).to(device)
    Ya, Yb = (torch.randn(E, (lmax + 1) ** 2, generator=g).to(device) for _ in range(2))
    # one cotangent as a view 4 bytes into a buffer (not 16-byte aligned): the op realigns it
    buf = torch.zeros(E * (lmax + 1) ** 2 + 1, device=device)
    buf[1:] = Yb.reshape(-1)
    Yb = buf[1:].view(E, (lmax + 1) ** 2)
    assert Yb.data_ptr() % 16 != 0
    use = {"both": (True, True, True, True), "first_only": (True, False, True, False),
           "second_only": (False, True, False, True), "mixed": (True, False, False, True)}[cot]

    def run(two):
        pd = pos.float().to(device).requires_grad_(True)
        sd = shift.float().to(device).requires_grad_(True)
        if two:
            r, r2, Y, Y2, _ = edge_harmonics(pd, sd, topo, 4.5, lmax, uses=2)
            ts = [t for t, u in zip((r, r2, Y, Y2), use) if u]
            gs = [t for t, u in zip((ga, gb, Ya, Yb), use) if u]
        else:
            r, Y, _ = edge_harmonics(pd, sd, topo, 4.5, lmax)
            sr = ga + gb if use[0] and use[1] else (ga if use[0] else gb if use[1] else None)
            sY = Ya + Yb if use[2] and use[3] else (Ya if use[2] else Yb if use[3] else None)
            ts = [t for t, gg in ((r, sr), (Y, sY)) if gg is not None]
            gs = [gg for gg in (sr, sY) if gg is not None]
        torch.autograd.backward(ts, gs)
        return pd.grad.clone(), sd.grad.clone()

    a, b = run(True), run(False)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_edge_unit_derivatives(device):
    """edge_unit (r, n of edge vectors that are autograd inputs, ictc_edge_unit): values, the adjoint, its
    derivative (the force-loss second order) and a third derivative (composed form) against float64 autograd of
    norm and clamped division, 1e-5; vectors below the clamp and a zero vector included."""
    from ictc_o3.ops.geometry import edge_unit
    g = torch.Generator().manual_seed(11)
    v64 = torch.randn(3000, 3, generator=g, dtype=torch.float64) * 2
    v64[:5] *= 1e-9          # below the 1e-8 clamp
    v64[5] = 0.0
    gr = torch.randn(3000, generator=g, dtype=torch.float64)
    gn = torch.randn(3000, 3, generator=g, dtype=torch.float64)
    h = torch.randn(3000, 3, generator=g, dtype=torch.float64)
    w = torch.randn(3000, 3, generator=g, dtype=torch.float64)

    def ref_unit(v):
        r = v.norm(dim=1)
        return r, v / r.clamp(min=1e-8).unsqueeze(-1)

    def run(f, v, gr, gn, h, w, third):
        v = v.clone().requires_grad_(True)
        gr = gr.clone().requires_grad_(True)
        gn = gn.clone().requires_grad_(True)
        r, n = f(v)
        (gv,) = torch.autograd.grad((r, n), v, (gr, gn), create_graph=True)
        # without a graph the second derivative runs on the kernel (order 2); with one, on the composed form
        d2 = torch.autograd.grad(gv, (v, gr, gn), h, create_graph=third)
        if not third:
            return [r, n, gv, *d2]
        (d3,) = torch.autograd.grad(d2[0], v, w)
        return [d3]

    ok = slice(6, None)   # derivatives of the clamped branch are compared on the regular edges only
    for third in (False, True):
        ref = run(ref_unit, v64, gr, gn, h, w, third)
        got = run(edge_unit, *[t.float().to(device) for t in (v64, gr, gn, h, w)], third)
        for k, (a, b) in enumerate(zip(got, ref)):
            assert rel_err(a[ok], b[ok]) < 1e-5, (third, k)
        if not third:
            # below the clamp: r and n exact forms, and finite first and second derivatives on the kernel
            assert torch.equal(got[0][5].cpu(), torch.tensor(0.0))
            assert torch.equal(got[1][5].cpu(), torch.zeros(3))
            for t in got:
                assert bool(torch.isfinite(t).all())
