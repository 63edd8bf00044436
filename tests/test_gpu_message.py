"""GPU parity of the CSR graph message (PackedGraphMessage / GraphMessage) vs the float64 oracle.

Tolerance 1e-5 relative (max-norm).  Also: bitwise determinism across runs,
unsorted edge lists, masks, isolated nodes, empty graphs, out-of-range
edge ids contributing nothing.
"""
import pytest
import torch

import ictc_oracle as orc
from helpers import rel_err, unit_vectors

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _graph(N, E, C, li, le, lo, seed, sort=False, mask=False):
    g = torch.Generator().manual_seed(seed)
    P = len(orc.natural_paths(li, le, lo))
    feats = torch.randn(N, C * (li + 1) ** 2, generator=g, dtype=torch.float64)
    sh = torch.cat(orc.direction_harmonics(unit_vectors(E, seed + 1), le), -1)
    gates = torch.randn(E, P * C, generator=g, dtype=torch.float64)
    src = torch.randint(0, N, (E,), generator=g)
    dst = torch.randint(0, N, (E,), generator=g)
    if sort:
        o = torch.argsort(dst, stable=True)
        src, dst, sh, gates = src[o], dst[o], sh[o], gates[o]
    m = (torch.rand(E, generator=g) > 0.3).double() if mask else None
    return feats, sh, gates, src, dst, m


CASES = [(64, 2000, 64, 2, 2, 2, False, False), (50, 700, 32, 2, 2, 2, True, True),
         (40, 500, 128, 2, 3, 3, False, True), (30, 300, 128, 0, 3, 3, True, False),
         (33, 400, 64, 0, 2, 2, False, False), (20, 150, 17, 1, 2, 2, False, True)]


@pytest.mark.parametrize("N,E,C,li,le,lo,sort,mask", CASES)
def test_message_forward_backward(device, N, E, C, li, le, lo, sort, mask):
    from ictc_o3 import PackedGraphMessage
    op = PackedGraphMessage.create(channels=C, input_lmax=li, edge_lmax=le, output_lmax=lo, device=device)
    f64, sh64, g64, src, dst, m64 = _graph(N, E, C, li, le, lo, 10 + N, sort, mask)
    ref_in = [t.clone().requires_grad_(True) for t in (f64, sh64, g64)]
    ref = orc.message_packed(*ref_in, src, dst, m64, li, le, lo, C)
    x = [t.float().to(device).requires_grad_(True) for t in (f64, sh64, g64)]
    m = None if m64 is None else m64.float().to(device)
    out = op(*x, src.to(device), dst.to(device), m)
    assert rel_err(out, ref) < TOL
    go = torch.randn(ref.shape, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    torch.autograd.backward(ref, go)
    torch.autograd.backward(out, go.float().to(device))
    for a, b in zip(x, ref_in):
        assert rel_err(a.grad, b.grad) < TOL


@pytest.mark.parametrize("C,li,le,lo,which,create", [
    (64, 2, 2, 2, (0, 1, 2), False), (128, 2, 3, 3, (0, 1, 2), False), (64, 2, 2, 2, (0, 1, 2), True),
    (128, 2, 3, 3, (0,), False), (64, 2, 2, 2, (1, 2), False), (33, 0, 2, 2, (2,), False), (64, 1, 2, 2, (1,), True)])
def test_message_mixed_second_derivatives(device, C, li, le, lo, which, create):
    """Fused (create=False) and composed (create=True) mixed second derivatives vs float64 autograd;
    ``which`` selects the first-order gradients the objective uses (the rest give absent tangents)."""
    from ictc_o3 import PackedGraphMessage
    N, E = 24, 200
    op = PackedGraphMessage.create(channels=C, input_lmax=li, edge_lmax=le, output_lmax=lo, device=device)
    f64, sh64, g64, src, dst, m64 = _graph(N, E, C, li, le, lo, 77, mask=True)
    gen = torch.Generator().manual_seed(78)
    go64 = torch.randn(N, op.output_width, generator=gen, dtype=torch.float64)
    v = [torch.randn(t.shape, generator=gen, dtype=torch.float64) for t in (f64, sh64, g64)]

    def run(tensors, gov, fn):
        xs = [t.clone().requires_grad_(True) for t in tensors]
        gov = gov.clone().requires_grad_(True)
        grads = torch.autograd.grad(fn(*xs), xs, gov, create_graph=True)
        s = sum((grads[k] * v[k].to(grads[k])).sum() for k in which)
        return torch.autograd.grad(s, xs + [gov], allow_unused=True, create_graph=create)

    ref = run((f64, sh64, g64), go64,
              lambda a, b, c: orc.message_packed(a, b, c, src, dst, m64, li, le, lo, C))
    s, d, m = src.to(device), dst.to(device), m64.float().to(device)
    got = run([t.float().to(device) for t in (f64, sh64, g64)], go64.float().to(device),
              lambda a, b, c: op(a, b, c, s, d, m))
    for name, a, b in zip(("dx", "dsh", "dg", "dgo"), got, ref):
        if b is None or not b.abs().max() > 0:
            assert a is None or torch.count_nonzero(a) == 0, name
        else:
            assert rel_err(a, b) < TOL, name


def test_message_second_raw_abi(device):
    """ictc_msg_second directly: no edges zero-fills the node outputs; out-of-range ids and masks drop edges."""
    from ictc_o3 import PackedGraphMessage
    from ictc_o3.ops import tensor_product as tpo
    op = PackedGraphMessage.create(channels=32, input_lmax=2, edge_lmax=2, device=device)
    spec = op.edge._prepare()
    N = 9
    x = torch.randn(N, 32 * 9, device=device)
    e0 = torch.zeros(0, dtype=torch.int64, device=device)
    topo = tpo.Topology(e0, e0, N)
    go = torch.randn(N, op.output_width, device=device)
    tx = torch.randn_like(x)
    dx, dsh, dg, dgo = tpo._msg_second_raw(spec, topo, x, torch.zeros(0, 9, device=device),
                                           torch.zeros(0, op.gate_width, device=device), None, go, tx, None, None,
                                           (True, True, True, True))
    assert dx is None and dgo is not None and torch.count_nonzero(dgo) == 0
    # out-of-range ids contribute nothing: same as dropping those edges
    f64, sh64, g64, src, dst, m64 = _graph(N, 120, 32, 2, 2, 2, 31, mask=True)
    bad_src, bad_dst = src.clone(), dst.clone()
    bad_src[::5] = N + 2
    bad_dst[2::7] = -3
    keep = (bad_src < N) & (bad_dst >= 0)
    args = [t.float().to(device) for t in (f64, sh64, g64)]
    tans = [torch.randn_like(t) for t in args]
    m = m64.float().to(device)
    full = tpo._msg_second_raw(spec, tpo.Topology(bad_src.to(device), bad_dst.to(device), N), *args, m, go, *tans,
                               (True, True, True, True))
    k = keep.to(device)
    part = tpo._msg_second_raw(spec, tpo.Topology(src[keep].to(device), dst[keep].to(device), N), args[0],
                               args[1][k], args[2][k], m[k], go, tans[0], tans[1][k], tans[2][k],
                               (True, True, True, True))
    assert rel_err(full[0], part[0]) < TOL and rel_err(full[3], part[3]) < TOL
    assert rel_err(full[1][k], part[1]) < TOL and rel_err(full[2][k], part[2]) < TOL
    assert torch.count_nonzero(full[1][~k]) == 0 and torch.count_nonzero(full[2][~k]) == 0


@pytest.mark.parametrize("li,le,lo,C,need", [(2, 2, 2, 64, (True, True, True)), (2, 3, 3, 128, (True, True, True)),
                                             (2, 2, 2, 64, (False, True, True)), (0, 3, 3, 128, (False, False, True))])
def test_message_adjoint_accumulates_gate_gradient(device, li, le, lo, C, need):
    """ictc_msg_bwd_accumulate: the gate gradient is added to the rows dgates holds (bitwise the stored rows
    plus ictc_msg_bwd's gate gradient), the other outputs are ictc_msg_bwd's; one-pass source-owned and
    two-kernel routes, masks and out-of-range ids."""
    from ictc_o3.ops import tensor_product as tpo
    N, E = 60, 2400
    f64, sh64, g64, src, dst, m64 = _graph(N, E, C, li, le, lo, 77, mask=True)
    src[::11] = N + 1
    spec = tpo.make_spec(li, le, lo, C)
    topo = tpo.Topology(src.to(device), dst.to(device), N)
    x, sh, gt = (t.float().to(device) for t in (f64, sh64, g64))
    m = m64.float().to(device)
    go = torch.randn(N, spec.out_components * C, device=device, generator=torch.Generator(device=device).manual_seed(3))
    dx0, dsh0, dg0 = tpo._msg_bwd_raw(spec, topo, x, sh, gt, m, go, need)
    held = torch.randn_like(gt)
    expect = held + dg0
    dx1, dsh1, dg1 = tpo._msg_bwd_raw(spec, topo, x, sh, gt, m, go, need, dg_into=held)
    assert dg1 is held and torch.equal(dg1, expect)
    for a, b in ((dx0, dx1), (dsh0, dsh1)):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)


def test_message_deterministic_bitwise(device):
    from ictc_o3 import PackedGraphMessage
    op = PackedGraphMessage.create(channels=64, input_lmax=2, edge_lmax=2, device=device)
    f64, sh64, g64, src, dst, _ = _graph(100, 5000, 64, 2, 2, 2, 5)
    x = [t.float().to(device).requires_grad_(True) for t in (f64, sh64, g64)]
    results = []
    for _ in range(2):
        out = op(*x, src.to(device), dst.to(device))
        grads = torch.autograd.grad(out, x, torch.ones_like(out))
        results.append((out, *grads))
    for a, b in zip(*results):
        assert torch.equal(a, b)


def test_message_isolated_nodes_and_empty(device):
    from ictc_o3 import PackedGraphMessage
    op = PackedGraphMessage.create(channels=32, input_lmax=2, edge_lmax=2, device=device)
    N = 10
    f = torch.randn(N, 32 * 9, device=device, requires_grad=True)
    e0 = torch.zeros(0, dtype=torch.int64, device=device)
    out = op(f, torch.zeros(0, 9, device=device), torch.zeros(0, op.gate_width, device=device), e0, e0)
    assert out.shape == (N, op.output_width) and torch.count_nonzero(out) == 0
    out.sum().backward()
    assert torch.count_nonzero(f.grad) == 0
    # all edges into node 0: every other output row is exactly zero
    f64, sh64, g64, src, _, _ = _graph(N, 50, 32, 2, 2, 2, 6)
    dst = torch.zeros(50, dtype=torch.int64)
    out = op(f64.float().to(device), sh64.float().to(device), g64.float().to(device), src.to(device), dst.to(device))
    ref = orc.message_packed(f64, sh64, g64, src, dst, None, 2, 2, 2, 32)
    assert rel_err(out, ref) < TOL
    assert torch.count_nonzero(out[1:]) == 0


def test_message_out_of_range_ids_contribute_nothing(device):
    from ictc_o3 import PackedGraphMessage
    op = PackedGraphMessage.create(channels=32, input_lmax=2, edge_lmax=2, device=device)
    N = 12
    f64, sh64, g64, src, dst, _ = _graph(N, 80, 32, 2, 2, 2, 7)
    bad_src, bad_dst = src.clone(), dst.clone()
    bad_src[::7] = N + 5
    bad_dst[3::11] = -1
    keep = (bad_src < N) & (bad_dst >= 0)
    ref = orc.message_packed(f64, sh64[keep], g64[keep], src[keep], dst[keep], None, 2, 2, 2, 32)
    x = [t.float().to(device).requires_grad_(True) for t in (f64, sh64, g64)]
    out = op(*x, bad_src.to(device), bad_dst.to(device))
    assert rel_err(out, ref) < TOL
    out.sum().backward()
    assert torch.count_nonzero(x[2].grad[~keep.to(device)]) == 0
    assert torch.count_nonzero(x[1].grad[~keep.to(device)]) == 0


def test_graph_message_dict_api(device):
    from ictc_o3 import EdgeTensorProduct, GraphMessage
    C, N, E = 16, 20, 120
    edge = EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, channels=C, device=device)
    gm = GraphMessage(edge.tp, input_lmax=2, edge_lmax=2)
    f64, sh64, g64, src, dst, _ = _graph(N, E, C, 2, 2, 2, 8)
    blocks = orc.unpack_ir_mul(f64, C, 2)
    feats = {l: blocks[l].float().to(device) for l in blocks}
    harm = {l: sh64[:, l * l:(l + 1) ** 2].reshape(E, 1, 2 * l + 1).float().to(device) for l in range(3)}
    out = gm(feats, harm, g64.float().to(device), src.to(device), dst.to(device))
    ref = orc.message_packed(f64, sh64, g64, src, dst, None, 2, 2, 2, C)
    paths = orc.natural_paths(2, 2, 2)
    _, _, counts = orc.path_tables(paths)
    packed = orc.pack_output({l: out[l].double().cpu() for l in out}, counts, C)
    assert rel_err(packed, ref) < TOL


def _morton_np(pos, spacing):
    """Stable argsort of the 30-bit Morton key of floor(pos / spacing) mod 1024 (bit i of axis d -> bit 3i+d)."""
    import numpy as np
    q = (np.floor(pos.astype(np.float32) * np.float32(1.0 / spacing)).astype(np.int64) & 0x3FF)
    key = np.zeros(len(pos), dtype=np.int64)
    for i in range(10):
        for d in range(3):
            key |= ((q[:, d] >> i) & 1) << (3 * i + d)
    return np.argsort(key, kind="stable")


def test_morton_order_matches_restatement(device):
    from ictc_o3.ops.tensor_product import morton_order
    g = torch.Generator().manual_seed(11)
    pos = (torch.rand(5000, 3, generator=g) * 80 - 20).float()
    got = morton_order(pos.to(device), 2.0).cpu().numpy()
    assert (got == _morton_np(pos.numpy(), 2.0)).all()
    assert morton_order(pos[:0].to(device), 2.0).numel() == 0


@pytest.mark.parametrize("li,le,lo,C", [(2, 2, 2, 64), (2, 3, 3, 128), (0, 2, 2, 17)])
def test_message_row_order_bitwise_identical(device, li, le, lo, C):
    """Visiting rows in a spatial or random order changes no bit of the output or of any gradient."""
    from ictc_o3 import PackedGraphMessage
    from ictc_o3.ops import tensor_product as tpo
    N, E = 300, 6000
    op = PackedGraphMessage.create(channels=C, input_lmax=li, edge_lmax=le, output_lmax=lo, device=device)
    f64, sh64, g64, src, dst, m64 = _graph(N, E, C, li, le, lo, 21, mask=True)
    s, d, m = src.to(device), dst.to(device), m64.float().to(device)
    pos = torch.rand(N, 3, generator=torch.Generator().manual_seed(4)).to(device) * 30
    results = []
    for rows in (None, "morton", "random"):
        topo = tpo.Topology(s, d, N, positions=pos if rows == "morton" else None)
        if rows == "random":
            topo.dst_rows = torch.randperm(N, generator=torch.Generator().manual_seed(5)).int().to(device)
            topo.src_rows = torch.randperm(N, generator=torch.Generator().manual_seed(6)).int().to(device)
        elif rows == "morton":
            topo.dst_rows = topo.src_rows
        x = [t.float().to(device).requires_grad_(True) for t in (f64, sh64, g64)]
        out = op(*x, s, d, m, topology=topo)
        grads = torch.autograd.grad(out, x, torch.cos(out))
        results.append((out, *grads))
    for other in results[1:]:
        for a, b in zip(results[0], other):
            assert torch.equal(a, b)


@pytest.mark.parametrize("which", [(1, 2), (0,), (0, 1, 2)])
def test_message_backward_without_edges(device, which):
    """E = 0: any subset of gradients comes back correctly shaped (dx zero, dsh and dg empty)."""
    from ictc_o3 import PackedGraphMessage
    op = PackedGraphMessage.create(channels=64, input_lmax=2, edge_lmax=2, output_lmax=2, device=device)
    x = torch.randn(7, 64 * 9, device=device, requires_grad=0 in which)
    sh = torch.zeros(0, 9, device=device, requires_grad=1 in which)
    g = torch.zeros(0, op.gate_width, device=device, requires_grad=2 in which)
    e = torch.zeros(0, dtype=torch.long, device=device)
    out = op(x, sh, g, e, e)
    assert out.shape == (7, op.output_width) and float(out.abs().max()) == 0.0
    grads = torch.autograd.grad(out.sum(), [t for t in (x, sh, g) if t.requires_grad], allow_unused=True)
    for t, d in zip([t for t in (x, sh, g) if t.requires_grad], grads):
        assert d is None or (d.shape == t.shape and (d.numel() == 0 or float(d.abs().max()) == 0.0))


@pytest.mark.parametrize("N,E,C,li,le,lo", [(64, 2000, 64, 2, 2, 2), (40, 500, 128, 2, 3, 3), (20, 150, 17, 1, 2, 2)])
def test_message_fixed_path_weight(device, N, E, C, li, le, lo):
    """Fixed non-unit path coefficients (the TP's weight [P, C]): forward, adjoint and gate-tangent adjoint
    against the float64 oracle with the weight folded into the gates (the same products).  The
    pipelined kernels (forward and gate-tangent adjoint at (2, 2, 2)) run a separate weighted loop."""
    from ictc_o3 import PackedGraphMessage
    from ictc_o3.ops import tensor_product as tpo
    op = PackedGraphMessage.create(channels=C, input_lmax=li, edge_lmax=le, output_lmax=lo, device=device)
    P = len(orc.natural_paths(li, le, lo))
    gen = torch.Generator().manual_seed(900 + N)
    w64 = 0.5 + torch.rand(P, C, generator=gen, dtype=torch.float64)
    with torch.no_grad():
        op.tp.weight.copy_(w64.float().to(device))
    spec = op.edge._prepare()
    assert spec.weight is not None
    f64, sh64, g64, src, dst, m64 = _graph(N, E, C, li, le, lo, 900 + N, mask=True)
    ref_in = [t.clone().requires_grad_(True) for t in (f64, sh64, g64)]
    gw = (ref_in[2].view(E, P, C) * w64).view(E, P * C)
    ref = orc.message_packed(ref_in[0], ref_in[1], gw, src, dst, m64, li, le, lo, C)
    x = [t.float().to(device).requires_grad_(True) for t in (f64, sh64, g64)]
    m = m64.float().to(device)
    out = op(*x, src.to(device), dst.to(device), m)
    assert rel_err(out, ref) < TOL
    go = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    torch.autograd.backward(ref, go)
    torch.autograd.backward(out, go.float().to(device))
    for a, b in zip(x, ref_in):
        assert rel_err(a.grad, b.grad) < TOL
    # gate-tangent adjoint: dr = sum over gates of dL/dgates * gdot (the weight is inside dL/dgates)
    topo = tpo.Topology(src.to(device), dst.to(device), N)
    gdot64 = torch.randn(g64.shape, generator=gen, dtype=torch.float64)
    xs, shs, gs = (t.detach() for t in x)
    dx, dsh, dr = tpo._msg_bwd_tangent_raw(spec, topo, xs, shs, gs, gdot64.float().to(device), m,
                                           go.float().to(device), (True, True))
    assert rel_err(dx, ref_in[0].grad) < TOL
    assert rel_err(dsh, ref_in[1].grad) < TOL
    assert rel_err(dr, (ref_in[2].grad * gdot64).sum(1)) < TOL


@pytest.mark.parametrize("inputs", [(0, 1, 2), (2,), (0,), (1, 2)])
def test_gate_link_partial_inputs_and_retained_graph(device, inputs):
    """Force-loss objective L = a.E + <dE/dx, v> (both the forward message's first-order adjoint and the
    mixed second derivative reach the gates): autograd.grad over a subset of the inputs, and two backward
    passes over one retained graph, give the float64 gradients, and the gate-gradient hand-off between the
    two passes (LINK_GATE_GRADIENTS) gives bitwise the gradients of autograd's own add."""
    from ictc_o3 import PackedGraphMessage
    from ictc_o3.ops import tensor_product as tp
    N, E, C = 24, 200, 64
    op = PackedGraphMessage.create(channels=C, input_lmax=2, edge_lmax=2, output_lmax=2, device=device)
    f64, sh64, g64, src, dst, m64 = _graph(N, E, C, 2, 2, 2, 91, mask=True)
    gen = torch.Generator().manual_seed(92)
    a64 = torch.randn(N, op.output_width, generator=gen, dtype=torch.float64)
    v64 = torch.randn(f64.shape, generator=gen, dtype=torch.float64)

    def objective(xs, fn, a, v):
        out = fn(*xs)
        (dx,) = torch.autograd.grad(out, xs[0], a, create_graph=True)
        return (out * a).sum() + (dx * v).sum()

    ref_x = [t.clone().requires_grad_(True) for t in (f64, sh64, g64)]
    ref = torch.autograd.grad(objective(ref_x, lambda p, q, r: orc.message_packed(
        p, q, r, src, dst, m64, 2, 2, 2, C), a64, v64), [ref_x[k] for k in inputs])
    s, d, m = src.to(device), dst.to(device), m64.float().to(device)
    a, v = a64.float().to(device), v64.float().to(device)
    results = {}
    for link in (True, False):
        tp.LINK_GATE_GRADIENTS = link
        try:
            xs = [t.float().to(device).requires_grad_(True) for t in (f64, sh64, g64)]
            L = objective(xs, lambda p, q, r: op(p, q, r, s, d, m), a, v)
            got = torch.autograd.grad(L, [xs[k] for k in inputs], retain_graph=True)
            again = torch.autograd.grad(L, [xs[k] for k in inputs])
        finally:
            tp.LINK_GATE_GRADIENTS = True
        for g1, g2, r in zip(got, again, ref):
            assert torch.equal(g1, g2)
            assert rel_err(g1, r) < TOL
        results[link] = got
    for g1, g2 in zip(results[True], results[False]):
        assert torch.equal(g1, g2)
