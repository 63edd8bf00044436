"""Fused radial-gate message (gates projected per edge tile inside the message kernels).

The forward and the energy-and-forces adjoint (features, harmonics and edge
lengths) against the float64 oracle: the radial MLP restatement gives the
gates, the message oracle the output, float64 autograd the gradients
(1e-5 relative, max-norm).  Covered: every compiled input degree (path groups
l1 = 0, 1, 2), two channel groups, masks, unsorted edges, out-of-range ids,
isolated nodes, a spatial (Morton) row order, edges beyond the cutoff; the
route that asks for weight gradients; agreement with the materialised-gate
route; bitwise repeatability.
"""
import math

import pytest
import torch

import ictc_oracle as orc
import model_oracle as mo
from helpers import rel_err, unit_vectors
from test_gpu_gate_tangent import _fc
from test_gpu_radial_mlp import _ref_gates

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.fixture(autouse=True)
def _fused_everywhere():
    from ictc_o3.ops import tensor_product as tpo
    old, tpo.FUSED_GATES = tpo.FUSED_GATES, "always"
    yield
    tpo.FUSED_GATES = old
CFG = (4.5, 5, mo.SILU)


def _case(N, E, C, li, seed, mask=True, bad_ids=True):
    g = torch.Generator().manual_seed(seed)
    P = len(orc.natural_paths(li, 2, 2))
    x = torch.randn(N, C * (li + 1) ** 2, generator=g, dtype=torch.float64)
    sh = torch.cat(orc.direction_harmonics(unit_vectors(E, seed + 1), 2), -1)
    r = torch.rand(E, generator=g, dtype=torch.float64) * 4.6 + 0.4          # some beyond the 4.5 cutoff
    src = torch.randint(0, N - 2, (E,), generator=g)                          # nodes N-2, N-1 send nothing
    dst = torch.randint(0, N - 1, (E,), generator=g)                          # node N-1 receives nothing
    if bad_ids:
        src[::13] = N + 1
        dst[5::17] = -2
    m = (torch.rand(E, generator=g) > 0.3).double() if mask else None
    sizes = [8, 64, 64, 64, P * C]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    return x, sh, r, src, dst, m, Ws


def _oracle(x, sh, r, src, dst, m, Ws, li, C, go, keep):
    xr, shr, rr = (t.clone().requires_grad_(True) for t in (x, sh, r))
    gates = _ref_gates(rr, Ws, 4.5, 5)
    k = keep
    out = orc.message_packed(xr, shr[k], gates[k], src[k], dst[k], None if m is None else m[k], li, 2, 2, C)
    torch.autograd.backward(out, go)
    return out.detach(), xr.grad, shr.grad, rr.grad


def _product(x, sh, r, src, dst, m, Ws, li, C, go, device, positions=None, params=False, dfeatures=True):
    from ictc_o3.ops import tensor_product as tpo
    fc = _fc(Ws[-1].shape[0], Ws, device)
    for p in fc.parameters():
        p.requires_grad_(params)
    spec = tpo.make_spec(li, 2, 2, C)
    topo = tpo.Topology(src.to(device), dst.to(device), x.shape[0], positions=positions)
    xd, shd, rd = (t.float().to(device).requires_grad_(True) for t in (x, sh, r))
    xd.requires_grad_(dfeatures)
    md = None if m is None else m.float().to(device)
    out = tpo.radial_message(xd, shd, rd, fc, spec, topo, md, CFG)
    wrt = ([xd] if dfeatures else []) + [shd, rd] + ([p for p in fc.parameters()] if params else [])
    grads = torch.autograd.grad(out, wrt, go.float().to(device))
    return out.detach(), grads, out.grad_fn


CASES = [(64, 2000, 64, 2, True), (50, 1500, 64, 0, False), (40, 900, 128, 2, True), (30, 700, 64, 1, True),
         (20, 37, 64, 2, True)]


@pytest.mark.parametrize("N,E,C,li,mask", CASES)
def test_fused_message_matches_oracle(device, N, E, C, li, mask):
    x, sh, r, src, dst, m, Ws = _case(N, E, C, li, 100 + N + li, mask)
    NO = orc.path_tables(orc.natural_paths(li, 2, 2))[2]
    go = torch.randn(N, sum(c * (2 * l + 1) for l, c in NO.items()) * C,
                     generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    keep = (src >= 0) & (src < N) & (dst >= 0) & (dst < N)
    ref, dx0, dsh0, dr0 = _oracle(x, sh, r, src, dst, m, Ws, li, C, go, keep)
    out, (dx, dsh, dr), fn = _product(x, sh, r, src, dst, m, Ws, li, C, go, device)
    assert type(fn).__name__.startswith("FusedRadialMessage")
    assert rel_err(out, ref) < TOL
    assert rel_err(dx, dx0) < TOL
    assert rel_err(dsh, dsh0) < TOL
    assert rel_err(dr, dr0) < TOL
    assert torch.count_nonzero(dr[~keep.to(device)]) == 0
    assert torch.count_nonzero(dsh[~keep.to(device)]) == 0
    # repeatable bit for bit
    out2, (dx2, dsh2, dr2), _ = _product(x, sh, r, src, dst, m, Ws, li, C, go, device)
    assert torch.equal(out, out2) and torch.equal(dx, dx2) and torch.equal(dsh, dsh2) and torch.equal(dr, dr2)


@pytest.mark.parametrize("N,E,C,mask", [(50, 1500, 64, True), (40, 1100, 128, True), (33, 29, 64, False),
                                         (10, 1500, 64, True)])
def test_fused_scalar_input_receiver_adjoint(device, N, E, C, mask):
    """Input degree 0 without a feature gradient (the model's first layer): the receiver-owned adjoint
    (harmonic and edge-length gradients only) and the forward, against the oracle; partial edge tiles,
    two channel groups, masks, out-of-range ids, and receivers with several 64-edge chunks (N = 10)."""
    li = 0
    x, sh, r, src, dst, m, Ws = _case(N, E, C, li, 300 + N, mask)
    go = torch.randn(N, 9 * C, generator=torch.Generator().manual_seed(9), dtype=torch.float64)
    keep = (src >= 0) & (src < N) & (dst >= 0) & (dst < N)
    ref, _, dsh0, dr0 = _oracle(x, sh, r, src, dst, m, Ws, li, C, go, keep)
    out, (dsh, dr), fn = _product(x, sh, r, src, dst, m, Ws, li, C, go, device, dfeatures=False)
    assert type(fn).__name__.startswith("FusedRadialMessage")
    assert rel_err(out, ref) < TOL
    assert rel_err(dsh, dsh0) < TOL
    assert rel_err(dr, dr0) < TOL
    assert torch.count_nonzero(dr[~keep.to(device)]) == 0
    assert torch.count_nonzero(dsh[~keep.to(device)]) == 0
    out2, (dsh2, dr2), _ = _product(x, sh, r, src, dst, m, Ws, li, C, go, device, dfeatures=False)
    assert torch.equal(out, out2) and torch.equal(dsh, dsh2) and torch.equal(dr, dr2)


def test_fused_message_spatial_rows_and_unfused_route(device):
    """A lattice-like graph in spatial row order; the materialised-gate route gives the same values."""
    from ictc_o3.ops import tensor_product as tpo
    from mace_ictc.hp import radius_graph_pbc
    from model_helpers import fcc_cells
    pos, _, _, cell = fcc_cells(4, 0.1, 0.3, 3, 1)
    src, dst, shf = radius_graph_pbc(pos, cell[0], 4.5)
    vec = pos[dst] - pos[src] + shf.double() @ cell[0]
    r = vec.norm(dim=1)
    sh = torch.cat(orc.direction_harmonics(vec / r[:, None], 2), -1)
    N, E, C = pos.shape[0], src.numel(), 64
    g = torch.Generator().manual_seed(5)
    x = torch.randn(N, 9 * C, generator=g, dtype=torch.float64)
    sizes = [8, 64, 64, 64, 11 * C]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    go = torch.randn(N, 35 * C, generator=g, dtype=torch.float64)
    keep = torch.ones(E, dtype=torch.bool)
    ref, dx0, dsh0, dr0 = _oracle(x, sh, r, src, dst, None, Ws, 2, C, go, keep)
    out, (dx, dsh, dr), fn = _product(x, sh, r, src, dst, None, Ws, 2, C, go, device, positions=pos.float().to(device))
    assert type(fn).__name__.startswith("FusedRadialMessage")
    assert rel_err(out, ref) < TOL and rel_err(dx, dx0) < TOL and rel_err(dsh, dsh0) < TOL and rel_err(dr, dr0) < TOL
    tpo.FUSED_GATES = "never"
    try:
        out1, (dx1, dsh1, dr1), fn1 = _product(x, sh, r, src, dst, None, Ws, 2, C, go, device)
    finally:
        tpo.FUSED_GATES = "always"
    assert not type(fn1).__name__.startswith("FusedRadialMessage")
    for a, b in ((out, out1), (dx, dx1), (dsh, dsh1), (dr, dr1)):
        assert rel_err(a, b.double().cpu()) < TOL


def test_fused_message_weight_gradient_route(device):
    """Weight gradients asked for: gates rebuilt from h3, ordinary adjoints; all gradients vs the oracle."""
    N, E, C, li = 48, 1200, 64, 2
    x, sh, r, src, dst, m, Ws = _case(N, E, C, li, 77, True, bad_ids=False)
    go = torch.randn(N, 35 * C, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    Wl = [W.clone().requires_grad_(True) for W in Ws]
    xr, shr, rr = (t.clone().requires_grad_(True) for t in (x, sh, r))
    ref = orc.message_packed(xr, shr, _ref_gates(rr, Wl, 4.5, 5), src, dst, m, li, 2, 2, C)
    torch.autograd.backward(ref, go)
    out, grads, fn = _product(x, sh, r, src, dst, m, Ws, li, C, go, device, params=True)
    assert type(fn).__name__.startswith("FusedRadialMessage")
    assert rel_err(out, ref.detach()) < TOL
    for a, b in zip(grads, [xr.grad, shr.grad, rr.grad] + [W.grad for W in Wl]):
        assert rel_err(a, b) < TOL


@pytest.mark.parametrize("li", [0, 2])
def test_fused_message_without_edges(device, li):
    """E = 0: zero output rows, zero feature gradient, empty harmonic and edge-length gradients."""
    from ictc_o3.ops import tensor_product as tpo
    N, C = 9, 64
    P = len(orc.natural_paths(li, 2, 2))
    sizes = [8, 64, 64, 64, P * C]
    Ws = [torch.randn(o, i, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    fc = _fc(P * C, Ws, device)
    spec = tpo.make_spec(li, 2, 2, C)
    e = torch.zeros(0, dtype=torch.long, device=device)
    topo = tpo.Topology(e, e, N)
    x = torch.randn(N, C * (li + 1) ** 2, device=device, requires_grad=True)
    sh = torch.zeros(0, 9, device=device, requires_grad=True)
    r = torch.zeros(0, device=device, requires_grad=True)
    out = tpo.radial_message(x, sh, r, fc, spec, topo, None, CFG)
    assert type(out.grad_fn).__name__.startswith("FusedRadialMessage")
    assert out.shape == (N, spec.out_components * C) and float(out.abs().max()) == 0.0
    dx, dsh, dr = torch.autograd.grad(out, [x, sh, r], torch.ones_like(out))
    assert float(dx.abs().max()) == 0.0 and dsh.shape == (0, 9) and dr.shape == (0,)
