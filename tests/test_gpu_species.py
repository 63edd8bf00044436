"""Species form of the first layer's radial message (SpeciesRadialMessage, ictc_species_message_fwd/_bwd).

The features of input degree 0 are a function of the species, x = xtab[species]; the
forward and the energy-and-forces adjoint (harmonics and edge lengths) are checked
against the float64 oracle (radial MLP restatement, message oracle, autograd;
1e-5 relative, max-norm).  Covered: 1 to 4 species (6: the fallback route), 16 to 256 channels, masks,
out-of-range source / receiver ids, an out-of-range species, isolated nodes,
receivers with several 64-edge chunks, a Morton row order, shared gate rows
(edge pairs), no edges; the route that asks for feature and weight gradients (the
general adjoint); agreement with the fused route; bitwise repeatability.
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
CFG = (4.5, 5, mo.SILU)


def _case(N, E, C, S, seed, mask=True, bad_ids=True):
    g = torch.Generator().manual_seed(seed)
    xtab = torch.randn(S, C, generator=g, dtype=torch.float64)
    species = torch.randint(0, S, (N,), generator=g)
    sh = torch.cat(orc.direction_harmonics(unit_vectors(max(E, 1), seed + 1), 2), -1)[:E]
    r = torch.rand(E, generator=g, dtype=torch.float64) * 4.6 + 0.4          # some beyond the 4.5 cutoff
    src = torch.randint(0, max(N - 2, 1), (E,), generator=g)                 # nodes N-2, N-1 send nothing
    dst = torch.randint(0, max(N - 1, 1), (E,), generator=g)                 # node N-1 receives nothing
    if bad_ids and E:
        src[::13] = N + 1
        dst[5::17] = -2
    m = (torch.rand(E, generator=g) > 0.3).double() if mask else None
    sizes = [8, 64, 64, 64, 3 * C]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    return xtab, species, sh, r, src, dst, m, Ws


def _oracle(x, sh, r, src, dst, m, Ws, C, go):
    keep = (src >= 0) & (src < x.shape[0]) & (dst >= 0) & (dst < x.shape[0])
    xr, shr, rr = (t.clone().requires_grad_(True) for t in (x, sh, r))
    gates = _ref_gates(rr, Ws, 4.5, 5)
    k = keep
    out = orc.message_packed(xr, shr[k], gates[k], src[k], dst[k], None if m is None else m[k], 0, 2, 2, C)
    if out.requires_grad:
        torch.autograd.backward(out, go)
    return out.detach(), xr.grad, shr.grad, rr.grad, keep


def _product(xtab, species, sh, r, src, dst, m, Ws, C, go, device, positions=None, pair_shifts=None,
             dfeatures=False, params=False, table=True, x=None):
    """x: the features when they are not xtab[species] (built on the host, so an out-of-table species id
    never reaches a device gather)."""
    from ictc_o3.ops import tensor_product as tpo
    fc = _fc(Ws[-1].shape[0], Ws, device)
    for p in fc.parameters():
        p.requires_grad_(params)
    spec = tpo.make_spec(0, 2, 2, C)
    topo = tpo.Topology(src.to(device), dst.to(device), species.shape[0], positions=positions)
    if pair_shifts is not None:
        topo.pair_edges(pair_shifts)
    xt = xtab.float().to(device)
    sp = species.to(device)
    xd = (xtab[species] if x is None else x).float().to(device).requires_grad_(dfeatures)
    shd, rd = (t.float().to(device).requires_grad_(True) for t in (sh, r))
    md = None if m is None else m.float().to(device)
    out = tpo.radial_message(xd, shd, rd, fc, spec, topo, md, CFG, species=(xt, sp) if table else None)
    wrt = ([xd] if dfeatures else []) + [shd, rd] + ([p for p in fc.parameters()] if params else [])
    grads = torch.autograd.grad(out, wrt, go.float().to(device)) if sh.shape[0] else [None] * len(wrt)
    return out.detach(), grads, out.grad_fn


CASES = [(64, 2000, 64, 3, True), (50, 1500, 128, 1, False), (40, 900, 32, 4, True), (30, 600, 64, 6, True), (10, 1500, 64, 3, True),
         (33, 29, 16, 3, True), (20, 400, 256, 2, True)]


@pytest.mark.parametrize("N,E,C,S,mask", CASES)
def test_species_message_matches_oracle(device, N, E, C, S, mask):
    xtab, species, sh, r, src, dst, m, Ws = _case(N, E, C, S, 500 + N + S, mask)
    go = torch.randn(N, 9 * C, generator=torch.Generator().manual_seed(11), dtype=torch.float64)
    ref, _, dsh0, dr0, keep = _oracle(xtab[species], sh, r, src, dst, m, Ws, C, go)
    print(f"[species N={N} E={E} C={C} S={S} mask={mask}]", flush=True)
    out, (dsh, dr), fn = _product(xtab, species, sh, r, src, dst, m, Ws, C, go, device)
    # more species than the species form holds (4): the fused / materialised route, same results
    assert type(fn).__name__.startswith("SpeciesRadialMessage") == (S <= 4)
    assert rel_err(out, ref) < TOL
    assert rel_err(dsh, dsh0) < TOL
    assert rel_err(dr, dr0) < TOL
    assert torch.count_nonzero(dr[~keep.to(device)]) == 0
    assert torch.count_nonzero(dsh[~keep.to(device)]) == 0
    out2, (dsh2, dr2), _ = _product(xtab, species, sh, r, src, dst, m, Ws, C, go, device)
    assert torch.equal(out, out2) and torch.equal(dsh, dsh2) and torch.equal(dr, dr2)


def test_species_message_rows_pairs_and_fused_agreement(device):
    """Morton row order and shared gate rows (a periodic FCC graph), against the oracle and the fused route."""
    from model_helpers import build_graph, fcc_cells
    pos, Z, batch, cell = fcc_cells(2, 0.1, 0.3, 21, 3)
    src, dst, shifts = build_graph(pos, batch, cell, 4.5)
    N, E, C, S = pos.shape[0], src.numel(), 64, 3
    g = torch.Generator().manual_seed(22)
    xtab = torch.randn(S, C, generator=g, dtype=torch.float64)
    species = torch.randint(0, S, (N,), generator=g)
    vec = pos[dst] - pos[src] + shifts.double() @ cell[0]
    r = vec.norm(dim=1)
    sh = torch.cat(orc.direction_harmonics(vec / r[:, None], 2), -1)
    sizes = [8, 64, 64, 64, 3 * C]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    go = torch.randn(N, 9 * C, generator=g, dtype=torch.float64)
    ref, _, dsh0, dr0, _ = _oracle(xtab[species], sh, r, src, dst, None, Ws, C, go)
    kw = dict(positions=pos.float().to(device), pair_shifts=shifts.float().to(device))
    out, (dsh, dr), fn = _product(xtab, species, sh, r, src, dst, None, Ws, C, go, device, **kw)
    assert type(fn).__name__.startswith("SpeciesRadialMessage")
    assert rel_err(out, ref) < TOL and rel_err(dsh, dsh0) < TOL and rel_err(dr, dr0) < TOL
    outf, (dshf, drf), fnf = _product(xtab, species, sh, r, src, dst, None, Ws, C, go, device, table=False, **kw)
    assert type(fnf).__name__.startswith("FusedRadialMessage")
    assert rel_err(out, outf.double().cpu()) < TOL and rel_err(dsh, dshf.double().cpu()) < TOL
    assert rel_err(dr, drf.double().cpu()) < TOL


def test_species_message_general_route_and_bad_species(device):
    """Feature and weight gradients asked for: the general adjoint (features from x), against the oracle;
    a species id outside the table makes that node send nothing."""
    N, E, C, S = 40, 900, 64, 3
    xtab, species, sh, r, src, dst, m, Ws = _case(N, E, C, S, 77)
    go = torch.randn(N, 9 * C, generator=torch.Generator().manual_seed(12), dtype=torch.float64)
    ref, dx0, dsh0, dr0, _ = _oracle(xtab[species], sh, r, src, dst, m, Ws, C, go)
    out, grads, fn = _product(xtab, species, sh, r, src, dst, m, Ws, C, go, device, dfeatures=True, params=True)
    assert type(fn).__name__.startswith("SpeciesRadialMessage")
    dx, dsh, dr = grads[:3]
    assert rel_err(out, ref) < TOL and rel_err(dx, dx0) < TOL
    assert rel_err(dsh, dsh0) < TOL and rel_err(dr, dr0) < TOL
    # node 3 carries species S (outside the table): its edges contribute nothing
    bad = species.clone()
    bad[3] = S
    x_bad = xtab[species].clone()
    x_bad[3] = 0.0
    ref_b, _, dsh_b, dr_b, _ = _oracle(x_bad, sh, r, src, dst, m, Ws, C, go)
    out_b, (dsh2, dr2), _ = _product(xtab, bad, sh, r, src, dst, m, Ws, C, go, device, x=x_bad)
    assert rel_err(out_b, ref_b) < TOL and rel_err(dsh2, dsh_b) < TOL and rel_err(dr2, dr_b) < TOL


def test_species_message_without_edges(device):
    N, C, S = 12, 64, 3
    xtab, species, sh, r, src, dst, m, Ws = _case(N, 0, C, S, 5, bad_ids=False)
    go = torch.randn(N, 9 * C, generator=torch.Generator().manual_seed(13), dtype=torch.float64)
    out, _, fn = _product(xtab, species, sh, r, src, dst, m, Ws, C, go, device)
    assert out.shape == (N, 9 * C) and torch.count_nonzero(out) == 0
