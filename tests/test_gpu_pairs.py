"""Shared radial-gate rows of an edge and its reverse (Topology.pair_edges, ictc_edge_pairs).

* The pairing equals a brute-force pairing on the host of the same rule: an
  edge with s < d (s == d: shift zero or lexicographically positive) owns a
  row; any other edge reads the row of its reverse, the first edge into s,
  in receiver-CSR order, with source d and shift -S, or owns a row when
  there is none; owners are numbered in edge order.  Symmetric periodic
  lists halve the rows; edges without a reverse and out-of-range ids own
  rows; every edge that reads another edge's row reads its reverse's.
* For a symmetric list the same lookup yields the source CSR (the reverses
  of each node's incoming edges, ranked into edge order): bitwise the stable
  sort over src; asymmetric lists, duplicates and bad ids fall back to the sort.
* Shared rows change no result bit: energies, forces and per-atom energies of
  the first-order (forces only) model route are bitwise those with one row
  per edge, on the fused and the materialised-gate message, for one periodic
  cell and a batch of cells; the parameter-gradient route (gates expanded
  per edge) is bitwise too.
"""
import pytest
import torch

from model_helpers import build_graph, fcc_cells

pytestmark = pytest.mark.gpu


def _brute_pairs(src, dst, sh, N):
    """Host restatement of the pairing rule: (gate_rows [E], reps [rows])."""
    src, dst = src.tolist(), dst.tolist()
    sh = [tuple(v) for v in sh.tolist()] if sh is not None else [(0.0, 0.0, 0.0)] * len(src)
    into = {}
    order = sorted(range(len(src)), key=lambda e: (dst[e] if 0 <= dst[e] < N else N, e))   # stable by receiver
    for e in order:
        into.setdefault(dst[e], []).append(e)
    def reader(e):
        if src[e] != dst[e]:
            return src[e] > dst[e]
        nz = [v for v in sh[e] if v != 0]
        return bool(nz) and nz[0] < 0

    partner = []
    for e in range(len(src)):
        p = -1
        if 0 <= src[e] < N and 0 <= dst[e] < N and reader(e):
            want = tuple(-v for v in sh[e])
            for q in into.get(src[e], []):
                if q != e and src[q] == dst[e] and sh[q] == want:
                    p = q
                    break
        partner.append(p)
    canon = [p < 0 for p in partner]
    idx, reps = [], []
    for e in range(len(src)):
        idx.append(len(reps))
        if canon[e]:
            reps.append(e)
    rows = [idx[e] if canon[e] else idx[partner[e]] for e in range(len(src))]
    return torch.tensor(rows), torch.tensor(reps)


def _check_source_csr(topo, src, N, device, symmetric):
    """The source CSR pair_edges derives from the reverse lookup (symmetric lists) equals the stable sort over
    src bit for bit; other lists fall back to that sort."""
    from ictc_o3.ops import tensor_product as tpo
    topo._resolve()
    assert (topo._by_src is not None) == symmetric
    got = topo.by_src
    want = tpo.Csr(src.to(device), N)
    E = src.numel()
    assert torch.equal(got.ptr.cpu(), want.ptr.cpu())
    assert torch.equal(got.order[:E].cpu(), want.order[:E].cpu())


def _pairs(src, dst, sh, N, device):
    from ictc_o3.ops import tensor_product as tpo
    topo = tpo.Topology(src.to(device), dst.to(device), N)
    topo.pair_edges(None if sh is None else sh.float().to(device))
    return topo


@pytest.mark.parametrize("case", ["periodic", "self_images", "one_sided", "duplicates", "bad_ids", "no_shifts"])
def test_pairing_matches_brute_force(device, case):
    # self_images: one FCC unit cell (3.4 A box) under a 4.5 A cutoff, so atoms see their own images
    pos, Z, batch, cell = fcc_cells(1 if case == "self_images" else 2, 0.1, 0.3, 4, 3)
    src, dst, sh = build_graph(pos, batch, cell, 4.5)
    if case == "self_images":
        assert bool((src == dst).any())
    N, E = pos.shape[0], src.numel()
    g = torch.Generator().manual_seed(7)
    if case == "one_sided":
        keep = torch.rand(E, generator=g) < 0.8
        src, dst, sh = src[keep], dst[keep], sh[keep]
    elif case == "duplicates":
        extra = torch.randint(0, E, (E // 10,), generator=g)
        src, dst, sh = torch.cat([src, src[extra]]), torch.cat([dst, dst[extra]]), torch.cat([sh, sh[extra]])
        perm = torch.randperm(src.numel(), generator=g)
        src, dst, sh = src[perm], dst[perm], sh[perm]
    elif case == "bad_ids":
        src, dst = src.clone(), dst.clone()
        src[::17] = N + 3
        dst[5::23] = -1
    elif case == "no_shifts":
        # an open cluster: all pairs within the cutoff, no images
        d = torch.cdist(pos, pos)
        near = (d < 4.5) & ~torch.eye(N, dtype=torch.bool)
        dst, src = torch.nonzero(near & near.t(), as_tuple=True)     # cdist is not exactly symmetric
        sh = None
    topo = _pairs(src, dst, sh, N, device)
    rows, reps = _brute_pairs(src, dst, sh, N)
    _check_source_csr(topo, src, N, device, symmetric=case in ("periodic", "self_images", "no_shifts"))
    if case in ("periodic", "self_images", "no_shifts"):
        assert reps.numel() * 2 == src.numel()
    if reps.numel() == src.numel():
        assert topo.gate_rows is None
        return
    assert torch.equal(topo.gate_rows.long().cpu(), rows)
    assert torch.equal(topo.gate_reps.long().cpu(), reps)
    # gate_input: the lengths of the gate rows, the gather kept for the same (unchanged) lengths
    r = torch.rand(src.numel(), device=device)
    g1 = topo.gate_input(r)
    assert torch.equal(g1.cpu(), r.cpu()[reps])
    assert topo.gate_input(r.view_as(r)) is g1
    r.mul_(2.0)                                   # an in-place change is seen
    g2 = topo.gate_input(r)
    assert g2 is not g1 and torch.equal(g2.cpu(), r.cpu()[reps])
    other_r = torch.rand(src.numel(), device=device)
    assert torch.equal(topo.gate_input(other_r).cpu(), other_r.cpu()[reps])
    # each row is its owner's; an edge reading another edge's row reads its reverse's
    assert torch.equal(rows[reps], torch.arange(reps.numel()))
    owner = reps[rows]
    other = owner != torch.arange(src.numel())
    assert torch.equal(src[other], dst[owner[other]]) and torch.equal(dst[other], src[owner[other]])
    if sh is not None:
        assert torch.equal(sh[other].float(), -sh[owner[other]].float())


def _model(device, channels=64, lmax=2):
    from mace_ictc.hp import create_model
    torch.manual_seed(3)
    return create_model(channels=channels, lmax=lmax, atomic_numbers=(1, 6, 8), cutoff=4.5, avg_num_neighbors=38.0,
                        device=device)


def _run(model, pos, Z, batch, src, dst, sh, cell, device, pair, fused):
    from ictc_o3.ops import tensor_product as tpo
    from mace_ictc.hp import energy_and_forces
    old = tpo.PAIR_GATES, tpo.FUSED_GATES
    tpo.PAIR_GATES, tpo.FUSED_GATES = pair, fused
    try:
        out = energy_and_forces(model, pos.float().to(device), Z.to(device), batch.to(device), src.to(device),
                                dst.to(device), sh.float().to(device), cell.float().to(device))
        torch.cuda.synchronize()
        return out
    finally:
        tpo.PAIR_GATES, tpo.FUSED_GATES = old


@pytest.mark.parametrize("fused", ["always", "never"])
@pytest.mark.parametrize("cells", [1, 3])
def test_shared_rows_bitwise(device, fused, cells):
    model = _model(device)
    pos, Z, batch, cell = fcc_cells(3 if cells == 1 else 2, 0.1, 0.3, 11, 3, cells=cells)
    src, dst, sh = build_graph(pos, batch, cell, 4.5)
    a = _run(model, pos, Z, batch, src, dst, sh, cell, device, True, fused)
    b = _run(model, pos, Z, batch, src, dst, sh, cell, device, False, fused)
    for k in ("energy", "forces", "atomic_energy"):
        assert torch.equal(a[k], b[k]), k


def test_shared_rows_parameter_gradients_bitwise(device):
    """A backward asking for parameter gradients after the forces-only forward expands the shared rows."""
    from ictc_o3.ops import tensor_product as tpo
    model = _model(device)
    pos, Z, batch, cell = fcc_cells(2, 0.1, 0.3, 5, 3)
    src, dst, sh = build_graph(pos, batch, cell, 4.5)
    grads = []
    for pair in (True, False):
        old = tpo.PAIR_GATES
        tpo.PAIR_GATES = pair
        try:
            model.zero_grad(set_to_none=True)
            p = pos.float().to(device).requires_grad_(True)
            e = model(p, Z.to(device), batch.to(device), src.to(device), dst.to(device), sh.float().to(device),
                      cell.float().to(device), second_order=False, forces_only=True).sum()
            e.backward()
            grads.append([p.grad.clone()] + [q.grad.clone() for q in model.parameters() if q.grad is not None])
        finally:
            tpo.PAIR_GATES = old
    assert len(grads[0]) == len(grads[1]) > 5
    for x, y in zip(*grads):
        assert torch.equal(x, y)


@pytest.mark.parametrize("cells", [1, 3])
def test_paired_edges_have_bitwise_equal_lengths(device, cells):
    """The premise of shared rows: with the model's own shift vectors (mace_ictc.hp.model.shift_vectors) and
    edge geometry, every edge reading its reverse's gate row has bitwise that edge's length."""
    from ictc_o3.ops.geometry import edge_geometry
    from mace_ictc.hp.model import shift_vectors
    pos, Z, batch, cell = fcc_cells(3 if cells == 1 else 2, 0.1, 0.3, 13, 3, cells=cells)
    src, dst, sh = build_graph(pos, batch, cell, 4.5)
    topo = _pairs(src, dst, sh, pos.shape[0], device)
    assert topo.gate_rows is not None
    shift = shift_vectors(sh.float().to(device), cell.float().to(device), batch.to(device), src.to(device))
    r, _, _ = edge_geometry(pos.float().to(device), shift, topo, 4.5)
    rows, reps = topo.gate_rows.long(), topo.gate_reps.long()
    owner = reps[rows]
    other = owner != torch.arange(src.numel(), device=device)
    assert int(other.sum()) * 2 == src.numel()
    assert torch.equal(r[other], r[owner[other]])
