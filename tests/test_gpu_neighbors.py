"""GPU cell-list neighbour search vs the torch formulation and brute force.

The HIP kernels must emit exactly the torch formulation's edges, in the same
(receiver-sorted) order, with identical shifts; the edge set is also checked
against an all-images brute force on a small triclinic cell.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _fcc(n, a, jitter, seed):
    g = torch.Generator().manual_seed(seed)
    base = torch.tensor([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]], dtype=torch.float64)
    grid = torch.stack(torch.meshgrid(*[torch.arange(n)] * 3, indexing="ij"), -1).reshape(-1, 3).double()
    pos = (grid[:, None, :] + base[None]).reshape(-1, 3) * a
    pos = pos + (torch.rand(pos.shape, generator=g, dtype=torch.float64) * 2 - 1) * jitter
    return pos.float(), (torch.eye(3, dtype=torch.float64) * a * n).float()


@pytest.mark.parametrize("n,cutoff,seed", [(8, 4.5, 0), (12, 5.0, 1), (6, 4.5, 2)])
def test_cell_list_matches_torch(device, n, cutoff, seed):
    from mace_ictc.hp.neighbors import _radius_graph_torch, radius_graph_pbc
    pos, cell = _fcc(n, 3.42, 0.3, seed)
    pos = pos - 5.0          # atoms outside the home cell exercise the image shifts
    s1, d1, h1 = radius_graph_pbc(pos.to(device), cell.to(device), cutoff)
    s0, d0, h0 = _radius_graph_torch(pos.to(device), cell.to(device), cutoff)
    assert torch.equal(s1, s0) and torch.equal(d1, d0) and torch.equal(h1, h0)
    assert bool((d1[1:] >= d1[:-1]).all())


def test_fill_capacity_from_earlier_counts(device):
    """Repeated calls on one kind of system fill arrays sized by the previous count before reading the new one:
    the same edges as the torch formulation when the count fits, when it shrinks, and when it grows past the
    estimate (the atoms gathered into a smaller region, about twice the pairs: the exact-size refill)."""
    from mace_ictc.hp import neighbors as nb
    pos, cell = _fcc(8, 3.42, 0.3, 4)
    nb._fill_capacity.clear()
    cases = [pos, pos + 0.01, pos * 0.98, pos * 0.6]
    counts = []
    for p in cases:
        s1, d1, h1 = nb.radius_graph_pbc(p.to(device), cell.to(device), 4.5)
        s0, d0, h0 = nb._radius_graph_torch(p.to(device), cell.to(device), 4.5)
        assert torch.equal(s1, s0) and torch.equal(d1, d0) and torch.equal(h1, h0)
        assert s1.is_contiguous() and h1.is_contiguous()
        counts.append(s1.numel())
    assert counts[3] > counts[0] + counts[0] // 32 + 1024     # the last case ran the refill
    assert len(nb._fill_capacity) == 1


def test_triclinic_against_brute_force(device):
    from mace_ictc.hp.neighbors import radius_graph_pbc
    g = torch.Generator().manual_seed(5)
    cell = torch.tensor([[14.0, 0.0, 0.0], [3.0, 13.5, 0.0], [-2.0, 1.5, 14.2]])
    frac = torch.rand(300, 3, generator=g, dtype=torch.float64)
    pos = (frac.float() @ cell) + 1.7
    s, d, h = radius_graph_pbc(pos.to(device), cell.to(device), 4.2)
    got = {(int(a), int(b), tuple(int(x) for x in v)) for a, b, v in zip(s.cpu(), d.cpu(), h.cpu().round())}
    want = set()
    imgs = torch.tensor([[i, j, k] for i in (-1, 0, 1) for j in (-1, 0, 1) for k in (-1, 0, 1)], dtype=torch.float64)
    P, Cd = pos.double(), cell.double()
    for dst in range(300):
        vec = P[dst][None, None, :] - P[None, :, :] + (imgs @ Cd)[:, None, :]   # [27, N, 3]
        r2 = (vec * vec).sum(-1)
        for a, b in torch.nonzero((r2 < 4.2 ** 2) & (r2 > 1e-20)).tolist():
            want.add((b, dst, tuple(int(x) for x in imgs[a].tolist())))
    assert got == want


def test_receiver_sorted_mark_skips_sort(device):
    """The neighbour list marks its dst as receiver-sorted: Topology then builds only the receiver CSR
    pointers (order = identity), equal to the sorted build; an in-place change of dst clears the mark."""
    from ictc_o3.ops import tensor_product as tpo
    from mace_ictc.hp.neighbors import radius_graph_pbc
    pos, cell = _fcc(6, 3.42, 0.3, 4)
    s, d, _ = radius_graph_pbc(pos.to(device), cell.to(device), 4.5)
    N = pos.shape[0]
    assert tpo.receiver_sorted(d, N) and not tpo.receiver_sorted(d, N + 1)
    fast = tpo.Topology(s, d, N)
    assert fast.by_dst.order is None
    full = tpo.Csr(d, N)
    assert torch.equal(fast.by_dst.ptr, full.ptr)
    assert torch.equal(full.order[:d.numel()].long().cpu(), torch.arange(d.numel()))
    # the position adjoint of the edge geometry through the identity order is bitwise the sorted CSR's
    from ictc_o3.ops.geometry import edge_geometry
    slow = tpo.Topology(s, d.clone(), N)
    assert slow.by_dst.order is not None
    grads = []
    for topo in (fast, slow):
        p = pos.to(device).requires_grad_(True)
        r, n, _ = edge_geometry(p, None, topo, 4.5)
        (r.sum() + (n * n.flip(0)).sum()).backward()
        grads.append(p.grad)
    assert torch.equal(grads[0], grads[1])
    d.add_(0)
    assert not tpo.receiver_sorted(d, N)
    assert tpo.Topology(s, d, N).by_dst.order is not None


def test_host_cell_copy_follows_views_and_versions(device):
    """The cached host copy of a device cell (no host sync per step) is reused only for the same base
    tensor, view and version: a fresh `cell[0]` view hits, an in-place update misses."""
    import mace_ictc.hp.neighbors as nb
    cell = torch.eye(3, device=device)[None] * 4.0
    a = nb._host_cell(cell[0])
    assert nb._host_cell(cell[0]) is a
    cell[0, 0, 0] = 5.0
    b = nb._host_cell(cell[0])
    assert b is not a and float(b[0, 0]) == 5.0
    other = torch.eye(3, device=device) * 6.0
    assert float(nb._host_cell(other)[1, 1]) == 6.0


@pytest.mark.parametrize("n", [12, 60])
def test_receiver_row_order_choice(device, n):
    """A spatial atom numbering keeps index order for the receiver passes; a shuffled one takes the Morton rows
    (chosen on the device by ictc_receiver_rows, without a host read: both are row lists)."""
    from ictc_o3.ops.tensor_product import _receiver_rows
    g = torch.Generator().manual_seed(3)
    grid = torch.stack(torch.meshgrid(*[torch.arange(n)] * 3, indexing="ij"), -1).reshape(-1, 3).float() * 3.0
    pos = grid + (torch.rand(grid.shape, generator=g) - 0.5) * 0.6
    cell = torch.floor((pos - pos.min(0).values) / 2.0).long()
    key = torch.zeros(pos.shape[0], dtype=torch.long)
    for b in range(10):
        for d in range(3):
            key |= ((cell[:, d] >> b) & 1) << (3 * b + d)
    rows = torch.sort(key, stable=True).indices.int()
    got = _receiver_rows(pos.to(device), rows.to(device)).cpu()
    assert got.dtype == rows.dtype and torch.equal(got, torch.arange(rows.numel(), dtype=rows.dtype))
    perm = torch.randperm(pos.shape[0], generator=g)
    shuffled = pos[perm]
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    srows = inv[rows.long()].int()
    assert torch.equal(_receiver_rows(shuffled.to(device), srows.to(device)).cpu(), srows)
