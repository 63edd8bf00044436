"""Synthetic periodic systems for model tests (seeded)."""
import math

import torch


def fcc_cells(n_cells_per_dim, density, jitter, seed, species_count, cells=1, atomic_numbers=(1, 6, 8)):
    """`cells` independent periodic FCC boxes with n^3 unit cells each, jittered, random species."""
    g = torch.Generator().manual_seed(seed)
    a = (4.0 / density) ** (1.0 / 3.0)
    base = torch.tensor([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]], dtype=torch.float64)
    n = n_cells_per_dim
    grid = torch.stack(torch.meshgrid(*[torch.arange(n)] * 3, indexing="ij"), -1).reshape(-1, 3).double()
    unit = (grid[:, None, :] + base[None]).reshape(-1, 3) * a
    pos, Z, batch, cellv = [], [], [], []
    zs = torch.tensor(atomic_numbers)
    for b in range(cells):
        p = unit + (torch.rand(unit.shape, generator=g, dtype=torch.float64) * 2 - 1) * jitter
        pos.append(p)
        Z.append(zs[torch.randint(0, species_count, (p.shape[0],), generator=g)])
        batch.append(torch.full((p.shape[0],), b, dtype=torch.long))
        cellv.append(torch.eye(3, dtype=torch.float64) * a * n)
    return torch.cat(pos), torch.cat(Z), torch.cat(batch), torch.stack(cellv)


def build_graph(pos, batch, cell, cutoff):
    from mace_ictc.hp import radius_graph_pbc
    src_l, dst_l, sh_l = [], [], []
    for b in range(cell.shape[0]):
        idx = torch.nonzero(batch == b).flatten()
        s, d, sh = radius_graph_pbc(pos[idx], cell[b], cutoff)
        src_l.append(idx[s])
        dst_l.append(idx[d])
        sh_l.append(sh)
    return torch.cat(src_l), torch.cat(dst_l), torch.cat(sh_l)
