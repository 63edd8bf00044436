"""Force-loss training at cfg5's shape: C128, edge L3, hidden L2, 2 interactions, correlation 3,
10 species, cutoff 5.0 A, FCC 4^3 cells of 256 atoms at 0.1 atoms/A^3 (jitter 0.3 A).

* one cell: energy, forces and the force-loss parameter gradients (mixed second
  derivatives) against float64 autograd of the oracle;
* the full 32-cell batch: every cell's energy and forces against the oracle run
  on that cell alone (sampled cells), a duplicated cell gives the same energy,
  forces and loss gradient as its twin, a cell's loss gradient taken inside the
  batch equals the one taken on the cell alone, and the whole step is bitwise
  repeatable.

Tolerances (north star): energies 1e-6 relative to |E| of the cell,
forces 1e-5 relative (max-norm), parameter gradients relative L2 < 3e-5.
"""
import pytest
import torch

import model_oracle as mo
from helpers import assert_energy_close, rel_err
from model_helpers import build_graph, fcc_cells

pytestmark = pytest.mark.gpu

ZS = (1, 6, 8, 7, 9, 14, 15, 16, 17, 35)


def _model(device, seed=55):
    from mace_ictc.hp import create_model
    torch.manual_seed(seed)
    return create_model(channels=128, lmax=2, edge_lmax=3, num_interactions=2, correlation=3, atomic_numbers=ZS,
                        cutoff=5.0, avg_num_neighbors=50.0, device=device)


def _cells(cells, seed):
    pos, Z, batch, cell = fcc_cells(4, 0.1, 0.3, seed, 10, cells=cells, atomic_numbers=ZS)
    src, dst, sh = build_graph(pos, batch, cell, 5.0)
    return pos, Z, batch, cell, src, dst, sh


def _run(model, device, system, training):
    from mace_ictc.hp import energy_and_forces
    pos, Z, batch, cell, src, dst, sh = system
    return energy_and_forces(model, pos.float().to(device), Z.to(device), batch.to(device), src.to(device),
                             dst.to(device), sh.float().to(device), cell.float().to(device), training=training)


def _loss(E, F, E_t, F_t):
    return ((E - E_t) ** 2).mean() + ((F - F_t) ** 2).mean()


def _param_grads(model, loss):
    names = [k for k, p in model.named_parameters() if p.requires_grad]
    params = dict(model.named_parameters())
    return names, torch.autograd.grad(loss, [params[k] for k in names], allow_unused=True)


def _check_cell_against_oracle(model, out, system, b, E0, F0, A0):
    pos, Z, batch, cell, src, dst, sh = system
    rows = torch.nonzero(batch == b).flatten()
    assert_energy_close(out["energy"][b], E0[0], A0, f"cfg5 cell {b}")
    assert rel_err(out["forces"][rows.to(out["forces"].device)], F0) < 1e-5, b


def _oracle_cell(model, system, b):
    pos, Z, batch, cell, src, dst, sh = system
    rows = torch.nonzero(batch == b).flatten()
    keep = torch.nonzero(batch[src] == b).flatten()
    start = int(rows[0])
    one = (pos[rows], Z[rows], torch.zeros(rows.numel(), dtype=torch.long), cell[b:b + 1],
           src[keep] - start, dst[keep] - start, sh[keep])
    sd = {k: v.detach().double().cpu() for k, v in model.state_dict().items()}
    E0, F0, A0 = mo.energy_and_forces(sd, mo.config_of(model), one[0], one[1], one[2], one[4], one[5], one[6].double(),
                                      one[3], 1)
    return one, E0, F0, A0


def test_cfg5_cell_force_loss_gradients_match_oracle(device):
    model = _model(device)
    system = _cells(1, 501)
    pos, Z, batch, cell, src, dst, sh = system
    g = torch.Generator().manual_seed(56)
    E_t = torch.randn(1, generator=g, dtype=torch.float64) * 16.0
    F_t = torch.randn(pos.shape, generator=g, dtype=torch.float64) * 0.5
    # oracle: float64 autograd through the force (mixed second derivatives)
    sd = {k: v.detach().double().cpu().clone() for k, v in model.state_dict().items()}
    names = [k for k, p in model.named_parameters() if p.requires_grad]
    for k in names:
        sd[k].requires_grad_(True)
    cfg = mo.config_of(model)
    p = pos.clone().requires_grad_(True)
    atomic = mo.forward(sd, cfg, p, Z, batch, src, dst, sh.double(), cell)
    E = atomic.sum().reshape(1)
    (gpos,) = torch.autograd.grad(E.sum(), p, create_graph=True)
    ref = torch.autograd.grad(_loss(E, -gpos, E_t, F_t), [sd[k] for k in names], allow_unused=True)
    # product
    out = _run(model, device, system, training=True)
    assert_energy_close(out["energy"][0], E.detach()[0], atomic, "cfg5 force-loss cell")
    assert rel_err(out["forces"], -gpos.detach()) < 1e-5
    got_names, got = _param_grads(model, _loss(out["energy"].double(), out["forces"].double(), E_t.to(device),
                                               F_t.to(device)))
    assert got_names == names
    checked = 0
    for k, a, b in zip(names, got, ref):
        if b is None or float(b.norm()) == 0:
            continue
        assert a is not None, k
        rl2 = float((a.double().cpu() - b).norm() / b.norm())
        assert rl2 < 3e-5, (k, rl2)
        checked += 1
    assert checked >= 20


def test_cfg5_full_batch_properties(device):
    model = _model(device)
    pos, Z, batch, cell, src, dst, sh = _cells(32, 500)
    # cell 17 is an exact copy of cell 3 (positions and species)
    r3, r17 = torch.nonzero(batch == 3).flatten(), torch.nonzero(batch == 17).flatten()
    pos[r17], Z[r17] = pos[r3], Z[r3]
    src, dst, sh = build_graph(pos, batch, cell, 5.0)
    system = (pos, Z, batch, cell, src, dst, sh)
    assert pos.shape[0] == 32 * 256
    out = _run(model, device, system, training=True)
    # sampled cells against the oracle on the cell alone
    for b in (0, 3, 31):
        _, E0, F0, A0 = _oracle_cell(model, system, b)
        _check_cell_against_oracle(model, out, system, b, E0, F0, A0)
    # the duplicated cell
    f = out["forces"]
    assert abs(float(out["energy"][3]) - float(out["energy"][17])) <= 1e-6 * abs(float(out["energy"][3])) + 1e-6
    assert rel_err(f[r17.to(device)], f[r3.to(device)].double().cpu()) < 1e-5
    # loss of one cell taken inside the batch == taken on the cell alone; and it equals its twin's
    g = torch.Generator().manual_seed(9)
    E_t = torch.randn(1, generator=g, dtype=torch.float64).item()
    F_t = (torch.randn(256, 3, generator=g, dtype=torch.float64) * 0.5).to(device)

    def cell_loss(o, rows, b):
        return _loss(o["energy"][b].double(), o["forces"][rows.to(device)].double(), E_t, F_t)

    _, g3 = _param_grads(model, cell_loss(out, r3, 3))
    out = _run(model, device, system, training=True)
    _, g17 = _param_grads(model, cell_loss(out, r17, 17))
    one, *_ = _oracle_cell(model, system, 3)
    out1 = _run(model, device, one, training=True)
    _, g1 = _param_grads(model, cell_loss(out1, torch.arange(256), 0))
    for a, b, c in zip(g3, g17, g1):
        if c is None or float(c.norm()) == 0:
            continue
        assert float((a - c).norm() / c.norm()) < 3e-5
        assert float((b - c).norm() / c.norm()) < 3e-5
    # bitwise repeatability of the whole batched force-loss step
    def full_grads():
        o = _run(model, device, system, training=True)
        loss = ((o["energy"] - 1.0) ** 2).mean() + ((o["forces"] - 0.1) ** 2).mean()
        return _param_grads(model, loss)[1], o["energy"].detach(), o["forces"].detach()
    ga, ea, fa = full_grads()
    gb, eb, fb = full_grads()
    assert torch.equal(ea, eb) and torch.equal(fa, fb)
    names = [k for k, p in model.named_parameters() if p.requires_grad]
    differ = [k for k, a, b in zip(names, ga, gb) if not ((a is None and b is None) or torch.equal(a, b))]
    assert not differ, differ
