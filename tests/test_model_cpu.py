"""CPU checks of the neighbour list and of the whole-model oracle's invariances."""
import itertools
import math

import numpy as np
import pytest
import torch

import model_oracle as mo
from helpers import random_rotation
from model_helpers import build_graph, fcc_cells


def _brute(pos, cell, cutoff):
    pos, cell = pos.numpy(), cell.numpy()
    out = set()
    for i, j in itertools.product(range(len(pos)), repeat=2):
        for s in itertools.product(range(-2, 3), repeat=3):
            v = pos[i] - pos[j] + np.array(s) @ cell
            r = np.linalg.norm(v)
            if 1e-10 < r < cutoff:
                out.add((j, i, s))
    return out


@pytest.mark.parametrize("ncell,cutoff", [(2, 4.5), (3, 3.0)])
def test_radius_graph_matches_brute_force(ncell, cutoff):
    from mace_ictc.hp import radius_graph_pbc
    pos, _, _, cell = fcc_cells(ncell, 0.1, 0.3, 1, 1)
    pos = pos + 3.0 * torch.randn(pos.shape, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    src, dst, sh = radius_graph_pbc(pos, cell[0], cutoff)
    got = {(int(s), int(d), tuple(int(round(float(x))) for x in v)) for s, d, v in zip(src, dst, sh)}
    assert got == _brute(pos, cell[0], cutoff)
    assert bool((dst[1:] >= dst[:-1]).all())            # receiver-sorted
    vec = pos[dst] - pos[src] + sh.double() @ cell[0]
    assert float(vec.norm(dim=1).max()) < cutoff


def _model_and_system(seed=0, C=8, lmax=2, edge_lmax=2, S=3):
    from mace_ictc.hp.model import PureCartesianICTDFix
    torch.manual_seed(seed)
    zs = (1, 6, 8, 7, 9, 14, 15, 16, 17, 35)[:S]
    model = PureCartesianICTDFix(channels=C, lmax=lmax, edge_lmax=edge_lmax, atomic_numbers=zs, cutoff=4.5,
                                 avg_num_neighbors=40.0)
    pos, Z, batch, cell = fcc_cells(2, 0.1, 0.3, seed, S, atomic_numbers=zs)
    src, dst, sh = build_graph(pos, batch, cell, 4.5)
    return model, pos, Z, batch, cell, src, dst, sh


def test_model_oracle_invariances_and_force_consistency():
    model, pos, Z, batch, cell, src, dst, sh = _model_and_system()
    sd, cfg = model.state_dict(), mo.config_of(model)
    E, F, _ = mo.energy_and_forces(sd, cfg, pos, Z, batch, src, dst, sh, cell, 1)
    # rotation: rotate positions and cell -> same energy, rotated forces
    R = torch.tensor(random_rotation(3))
    E2, F2, _ = mo.energy_and_forces(sd, cfg, pos @ R.T, Z, batch, src, dst, sh, cell @ R.T, 1)
    assert torch.allclose(E2, E, rtol=1e-10, atol=1e-10)
    assert torch.allclose(F2, F @ R.T, rtol=1e-8, atol=1e-10)
    # translation invariance
    E3, _, _ = mo.energy_and_forces(sd, cfg, pos + 1.7, Z, batch, src, dst, sh, cell, 1)
    assert torch.allclose(E3, E, rtol=1e-10, atol=1e-10)
    # forces vs central finite differences of the energy
    h = 1e-5
    for atom, axis in [(0, 0), (5, 2), (17, 1)]:
        d = torch.zeros_like(pos)
        d[atom, axis] = h
        ep, _, _ = mo.energy_and_forces(sd, cfg, pos + d, Z, batch, src, dst, sh, cell, 1)
        em, _, _ = mo.energy_and_forces(sd, cfg, pos - d, Z, batch, src, dst, sh, cell, 1)
        fd = -(ep - em) / (2 * h)
        assert abs(float(fd) - float(F[atom, axis])) < 1e-6 * max(1.0, abs(float(F[atom, axis])))
    # force sum vanishes (translation invariance of the energy)
    assert float(F.sum(0).abs().max()) < 1e-9


def test_model_parameter_names_follow_reference():
    model, *_ = _model_and_system()
    keys = set(model.state_dict())
    for k in ["node_embedding.weight", "interactions.0.linear_up.adapters.0.weight", "interactions.1.tp.weight",
              "interactions.0.fc.0.weight", "interactions.0.fc.6.weight", "interactions.1.message_linear.weights.2",
              "interactions.0.self_connection.weights.0",
              "products.0.symmetric_contractions.symmetric_contractions.contractions.2.weights_max",
              "products.1.symmetric_contractions.symmetric_contractions.contractions.0.weights.1",
              "products.0.linear.weight", "layer_energy_readouts.0.readout.weight",
              "last_layer_energy_readout.linear_1.weight", "last_layer_energy_readout.linear_2.weight"]:
        assert k in keys, k


def test_geometry_oracle_gradcheck():
    """The oracle's edge geometry is differentiable as the reference formula says (finite differences)."""
    import model_oracle as mo
    g = torch.Generator().manual_seed(0)
    pos = (torch.rand(6, 3, generator=g, dtype=torch.float64) * 3).requires_grad_(True)
    src = torch.tensor([0, 1, 2, 3, 4, 5, 0, 2])
    dst = torch.tensor([1, 2, 3, 4, 5, 0, 3, 5])
    shift = torch.randn(8, 3, generator=g, dtype=torch.float64).requires_grad_(True)
    f = lambda p, s: tuple(mo.edge_geometry(p, src, dst, s, 4.5)[:2])
    assert torch.autograd.gradcheck(f, (pos, shift))
    r, n, _ = mo.edge_geometry(pos, src, dst, shift, 4.5)
    vec = pos[dst] - pos[src] + shift
    assert torch.allclose((n * n).sum(1), torch.ones(8, dtype=torch.float64))
    assert torch.allclose((n * vec).sum(1), r)


@pytest.mark.parametrize("bad_z", [200, 2])
def test_unknown_atomic_number_raises_before_any_kernel(bad_z):
    """backbone.py:996-1009: an atomic number past the map or without a species is a ValueError (host-side check)."""
    model, pos, Z, batch, cell, src, dst, sh = _model_and_system()
    Z = Z.clone()
    Z[3] = bad_z
    with pytest.raises(ValueError, match="atomic number"):
        model(pos.float(), Z, batch, src, dst, sh, cell.float())

