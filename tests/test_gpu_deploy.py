"""Deployment: checkpoint reload and the native LAMMPS MFF core on one GPU.

* A checkpoint written in the reference's layout reloads (load_checkpoint)
  into a model whose energies and forces match the float64 oracle fed the
  saved state dict (energies 1e-6 relative to |E|, forces 1e-5).
* The LAMMPS MFF call (mff_torch_engine.cpp:1724-1870) emulated on one
  domain: local atoms plus explicit ghost images within two cutoffs (the
  message-passing depth), every pair inside the cutoff as an edge,
  receiver-sorted, edge vectors built from a position leaf as the engine
  does.  The exported TorchScript core (export_native / register_core) and
  AtomForcesWrapper each give the periodic system's energy (plus E0 of the
  local atoms), its per-atom energies on the local atoms, and, once the ghost
  forces are added onto the atoms they image (LAMMPS' reverse
  communication), the periodic forces.
"""
import json

import pytest
import torch

import model_oracle as mo
from helpers import assert_energy_close, rel_err
from model_helpers import build_graph, fcc_cells

pytestmark = pytest.mark.gpu
E0 = {1: -0.5, 6: -37.8, 8: -75.0}


def _checkpoint(tmp_path, device, channels=64):
    from mace_ictc.hp import create_model
    torch.manual_seed(21)
    model = create_model(channels=channels, lmax=2, atomic_numbers=(1, 6, 8), cutoff=4.5, avg_num_neighbors=38.0,
                         device=device)
    hp = {"lmax": 2, "channel_in": channels, "num_interaction": 2, "function_type": "bessel",
          "avg_num_neighbors": 38.0, "polynomial_cutoff_p": 5, "radial_sqrt_num_basis": False,
          "ictd_fix_route": "baseline", "dtype": "float32"}
    ck = {"e3trans_state_dict": {k: v.cpu() for k, v in model.state_dict().items()}, "model_hyperparameters": hp,
          "tensor_product_mode": "pure-cartesian-ictd-fix", "max_radius": 4.5,
          "atomic_energy_keys": torch.tensor(list(E0)), "atomic_energy_values": torch.tensor(list(E0.values()),
                                                                                              dtype=torch.float64)}
    path = tmp_path / "model.pth"
    torch.save(ck, path)
    return model, path


def test_reloaded_checkpoint_matches_oracle(device, tmp_path):
    from mace_ictc.checkpoints import load_checkpoint
    from mace_ictc.hp import energy_and_forces
    model, path = _checkpoint(tmp_path, device)
    pot = load_checkpoint(str(path), ["H", "C", "O"], device=str(device))
    pos, Z, batch, cell = fcc_cells(2, 0.1, 0.3, 8, 3)
    src, dst, sh = build_graph(pos, batch, cell, 4.5)
    E0_, F0, A0 = mo.energy_and_forces(torch.load(path, weights_only=True)["e3trans_state_dict"], mo.config_of(model),
                                       pos, Z, batch, src, dst, sh, cell, 1)
    out = energy_and_forces(pot.model, pos.float().to(device), Z.to(device), batch.to(device), src.to(device),
                            dst.to(device), sh.float().to(device), cell.float().to(device))
    assert_energy_close(out["energy"][0], E0_[0], A0, "reloaded checkpoint")
    assert rel_err(out["forces"], F0) < 1e-5


def _lammps_domain(pos, Z, cell, cutoff, depth):
    """Local atoms, then ghost images within depth * cutoff of the box; all pairs inside the cutoff."""
    L = cell[0].diagonal()
    halo = depth * cutoff
    images, owners = [pos], [torch.arange(pos.shape[0])]
    rng = range(-1, 2)
    for a in rng:
        for b in rng:
            for c in rng:
                if a == b == c == 0:
                    continue
                p = pos + torch.tensor([a, b, c], dtype=pos.dtype) * L
                keep = ((p > -halo) & (p < L + halo)).all(1)
                images.append(p[keep])
                owners.append(torch.nonzero(keep).flatten())
    allp, owner = torch.cat(images), torch.cat(owners)
    d = torch.cdist(allp, allp)
    dst, src = torch.nonzero((d < cutoff) & (d > 0), as_tuple=True)    # receiver-sorted (row-major)
    return allp, Z[owner], owner, src, dst


def _engine_call(fn, allp, A, src, dst, nlocal, device):
    """What MFFTorchEngine::run_forward_backward does: position leaf, edge vectors, E_local, forces."""
    pos = allp.float().to(device).requires_grad_(True)
    vec = pos[dst.to(device)] - pos[src.to(device)]
    batch = torch.zeros(allp.shape[0], dtype=torch.long, device=device)
    e = fn(pos, A.to(device), batch, src.to(device), dst.to(device), torch.zeros_like(vec),
           torch.eye(3, device=device)[None], vec)
    e_local = e[:nlocal].sum()
    (g,) = torch.autograd.grad(e_local, pos)
    return e_local.detach(), e[:nlocal].detach(), -g


def test_native_core_and_wrapper_emulating_lammps(device, tmp_path):
    from mace_ictc.checkpoints import load_checkpoint
    from mace_ictc.hp import energy_and_forces
    from mace_ictc.interfaces import lammps_hp
    model, path = _checkpoint(tmp_path, device)
    pos, Z, batch, cell = fcc_cells(3, 0.1, 0.3, 9, 3)
    n = pos.shape[0]
    src_p, dst_p, sh_p = build_graph(pos, batch, cell, 4.5)
    ref = energy_and_forces(model, pos.float().to(device), Z.to(device), batch.to(device), src_p.to(device),
                            dst_p.to(device), sh_p.float().to(device), cell.float().to(device))
    allp, A, owner, src, dst = _lammps_domain(pos, Z, cell, 4.5, 2)
    assert allp.shape[0] > 5 * n

    def check(E, atom_e, forces):
        """E, per-atom energies of the model (no E0) and forces before the reverse communication."""
        assert_energy_close(E, ref["energy"][0], ref["atomic_energy"], "lammps domain")
        assert rel_err(atom_e, ref["atomic_energy"].double().cpu()) < 1e-5
        folded = torch.zeros(n, 3, dtype=torch.float64, device=device).index_add(
            0, owner.to(device), forces.double())
        assert rel_err(folded, ref["forces"].double().cpu()) < 1e-5

    # the exported TorchScript core, as the pair style loads it (E0 off: model energies compared in FP32)
    cores = {}
    for embed in (False, True):
        out_pt = tmp_path / f"core{int(embed)}" / "mff.pt"
        meta = lammps_hp.export_native(checkpoint=str(path), elements=["H", "C", "O"], out_pt=str(out_pt),
                                       embed_e0=embed, e0_keys=list(E0), e0_values=list(E0.values()),
                                       avg_num_neighbors=38.0)
        assert json.loads((out_pt.parent / "mff.pt.json").read_text())["model_id"] == meta["model_id"]
        lammps_hp.register_core(str(out_pt), str(device))
        cores[embed] = torch.jit.load(str(out_pt))
    plain = _engine_call(cores[False], allp, A, src, dst, n, device)
    check(*plain)
    # with E0 embedded: each local atom's energy gains its species' E0 (FP32 resolution at |E0| ~ 75)
    _, atom_e0, forces_e0 = _engine_call(cores[True], allp, A, src, dst, n, device)
    e0_atoms = torch.tensor([E0[int(z)] for z in Z], dtype=torch.float64, device=device)
    assert float((atom_e0.double() - plain[1].double() - e0_atoms).abs().max()) < 1e-4
    assert torch.equal(forces_e0, plain[2])
    # AtomForcesWrapper of the loaded potential: rij given, its own position leaf; E_total carries E0 in FP64
    pot = load_checkpoint(str(path), ["H", "C", "O"], device=str(device))
    rij = (allp[dst] - allp[src]).float().to(device)
    E, atom_e, forces = pot.wrapper(rij, A.to(device), torch.zeros(allp.shape[0], dtype=torch.long, device=device),
                                    src.to(device), dst.to(device), torch.zeros_like(rij),
                                    torch.eye(3, device=device)[None], n)
    check(float(E) - sum(E0[int(z)] for z in Z), atom_e, forces)
    core = cores[False]
    with pytest.raises((ValueError, RuntimeError), match="one GPU"):   # raised inside the op: may surface wrapped
        core.forward_distributed(allp.float().to(device), A.to(device), A.to(device) * 0, src.to(device),
                                 dst.to(device), torch.zeros(src.numel(), 3, device=device),
                                 torch.eye(3, device=device)[None], rij, n, A.new_zeros(0, 2).to(device), 0, 2)
