"""Whole-model parity on the GPU vs the float64 oracle.

Tolerances (north star): energies 1e-6 relative, forces 1e-5 relative
(max-norm), force-loss parameter gradients relative L2 < 3e-5 (the
reference's own gate, tests/test_foundation_species_precision.py:114).
"""
import pytest
import torch

import model_oracle as mo
from helpers import assert_energy_close, rel_err
from model_helpers import build_graph, fcc_cells

pytestmark = pytest.mark.gpu


def _setup(device, seed, C, lmax, edge_lmax, S, cells=1, ncell=2, cutoff=4.5):
    from mace_ictc.hp import create_model
    torch.manual_seed(seed)
    zs = (1, 6, 8, 7, 9, 14, 15, 16, 17, 35)[:S]
    model = create_model(channels=C, lmax=lmax, edge_lmax=edge_lmax, atomic_numbers=zs, cutoff=cutoff,
                         avg_num_neighbors=40.0, device=device)
    pos, Z, batch, cell = fcc_cells(ncell, 0.1, 0.3, seed, S, cells=cells, atomic_numbers=zs)
    src, dst, sh = build_graph(pos, batch, cell, cutoff)
    return model, pos, Z, batch, cell, src, dst, sh


@pytest.mark.parametrize("C,lmax,edge_lmax,S,cells", [(16, 2, 2, 3, 1), (32, 2, 3, 10, 2), (64, 2, 2, 3, 1)])
def test_energy_and_forces_match_oracle(device, C, lmax, edge_lmax, S, cells):
    from mace_ictc.hp import energy_and_forces
    model, pos, Z, batch, cell, src, dst, sh = _setup(device, 1, C, lmax, edge_lmax, S, cells)
    E0, F0, A0 = mo.energy_and_forces(model.state_dict(), mo.config_of(model), pos, Z, batch, src, dst, sh, cell,
                                      cells)
    out = energy_and_forces(model, pos.float().to(device), Z.to(device), batch.to(device), src.to(device),
                            dst.to(device), sh.float().to(device), cell.float().to(device))
    for b in range(cells):
        assert_energy_close(out["energy"][b], E0[b], A0[batch == b], f"C{C} L{edge_lmax} S{S} graph {b}")
    assert rel_err(out["forces"], F0) < 1e-5
    assert rel_err(out["atomic_energy"], A0) < 1e-5


def test_force_loss_parameter_gradients(device):
    """E+F MSE loss backward (mixed second derivatives) vs float64 autograd of the oracle."""
    from mace_ictc.hp import energy_and_forces
    model, pos, Z, batch, cell, src, dst, sh = _setup(device, 2, 16, 2, 3, 4, cells=2)
    g = torch.Generator().manual_seed(3)
    E_t = torch.randn(2, generator=g, dtype=torch.float64)
    F_t = torch.randn(pos.shape, generator=g, dtype=torch.float64) * 0.5
    # oracle
    sd = {k: v.detach().double().cpu().clone() for k, v in model.state_dict().items()}
    names = [k for k, p in model.named_parameters() if p.requires_grad]
    for k in names:
        sd[k].requires_grad_(True)
    cfg = mo.config_of(model)
    p = pos.clone().requires_grad_(True)
    atomic = mo.forward(sd, cfg, p, Z, batch, src, dst, sh, cell)
    E = torch.zeros(2, dtype=torch.float64).index_add(0, batch, atomic)
    (gpos,) = torch.autograd.grad(E.sum(), p, create_graph=True)
    loss = ((E - E_t) ** 2).mean() + ((-gpos - F_t) ** 2).mean()
    ref = torch.autograd.grad(loss, [sd[k] for k in names], allow_unused=True)
    # product
    out = energy_and_forces(model, pos.float().to(device), Z.to(device), batch.to(device), src.to(device),
                            dst.to(device), sh.float().to(device), cell.float().to(device), training=True)
    loss_g = ((out["energy"].double() - E_t.to(device)) ** 2).mean() + \
        ((out["forces"].double() - F_t.to(device)) ** 2).mean()
    params = dict(model.named_parameters())
    got = torch.autograd.grad(loss_g, [params[k] for k in names], allow_unused=True)
    for k, a, b in zip(names, got, ref):
        if b is None or float(b.norm()) == 0:
            continue
        assert a is not None, k
        rl2 = float((a.double().cpu() - b).norm() / b.norm())
        assert rl2 < 3e-5, (k, rl2)


def test_force_loss_gate_gradient_handoff(device):
    """The mixed second derivative's gate gradient, handed to the forward message's first-order adjoint and
    added in its store (ictc_msg_bwd_accumulate), gives bitwise the gradients of autograd's separate add;
    it is handed over once per message layer per backward pass."""
    from ictc_o3.ops import tensor_product as tpo
    from mace_ictc.hp import energy_and_forces
    model, pos, Z, batch, cell, src, dst, sh = _setup(device, 4, 64, 2, 3, 4, cells=2)
    g = torch.Generator().manual_seed(5)
    E_t = torch.randn(2, generator=g).to(device)
    F_t = (torch.randn(pos.shape, generator=g) * 0.5).to(device)
    params = [p for p in model.parameters() if p.requires_grad]
    args = (pos.float().to(device), Z.to(device), batch.to(device), src.to(device), dst.to(device),
            sh.float().to(device), cell.float().to(device))

    def grads():
        out = energy_and_forces(model, *args, training=True)
        loss = ((out["energy"] - E_t) ** 2).mean() + ((out["forces"] - F_t) ** 2).mean()
        return torch.autograd.grad(loss, params, allow_unused=True)

    held = []
    hold = tpo._GateLink.hold
    tpo._GateLink.hold = lambda self, dg: (held.append(self.what), hold(self, dg))[1]
    try:
        with_handoff = grads()
    finally:
        tpo._GateLink.hold = hold
    # one gate-gradient hand-off per message, one radial-MLP hand-off per interaction's hidden layers
    # (the latter changes the summation order, so its parity is tested against float64 in
    # test_gpu_radial_mlp; here only the message hand-off is switched off, which must be bitwise neutral)
    assert sum(w.startswith("message") for w in held) == len(model.interactions)
    assert sum(w.startswith("cotangent of the radial") for w in held) == len(model.interactions)
    can_hold = tpo._GateLink.can_hold
    tpo._GateLink.can_hold = lambda self: False if self.what.startswith("message") else can_hold(self)
    try:
        without = grads()
    finally:
        tpo._GateLink.can_hold = can_hold
    for a, b in zip(with_handoff, without):
        assert (a is None) == (b is None)
        if a is not None:
            assert torch.equal(a, b)


def test_fused_hidden_matches_composed_radial_mlp(device, monkeypatch):
    """Force-loss training gradients (every parameter, energies and forces) with the radial MLP's hidden layers
    on the fused second-order kernels (radial_hidden) against the composed Linear / SiLU route, 1e-5."""
    from ictc_o3.ops import tensor_product as tpo
    from mace_ictc.hp import energy_and_forces
    model, pos, Z, batch, cell, src, dst, sh = _setup(device, 6, 32, 2, 3, 4, cells=2)
    g = torch.Generator().manual_seed(7)
    E_t = torch.randn(2, generator=g).to(device)
    F_t = (torch.randn(pos.shape, generator=g) * 0.5).to(device)
    params = [p for p in model.parameters() if p.requires_grad]
    args = (pos.float().to(device), Z.to(device), batch.to(device), src.to(device), dst.to(device),
            sh.float().to(device), cell.float().to(device))

    def run(fused):
        monkeypatch.setattr(tpo, "FUSED_HIDDEN", fused)
        out = energy_and_forces(model, *args, training=True)
        loss = ((out["energy"] - E_t) ** 2).mean() + ((out["forces"] - F_t) ** 2).mean()
        grads = torch.autograd.grad(loss, params, allow_unused=True)
        return [out["energy"].detach(), out["forces"].detach()] + [gr for gr in grads]

    fused, composed = run(True), run(False)
    for a, b in zip(fused, composed):
        assert (a is None) == (b is None)
        if a is not None and b.abs().max() > 0:
            assert rel_err(a, b) < 1e-5


def test_configure_model_contract(device):
    from mace_ictc.hp import configure_model, create_model
    model = create_model(channels=8, lmax=2, device=device)
    before = {k: v for k, v in model.named_parameters()}
    info = configure_model(model, training=True)
    assert info["selected"] == "generated"
    assert info["training_gate_schedule"] == "materialized"
    assert info["training_message_linear_layout"] == "node_component"
    assert all(before[k] is v for k, v in model.named_parameters())
    assert configure_model(model, policy="reference")["selected"] == "reference"
    with pytest.raises(ValueError):
        configure_model(model, layout="bogus")
    with pytest.raises(ValueError):
        configure_model(model, training=True, gate_cache_bytes=10)


@pytest.mark.parametrize("training", [False, True])
def test_energy_and_forces_without_edges(device, training):
    """Atoms farther apart than the cutoff (runtime.py:107 keeps zero-edge graphs differentiable):
    energies from the node embedding alone, zero forces, on both the first-order and the training route."""
    from mace_ictc.hp import create_model, energy_and_forces
    torch.manual_seed(4)
    model = create_model(channels=16, lmax=2, atomic_numbers=(1, 6, 8), cutoff=4.5, device=device)
    pos = torch.tensor([[0.0, 0.0, 0.0], [10.0, 0.0, 0.0], [0.0, 10.0, 0.0]], dtype=torch.float64)
    Z = torch.tensor([1, 6, 8])
    batch = torch.zeros(3, dtype=torch.long)
    cell = (torch.eye(3, dtype=torch.float64) * 30.0)[None]
    src = dst = torch.zeros(0, dtype=torch.long)
    sh = torch.zeros(0, 3)
    E0, F0, A0 = mo.energy_and_forces(model.state_dict(), mo.config_of(model), pos, Z, batch, src, dst,
                                      sh.double(), cell, 1)
    out = energy_and_forces(model, pos.float().to(device), Z.to(device), batch.to(device), src.to(device),
                            dst.to(device), sh.to(device), cell.float().to(device), training=training)
    assert_energy_close(out["energy"][0], E0[0], A0, "no edges")
    assert float(out["forces"].abs().max()) == 0.0
    assert rel_err(out["atomic_energy"], A0) < 1e-5
