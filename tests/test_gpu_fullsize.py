"""Parity at the BASELINE.json full sizes, through checks that do not need the oracle to run at that size.

cfg4 (131,072-atom MACE E+F): the 32^3 system is built as 4^3 periodic copies
of an 8^3 jittered cell, so every atom's environment (2 layers x 4.5 A = 9 A
< the 27.4 A small box) equals one of the 2,048 atoms of the small system,
whose energies and forces the float64 oracle computes (positions on a 2^-12 A
grid, so the FP32 inputs of the full system are exact).  Per-atom energies and
forces of the full system must match the oracle's within 1e-5 relative
(max-norm).  Also at full size: zero net force, bitwise determinism, and
invariance under atom renumbering and rigid translation.

cfg2 (156k-edge message), cfg3 (32,768-node SC) and cfg1 at E = 2^20 (edge
TP): the operators are row-local, so rows sampled from the full-size run are
compared with the oracle evaluated on exactly those rows' inputs (1e-5).
"""

import pytest
import torch

import ictc_oracle as orc
import model_oracle as mo
import sc_oracle as so
from helpers import assert_energy_close, rel_err, unit_vectors
from model_helpers import fcc_cells

pytestmark = pytest.mark.gpu


def _tiled_cfg4(device):
    from mace_ictc.hp import create_model
    torch.manual_seed(2024)
    model = create_model(channels=64, lmax=2, num_interactions=2, correlation=3, atomic_numbers=(1, 6, 8),
                         cutoff=4.5, avg_num_neighbors=42.0, device=device)
    pos8, Z8, _, cell8 = fcc_cells(8, 0.1, 0.3, 77, 3)
    # positions and box on a 2^-12 A grid: every tiled coordinate (< 128 A) is exact in FP32,
    # so the full-size run and the oracle see identical inputs
    q = 4096.0
    pos8 = torch.round(pos8 * q) / q
    cell8 = torch.round(cell8 * q) / q
    L8 = float(cell8[0, 0, 0])
    shifts = torch.stack(torch.meshgrid(*[torch.arange(4)] * 3, indexing="ij"), -1).reshape(-1, 3).double() * L8
    pos = (shifts[:, None, :] + pos8[None]).reshape(-1, 3)
    Z = Z8.repeat(64)
    cell = cell8 * 4
    return model, pos8, Z8, cell8, pos, Z, cell


def _ef(model, pos, Z, cell, device):
    from mace_ictc.hp import energy_and_forces, radius_graph_pbc
    p = pos.float().to(device)
    c = cell.float().to(device)
    src, dst, sh = radius_graph_pbc(p, c[0], 4.5)
    batch = torch.zeros(p.shape[0], dtype=torch.long, device=device)
    return energy_and_forces(model, p, Z.to(device), batch, src, dst, sh, c)


def test_cfg4_full_size_against_oracle_and_invariants(device):
    from mace_ictc.hp import radius_graph_pbc
    model, pos8, Z8, cell8, pos, Z, cell = _tiled_cfg4(device)
    assert pos.shape[0] == 131072
    out = _ef(model, pos, Z, cell, device)
    # oracle on the 2,048-atom cell (float64)
    s8, d8, h8 = radius_graph_pbc(pos8, cell8[0], 4.5)
    b8 = torch.zeros(pos8.shape[0], dtype=torch.long)
    E8, F8, A8 = mo.energy_and_forces(model.state_dict(), mo.config_of(model), pos8, Z8, b8, s8, d8, h8, cell8, 1)
    A = out["atomic_energy"].double().cpu().reshape(64, -1)
    F = out["forces"].double().cpu().reshape(64, -1, 3)
    assert rel_err(A, A8.expand(64, -1)) < 1e-5
    assert rel_err(F, F8.expand(64, -1, -1)) < 1e-5
    assert_energy_close(out["energy"][0], 64 * float(E8[0]), A8.repeat(64), "cfg4 131072 atoms")
    # net force vanishes (translation invariance of E)
    Fd = out["forces"].double()
    assert float(Fd.sum(0).abs().max()) <= 1e-6 * float(Fd.abs().sum(0).max())
    # bitwise determinism
    again = _ef(model, pos, Z, cell, device)
    assert torch.equal(again["forces"], out["forces"]) and torch.equal(again["energy"], out["energy"])
    # renumbering and rigid translation
    g = torch.Generator().manual_seed(3)
    perm = torch.randperm(pos.shape[0], generator=g)
    shifted = pos[perm] + torch.tensor([1.3, -0.7, 2.1], dtype=torch.float64)
    out2 = _ef(model, shifted, Z[perm], cell, device)
    assert_energy_close(out2["energy"][0], out["energy"][0], out["atomic_energy"], "cfg4 renumbered+shifted")
    assert rel_err(out2["forces"], out["forces"].cpu()[perm]) < 1e-5


def test_cfg2_full_size_message_rows(device):
    """cfg2 graph (4,096 atoms, ~156k edges): receiver rows sampled from the full run vs the oracle."""
    from ictc_o3 import PackedGraphMessage
    from mace_ictc.hp import radius_graph_pbc
    g = torch.Generator().manual_seed(1234)
    Lb = (4096 / 0.1) ** (1 / 3)
    pos = torch.rand(4096, 3, generator=g, dtype=torch.float64) * Lb
    cell = torch.eye(3, dtype=torch.float64) * Lb
    src, dst, sh = radius_graph_pbc(pos.float().to(device), cell.float().to(device), 4.5)
    E = src.numel()
    assert 140000 < E < 175000
    C = 64
    op = PackedGraphMessage.create(channels=C, input_lmax=2, edge_lmax=2, output_lmax=2, device=device)
    x = torch.randn(4096, 9 * C, generator=g, dtype=torch.float64)
    Y = torch.cat(orc.direction_harmonics(unit_vectors(E, 9), 2), -1)
    gates = torch.randn(E, op.tp.num_paths * C, generator=g, dtype=torch.float64)
    out = op(x.float().to(device), Y.float().to(device), gates.float().to(device), src, dst).double().cpu()
    s, d = src.cpu(), dst.cpu()
    rows = torch.tensor([0, 1, 17, 1000, 2047, 3333, 4095])
    sel = torch.isin(d, rows)
    ref = orc.message_packed(x, Y[sel], gates[sel], s[sel], d[sel], None, 2, 2, 2, C)
    assert rel_err(out[rows], ref[rows]) < 1e-5
    # linearity in the gates at full size
    g2 = torch.randn(E, op.tp.num_paths * C, generator=g)
    xd, Yd = x.float().to(device), Y.float().to(device)
    a = op(xd, Yd, gates.float().to(device), src, dst)
    b = op(xd, Yd, g2.to(device), src, dst)
    ab = op(xd, Yd, gates.float().to(device) + g2.to(device), src, dst)
    assert rel_err(ab, (a + b).double().cpu()) < 1e-5


def test_cfg3_full_size_sc_rows(device):
    from ictc_o3 import create_symmetric_contraction
    N, C, S = 32768, 64, 4
    torch.manual_seed(11)
    mod = create_symmetric_contraction(num_elements=S, lmax=2, target_lmax=1, channels=C, correlation=3,
                                       device=device)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(N, C, 9, generator=g, dtype=torch.float64)
    species = torch.randint(0, S, (N,), generator=g)
    xp = x.transpose(1, 2).reshape(N, -1)
    out = mod.contract(xp.float().to(device), species.to(device)).double().cpu()
    rows = torch.randint(0, N, (512,), generator=g)
    W = {L: {nu: c.weight_for(nu).detach().double().cpu() for nu in range(1, 4)}
         for L, c in enumerate(mod.symmetric_contractions.contractions)}
    ref = so.symmetric_contraction(x[rows], species[rows], W, 2, 1, 3)
    # oracle output is channel-major per degree; the product's is component-major
    parts, off = [], 0
    for L in range(2):
        w = C * (2 * L + 1)
        parts.append(ref[:, off:off + w].reshape(-1, C, 2 * L + 1).transpose(1, 2).reshape(-1, w))
        off += w
    assert rel_err(out[rows], torch.cat(parts, -1)) < 1e-5


def test_cfg1_edge_tp_at_2_pow_20(device):
    from ictc_o3 import EdgeTensorProduct
    C, E = 32, 1 << 20
    op = EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, output_lmax=2, channels=C, device=device)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(E, 9 * C, generator=g)
    Y = torch.cat(orc.direction_harmonics(unit_vectors(E, 6), 2), -1).float()
    gates = torch.randn(E, op.gate_width, generator=g)
    out = op(x.to(device), Y.to(device), gates.to(device)).cpu()
    rows = torch.randint(0, E, (1024,), generator=g)
    ref = orc.edge_tp_packed(x[rows].double(), Y[rows].double(), gates[rows].double(), 2, 2, 2, C)
    assert rel_err(out[rows], ref) < 1e-5


def _oracle_gates(r, Ws, cutoff):
    """Bessel x polynomial cutoff (p = 5) -> 8-64-64-64-M MLP with normalized SiLU, float64 (layers.py:826-835)."""
    t = mo.radial(r, cutoff, 8, 5)
    for i, W in enumerate(Ws):
        t = t @ W.t()
        if i < len(Ws) - 1:
            t = mo._silu(t)
    return t


def test_cfg2_full_size_backward_with_radial_gates(device):
    """cfg2 forward + backward at full size with the gates from the fused Bessel + MLP kernel.

    Per-edge gradients (harmonics, edge length through the gates) of sampled
    edges, feature gradients of sampled sender rows, and receiver rows of the
    output, each against the float64 oracle evaluated on exactly the edges those
    rows depend on; the MLP weight gradients at full size against the oracle's
    MLP adjoint fed the same gate cotangent (itself checked on the sampled edges).
    """
    from ictc_o3 import PackedGraphMessage, direction_harmonics
    from ictc_o3.ops.radial_mlp import _RadialGates
    from mace_ictc.hp import radius_graph_pbc
    g = torch.Generator().manual_seed(4321)
    Lb = (4096 / 0.1) ** (1 / 3)
    N, C, cutoff = 4096, 64, 4.5
    pos = torch.rand(N, 3, generator=g, dtype=torch.float64) * Lb
    cell = torch.eye(3, dtype=torch.float64) * Lb
    src, dst, shf = radius_graph_pbc(pos.float().to(device), cell.float().to(device), cutoff)
    s, d = src.cpu(), dst.cpu()
    E = s.numel()
    assert 140000 < E < 175000
    vec = (pos[d] - pos[s] + shf.double().cpu() @ cell).float().double()     # FP32-exact inputs
    r = vec.norm(dim=1)
    op = PackedGraphMessage.create(channels=C, input_lmax=2, edge_lmax=2, output_lmax=2, device=device)
    P = op.tp.num_paths
    widths = [8, 64, 64, 64, P * C]
    Ws = [(torch.randn(o, i, generator=g, dtype=torch.float64) / i ** 0.5).float().double()
          for i, o in zip(widths[:-1], widths[1:])]
    x = torch.randn(N, 9 * C, generator=g).double()
    go = torch.randn(N, op.output_width, generator=g).double()
    # product: harmonics of the edge directions, fused radial gates, message; all gradients
    xd = x.float().to(device).requires_grad_(True)
    nd = (vec / r[:, None]).float().to(device)
    Yd = torch.cat(direction_harmonics(nd, 2), -1).detach().requires_grad_(True)
    rd = r.float().to(device).requires_grad_(True)
    Wd = [W.float().to(device).requires_grad_(True) for W in Ws]
    gates_d = _RadialGates.apply(rd, *Wd, cutoff, 5, mo.SILU)
    gates_d.retain_grad()
    out = op(xd, Yd, gates_d, src, dst)
    out.backward(go.float().to(device))
    Y = Yd.detach().double().cpu()
    # receiver rows of the output and per-edge gradients of the edges ending there
    rows = torch.tensor([0, 5, 777, 2048, 4095])
    sel = torch.isin(d, rows)
    rs = r[sel].clone().requires_grad_(True)
    Ys = Y[sel].clone().requires_grad_(True)
    Wl = [W.clone().requires_grad_(True) for W in Ws]
    gs = _oracle_gates(rs, Wl, cutoff)
    ref = orc.message_packed(x, Ys, gs, s[sel], d[sel], None, 2, 2, 2, C)
    assert rel_err(out.detach()[rows.to(device)], ref[rows]) < 1e-5
    torch.autograd.backward(ref, go)
    idx = torch.nonzero(sel).flatten().to(device)
    assert rel_err(Yd.grad[idx], Ys.grad) < 1e-5
    assert rel_err(rd.grad[idx], rs.grad) < 1e-5
    # feature gradients of sampled sender rows: every edge leaving them
    senders = torch.tensor([1, 100, 2049, 3000, 4094])
    ssel = torch.isin(s, senders)
    xs = x.clone().requires_grad_(True)
    ref2 = orc.message_packed(xs, Y[ssel], _oracle_gates(r[ssel], Ws, cutoff), s[ssel], d[ssel], None, 2, 2, 2, C)
    torch.autograd.backward(ref2, go)
    assert rel_err(xd.grad[senders.to(device)], xs.grad[senders]) < 1e-5
    # full-size MLP weight gradients: oracle adjoint of the gates fed the product's gate cotangent
    dg = gates_d.grad.double().cpu()
    Wf = [W.clone().requires_grad_(True) for W in Ws]
    torch.autograd.backward(_oracle_gates(r, Wf, cutoff), dg)
    for a, b in zip(Wd, Wf):
        assert float((a.grad.double().cpu() - b.grad).norm() / b.grad.norm()) < 3e-5


def test_cfg3_full_size_sc_backward(device):
    """cfg3 feature gradient on sampled nodes vs the oracle; weight gradients at full size as the
    sum of the weight gradients of two disjoint halves of the nodes (row-additivity)."""
    from ictc_o3 import create_symmetric_contraction
    N, C, S = 32768, 64, 4
    torch.manual_seed(11)
    mod = create_symmetric_contraction(num_elements=S, lmax=2, target_lmax=1, channels=C, correlation=3,
                                       device=device)
    g = torch.Generator().manual_seed(13)
    x = torch.randn(N, C, 9, generator=g, dtype=torch.float64)
    species = torch.randint(0, S, (N,), generator=g)
    go = torch.randn(N, 4 * C, generator=g, dtype=torch.float64)
    xp = x.transpose(1, 2).reshape(N, -1).float().to(device).requires_grad_(True)
    sd, god = species.to(device), go.float().to(device)
    out = mod.contract(xp, sd)
    params = [p for p in mod.parameters() if p.requires_grad]
    grads = torch.autograd.grad(out, [xp, *params], god)
    dx = grads[0].double().cpu()
    rows = torch.randint(0, N, (512,), generator=g)
    W = {L: {nu: c.weight_for(nu).detach().double().cpu() for nu in range(1, 4)}
         for L, c in enumerate(mod.symmetric_contractions.contractions)}
    xr = x[rows].clone().requires_grad_(True)
    ref = so.symmetric_contraction(xr, species[rows], W, 2, 1, 3)
    # the product's output and cotangent are component-major per degree; the oracle's channel-major
    parts, off = [], 0
    for L in range(2):
        w = C * (2 * L + 1)
        parts.append(go[rows][:, off:off + w].reshape(-1, 2 * L + 1, C).transpose(1, 2).reshape(-1, w))
        off += w
    torch.autograd.backward(ref, torch.cat(parts, -1))
    dx_ref = xr.grad.transpose(1, 2).reshape(len(rows), -1)
    assert rel_err(dx[rows], dx_ref) < 1e-5
    half = torch.randperm(N, generator=g)[: N // 2].to(device)
    mask = torch.zeros(N, dtype=torch.bool, device=device)
    mask[half] = True
    ga = torch.autograd.grad(mod.contract(xp, sd), params, god * mask[:, None])
    gb = torch.autograd.grad(mod.contract(xp, sd), params, god * (~mask)[:, None])
    for full, a, b in zip(grads[1:], ga, gb):
        assert float((full - (a + b)).norm() / full.norm()) < 1e-5
