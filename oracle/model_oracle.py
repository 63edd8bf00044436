"""CPU float64 oracle of the MACE-ICTC baseline energy and forces.

TEST INFRASTRUCTURE ONLY.  Restates the reference forward for the
create_model route in the reference's own layout (degree dictionaries
{l: [rows, C, 2l+1]}), reading parameters by their reference names:

  geometry          backbone.py:929-973 (vec = pos[dst] - pos[src] + shift @ cell,
                    mask r <= r_max, harmonics of vec / |vec|)
  radial basis      radial_basis.py:11-92 (bessel, polynomial cutoff p, no sqrt(K) norm)
  embedding         backbone.py:1016-1020 (h = W_emb^T[species])
  interaction       layers.py:1042-1368 (linear_up, fc MLP with SiLU*1.6791767923989418,
                    path-preserving TP, mask, scatter-sum, message_linear / avg, scalar sc)
  product           products.py:792-841 (SC, e3nn Linear: out[v] = sum_u w[u,v] x[u] / sqrt(C), + sc)
  readouts          pure_cartesian_ictd_layers.py:89-115, heads.py:12-27
  energy / forces   hp/runtime.py:86-113 (F = -dE/dpos)

Pinning: composes the pinned pieces of ictc_oracle / sc_oracle; whole-model
checks in tests are rotation invariance of E, force equivariance, finite
differences of E against F, and translation invariance.  The SC's U, the one
piece built from e3nn (absent here), is pinned block by block and path by
path in tests/test_sc_oracle.py (see sc_oracle).
"""
from __future__ import annotations

import math

import torch

import ictc_oracle as orc
import sc_oracle as so

SILU = 1.6791767923989418


def radial(r, r_max, K=8, p=5):
    n = torch.arange(1, K + 1, dtype=r.dtype)
    emb = math.sqrt(2.0 / r_max) * torch.sin(r[:, None] * n * math.pi / r_max) / r.clamp_min(1e-12)[:, None]
    u = r / r_max
    env = 1 - (p + 1) * (p + 2) / 2 * u ** p + p * (p + 2) * u ** (p + 1) - p * (p + 1) / 2 * u ** (p + 2)
    return emb * (env * (r < r_max).to(r.dtype))[:, None]


def edge_geometry(pos, src, dst, shift_vec, cutoff):
    """vec = pos[dst] - pos[src] + shift, r = |vec|, n = vec / max(r, 1e-8), mask = [r <= cutoff]
    (mace_ictc/models/pure_cartesian_ictd_layers.py:1293-1297)."""
    vec = pos[dst] - pos[src] + shift_vec
    r = vec.norm(dim=1)
    n = vec / r.clamp(min=1e-8)[:, None]
    return r, n, (r <= cutoff).to(pos.dtype)


def _silu(x):
    return torch.nn.functional.silu(x) * SILU


def forward(sd, cfg, pos, A, batch, src, dst, shifts, cell, dtype=torch.float64):
    """Per-atom energies [N] for parameters ``sd`` (state dict, reference names), computed in ``dtype``."""
    C, lmax, Le = cfg["channels"], cfg["lmax"], cfg["edge_lmax"]
    S = cfg["num_elements"]
    table = cfg["z_table"]
    species = table[A.long()]
    g = lambda k: sd[k].to(device="cpu", dtype=dtype)
    shift_vec = torch.einsum("ni,nij->nj", shifts.to(dtype), cell[batch[src]].to(dtype))
    r, n, mask = edge_geometry(pos, src, dst, shift_vec, cfg["cutoff"])
    Y = orc.direction_harmonics(n, Le)
    rad = radial(r, cfg["cutoff"], cfg.get("num_basis", 8), cfg.get("poly_p", 5))
    if cfg.get("radial_sqrt", False):      # historical sqrt(num_basis) norm (radial_basis.py:87-91)
        rad = rad * math.sqrt(cfg.get("num_basis", 8))
    N, E = pos.shape[0], src.numel()
    h = {0: g("node_embedding.weight").t()[species][:, :, None]}
    energy = torch.zeros(N, dtype=dtype)
    nint = cfg["num_interactions"]
    for i in range(nint):
        pre = f"interactions.{i}."
        li = 0 if i == 0 else lmax
        x = {l: torch.einsum("oc,ncm->nom", g(pre + f"linear_up.adapters.{l}.weight"), h[l]) for l in range(li + 1)}
        t = rad
        k = 0
        while pre + f"fc.{k}.weight" in sd:
            t = t @ g(pre + f"fc.{k}.weight").t()
            if pre + f"fc.{k + 2}.weight" in sd:
                t = _silu(t)
            k += 2
        paths = orc.natural_paths(li, Le, Le)
        P = len(paths)
        edge = orc.edge_tp_blocks({l: x[l][src] for l in x}, {l: Y[l] for l in range(Le + 1)},
                                  t.view(E, P, C), paths, lmax_out=Le)
        msg = {l: torch.zeros(N, v.shape[1], 2 * l + 1, dtype=dtype).index_add(0, dst, v * mask[:, None, None])
               for l, v in edge.items()}
        message = {l: torch.einsum("oc,ncm->nom", g(pre + f"message_linear.weights.{l}"), msg[l]) / cfg["avg"]
                   for l in range(Le + 1)}
        sc = torch.einsum("noi,ni->no", g(pre + "self_connection.weights.0")[species], h[0][:, :, 0])
        target = lmax if i < nint - 1 else 0
        ppre = f"products.{i}.symmetric_contractions.symmetric_contractions.contractions."
        W = {}
        for L in range(target + 1):
            corr = cfg["correlation"]
            W[L] = {corr: g(ppre + f"{L}.weights_max")}
            for j, nu in enumerate(range(corr - 1, 0, -1)):
                W[L][nu] = g(ppre + f"{L}.weights.{j}")
        xin = torch.cat([message[l] for l in range(Le + 1)], -1)           # [N, C, (Le+1)^2]
        flat = so.symmetric_contraction(xin, species, W, Le, target, cfg["correlation"])
        wlin = g(f"products.{i}.linear.weight")
        h, off = {}, 0
        for L in range(target + 1):
            blk = flat[:, off:off + C * (2 * L + 1)].reshape(N, C, 2 * L + 1)
            off += C * (2 * L + 1)
            w = wlin[L * C * C:(L + 1) * C * C].view(C, C)
            h[L] = torch.einsum("uv,num->nvm", w, blk) / math.sqrt(C)
        h[0] = h[0] + sc[:, :, None]
        h0 = h[0][:, :, 0]
        if i < nint - 1:
            e = h0 @ g(f"layer_energy_readouts.{i}.readout.weight").t()
        else:
            e = _silu(h0 @ g("last_layer_energy_readout.linear_1.weight").t()) @ \
                g("last_layer_energy_readout.linear_2.weight").t()
        energy = energy + e[:, 0]
    return energy


def energy_and_forces(sd, cfg, pos, A, batch, src, dst, shifts, cell, num_graphs, dtype=torch.float64):
    pos = pos.to(dtype).clone().requires_grad_(True)
    atomic = forward(sd, cfg, pos, A, batch, src, dst, shifts, cell, dtype)
    energy = torch.zeros(num_graphs, dtype=torch.float64).index_add(0, batch, atomic.double())
    (grad,) = torch.autograd.grad(energy.sum(), pos)
    return energy.detach(), -grad, atomic.detach()


def config_of(model):
    """Static config dict of a product model (read from public attributes)."""
    return {"channels": model.channels, "lmax": model.lmax, "edge_lmax": model.ictd_fix_edge_lmax,
            "num_elements": model.num_elements, "z_table": model.atomic_number_to_index.cpu(),
            "num_interactions": model.num_interaction, "cutoff": model.max_radius,
            "avg": model.avg_num_neighbors, "correlation": model.products[0].symmetric_contractions.correlation,
            "num_basis": model.number_of_basis, "poly_p": model.polynomial_cutoff_p,
            "radial_sqrt": bool(getattr(model, "radial_sqrt_num_basis", False))}
