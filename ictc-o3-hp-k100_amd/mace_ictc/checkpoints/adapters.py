"""Deployment wrapper: total energy, per-atom energies and per-atom forces of a loaded model.

Reference: AtomForcesWrapper (mace_ictc/checkpoints/adapters.py:796-892).  The
caller (a simulation engine such as LAMMPS) passes pair vectors rij [E, 3]
for edges between local and ghost atoms; a zero position leaf pos [N, 3]
makes edge_vec = pos[dst] - pos[src] + rij, so the gradient of the owned
energy lands on per-atom forces (ghost rows included, for the engine's
reverse communication).  The model takes rij as its edge shift against an
identity cell, which gives exactly that edge vector.
"""
from __future__ import annotations

import torch
import torch.nn as nn


def map_tensor_values(values: torch.Tensor, keys: torch.Tensor, table: torch.Tensor) -> torch.Tensor:
    """table[i] where keys[i] == values (0 where no key matches), elementwise."""
    match = values.to(torch.long)[:, None] == keys.to(values.device)[None, :]
    return (match.to(table.dtype) * table.to(values.device)[None, :]).sum(1)


class AtomForcesWrapper(nn.Module):
    """E_total, atom energies of the nlocal owned atoms, and forces -dE/dpos on every atom."""

    def __init__(self, model: nn.Module, atomic_energy_keys: torch.Tensor, atomic_energy_values: torch.Tensor):
        super().__init__()
        self.model = model
        self.register_buffer("atomic_energy_keys", torch.as_tensor(atomic_energy_keys, dtype=torch.long))
        self.register_buffer("atomic_energy_values", torch.as_tensor(atomic_energy_values, dtype=torch.float64))
        self.model.eval()
        for p in self.model.parameters():
            p.requires_grad = False

    def forward(self, rij: torch.Tensor, A: torch.Tensor, batch: torch.Tensor, edge_src: torch.Tensor,
                edge_dst: torch.Tensor, edge_shifts: torch.Tensor, cell: torch.Tensor, nlocal: int):
        n = A.size(0)
        with torch.enable_grad():
            pos = torch.zeros(n, 3, dtype=rij.dtype, device=rij.device, requires_grad=True)
            unit = torch.eye(3, dtype=rij.dtype, device=rij.device)[None]
            atomic = self.model(pos, A, torch.zeros_like(batch), edge_src, edge_dst, rij.detach(), unit,
                                second_order=False, forces_only=True)
            atomic = atomic.reshape(n)
            e0 = map_tensor_values(A, self.atomic_energy_keys, self.atomic_energy_values)
            owned = atomic[:nlocal].double().sum()
            total = owned + e0[:nlocal].sum()
            (grad,) = torch.autograd.grad(owned, pos)
        return total.detach(), atomic[:nlocal].detach(), -grad.detach()
