"""Native LAMMPS MFF core on one MI355X (reference: mace_ictc/interfaces/lammps_hp.py:114-420).

LAMMPS' MFF pair style (lammps_user_mfftorch, MFFTorchEngine::run_forward_backward,
mff_torch_engine.cpp:1724-1870) loads a small TorchScript module and calls

    atom_energy = core.forward(pos, A, batch, edge_src, edge_dst, edge_shifts, cell, edge_vec)

with edge_vec = pos[dst] - pos[src] + shifts . cell built from a position
leaf over the local and ghost atoms, sums atom_energy[:nlocal] and
differentiates it with respect to pos (ghost forces are reverse-communicated
by LAMMPS).  The TorchScript module (NativeCore) is a dispatch envelope: it
calls the custom op ``mff_ictc_hp::energy``, implemented here in Python on
the model of ``load_checkpoint`` (mace_ictc.checkpoints), whose per-atom
energies are differentiable in edge_vec.  The model takes edge_vec as its
edge shift against an identity cell and zero positions, which reproduces
exactly those edge vectors.

One GPU: size > 1 (the reference's layerwise RCCL ghost exchange,
lammps_hp.py:24-111) is outside this build and raises ValueError.
"""
from __future__ import annotations

import json
import shutil
import uuid
from pathlib import Path

import torch

from mace_ictc.interfaces.elements import atomic_number

_RUNTIMES: dict = {}


class _Runtime:
    """A loaded checkpoint, its species table and per-species E0 (lammps_hp.py:191-211)."""

    def __init__(self, checkpoint, metadata, device):
        from mace_ictc.checkpoints import load_checkpoint
        pot = load_checkpoint(str(checkpoint), metadata["elements"], device=str(device),
                              atomic_energy_keys=metadata.get("e0_keys"), atomic_energy_values=metadata.get("e0_values"),
                              avg_num_neighbors=metadata.get("avg_num_neighbors"))
        self.model = pot.model.to(device).eval().requires_grad_(False)
        self.model.skip_input_validation = True      # validated once below, per call topology is not cached
        numbers = list(self.model.atomic_numbers)
        self.numbers = torch.tensor(numbers, dtype=torch.int64, device=device)
        keys = pot.wrapper.atomic_energy_keys.tolist()
        values = pot.wrapper.atomic_energy_values.tolist()
        e0 = dict(zip(keys, values)) if metadata.get("embed_e0", True) else {}
        self.e0 = torch.tensor([float(e0.get(z, 0.0)) for z in numbers], dtype=torch.float32, device=device)
        self.metadata = metadata
        self.sorted_checked = False
        self.calls = 0

    def energy(self, pos, atomic, batch, src, dst, shifts, cell, vectors, owned, owners, rank, size):
        from ictc_o3.ops import tensor_product as tpo
        if size != 1:
            raise ValueError("This build runs the native MFF core on one GPU (size 1); the RCCL ghost exchange "
                             "is not built")
        if not self.sorted_checked:
            if src.numel() and not bool(torch.all(dst[1:] >= dst[:-1])):
                raise ValueError("Native MFF requires destination-sorted edges")
            if atomic.numel() and not bool((atomic[:, None] == self.numbers[None, :]).any(-1).all()):
                raise ValueError("LAMMPS atom type is absent from the native MFF checkpoint")
            self.sorted_checked = True
        self.calls += 1
        n = pos.shape[0]
        species = (atomic[:, None] == self.numbers[None, :]).long().argmax(-1)
        topo = tpo.Topology(src, dst, n, positions=pos.detach().float())
        zero = torch.zeros(n, 3, dtype=torch.float32, device=pos.device)
        unit = torch.eye(3, dtype=torch.float32, device=pos.device)[None]
        atomic_e = self.model(zero, atomic, torch.zeros_like(atomic), src, dst, vectors.float(), unit,
                              topology=topo, second_order=False, forces_only=True).reshape(n)
        # an explicit zero dependency keeps a graph without edges differentiable in pos
        return atomic_e + self.e0[species] + pos.sum() * 0.0


def register_core(path: str, device: str) -> None:
    """Load the native core described by ``path`` + ".json" on ``device`` (lammps_hp.py:287-297)."""
    target = torch.device(device)
    if target.type != "cuda":
        raise ValueError("The native MFF core runs on a ROCm GPU")
    torch.cuda.set_device(target)
    metadata = json.loads(Path(path + ".json").read_text())
    key = (int(metadata["model_id"]), torch.cuda.current_device())
    if key not in _RUNTIMES:
        checkpoint = Path(path).resolve().parent / metadata["checkpoint"]
        _RUNTIMES[key] = _Runtime(checkpoint, metadata, target)


def _energy(pos, atomic, batch, src, dst, shifts, cell, vectors, model_id, owned, owners, rank, size):
    runtime = _RUNTIMES[(model_id, pos.device.index)]
    with torch.enable_grad():
        return runtime.energy(pos, atomic, batch, src, dst, shifts, cell, vectors, owned, owners, rank, size)


def _release(anchor, model_id):
    return anchor


_LIBRARY = torch.library.Library("mff_ictc_hp", "DEF")
_LIBRARY.define("energy(Tensor pos, Tensor atomic, Tensor batch, Tensor src, Tensor dst, Tensor shifts, "
                "Tensor cell, Tensor vectors, int model_id, int owned, Tensor owners, int rank, int size) -> Tensor")
_LIBRARY.impl("energy", _energy, "CompositeImplicitAutograd")
_LIBRARY.define("release(Tensor anchor, int model_id) -> Tensor")
_LIBRARY.impl("release", _release, "CompositeImplicitAutograd")


class NativeCore(torch.nn.Module):
    """TorchScript dispatch envelope the pair style loads (lammps_hp.py:321-342)."""
    __constants__ = ["model_id"]

    def __init__(self, model_id: int):
        super().__init__()
        self.model_id = model_id

    def forward(self, pos, atomic, batch, src, dst, shifts, cell, vectors):
        return torch.ops.mff_ictc_hp.energy(pos, atomic, batch, src, dst, shifts, cell, vectors, self.model_id,
                                            pos.shape[0], atomic.new_empty((0, 2)), 0, 1)

    @torch.jit.export
    def forward_distributed(self, pos, atomic, batch, src, dst, shifts, cell, vectors, owned: int,
                            owners: torch.Tensor, rank: int, size: int):
        return torch.ops.mff_ictc_hp.energy(pos, atomic, batch, src, dst, shifts, cell, vectors, self.model_id,
                                            owned, owners, rank, size)

    @torch.jit.export
    def warmup_on_real_graph(self) -> bool:
        return True

    @torch.jit.export
    def after_force(self, anchor: torch.Tensor):
        return torch.ops.mff_ictc_hp.release(anchor, self.model_id)


def export_native(*, checkpoint, elements, out_pt, inference_mode="performance", head=None, embed_e0=True,
                  e0_keys=None, e0_values=None, avg_num_neighbors=None):
    """Write the TorchScript core, a copy of the checkpoint and the metadata sidecars (lammps_hp.py:345-420).

    The reference's E0 CSV (``e0_csv``) is replaced by explicit ``e0_keys`` /
    ``e0_values`` lists; FoundationHP checkpoints and heads are not built here.
    """
    if inference_mode not in ("performance", "capacity"):
        raise ValueError("inference_mode must be performance or capacity")
    if head is not None:
        raise ValueError("--head applies to FoundationHP checkpoints, which this build does not load")
    if not torch.cuda.is_available():
        raise ValueError("Export the native MFF core on the target GPU")
    saved = torch.load(checkpoint, map_location="cpu", weights_only=True)
    if not isinstance(saved, dict) or saved.get("tensor_product_mode") != "pure-cartesian-ictd-fix":
        raise ValueError("Native MFF expects a pure-cartesian-ictd-fix checkpoint")
    arch = saved.get("model_hyperparameters", {}) or {}
    numbers = saved.get("atomic_numbers", arch.get("atomic_numbers", saved.get("atomic_energy_keys")))
    if torch.is_tensor(numbers):
        numbers = numbers.tolist()
    if numbers is None:
        raise ValueError("Native MFF requires checkpoint atomic_numbers metadata")
    if not elements or len(set(elements)) != len(elements) or any(atomic_number(s) not in numbers for s in elements):
        raise ValueError("--elements must list distinct element symbols present in the checkpoint")
    depth = int(saved.get("num_interaction", arch.get("num_interaction", 2)))
    cutoff = float(saved.get("max_radius", arch.get("max_radius", 5.0)))
    target = Path(out_pt).resolve()
    if target.suffix == ".pt2":
        raise ValueError("The native MFF core is a .pt TorchScript archive, not .pt2")
    target.parent.mkdir(parents=True, exist_ok=True)
    copied = target.with_name(target.name + ".checkpoint.pth")
    if Path(checkpoint).resolve() != copied:
        shutil.copy2(checkpoint, copied)
    metadata = dict(backend="ictc-hp", model_id=uuid.uuid4().int & ((1 << 63) - 1), checkpoint=copied.name,
                    elements=list(elements), atomic_numbers=list(numbers), message_passing_depth=depth,
                    max_radius=cutoff, tensor_product_mode="pure-cartesian-ictd-fix", dtype="float32",
                    inference_mode=inference_mode, head=None, feature_exchange="none", embed_e0=bool(embed_e0),
                    avg_num_neighbors=avg_num_neighbors)
    if e0_keys is not None:
        metadata.update(e0_keys=list(e0_keys), e0_values=list(e0_values))
    # validate reconstruction before publishing the archive
    _Runtime(copied, metadata, torch.device("cuda", torch.cuda.current_device()))
    torch.jit.save(torch.jit.script(NativeCore(metadata["model_id"])), str(target))
    Path(str(target) + ".json").write_text(json.dumps(metadata, indent=2) + "\n")
    Path(str(target) + ".meta").write_text(f"backend ictc-hp\nmessage_passing_depth {depth}\nfeature_exchange none\n")
    return metadata
