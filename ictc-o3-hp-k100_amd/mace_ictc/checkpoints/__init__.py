"""Checkpoint reconstruction (reference: mace_ictc/checkpoints/__init__.py)."""
from mace_ictc.checkpoints.adapters import AtomForcesWrapper
from mace_ictc.checkpoints.loader import LoadedPotential, get_checkpoint_e3_state_dict, load_checkpoint

__all__ = ["load_checkpoint", "LoadedPotential", "AtomForcesWrapper", "get_checkpoint_e3_state_dict"]
