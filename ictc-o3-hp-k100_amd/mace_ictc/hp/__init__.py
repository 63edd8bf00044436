"""Whole-network HP API (reference: mace_ictc/hp/__init__.py:19-30)."""
from mace_ictc.hp.runtime import check_model, configure_model, create_model, energy_and_forces
from mace_ictc.hp.neighbors import radius_graph_pbc

__all__ = ["create_model", "configure_model", "energy_and_forces", "check_model", "radius_graph_pbc"]
