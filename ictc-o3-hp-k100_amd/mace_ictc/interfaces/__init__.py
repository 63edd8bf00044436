"""Simulation-engine interfaces (reference: mace_ictc/interfaces)."""
