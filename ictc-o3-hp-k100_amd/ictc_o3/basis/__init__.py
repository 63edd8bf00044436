"""ICTC angular basis: frozen harmonic basis, coupling tables, TP coefficient module."""
