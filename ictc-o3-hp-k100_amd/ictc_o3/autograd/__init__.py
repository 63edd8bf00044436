"""Autograd helpers (reference: ictc_o3/autograd/)."""
from ictc_o3.autograd.requirements import required_gradients

__all__ = ["required_gradients"]
