"""Alias of the standalone operators (reference: mace_ictc/hp/operators.py)."""
from ictc_o3.operators import *  # noqa: F401,F403
from ictc_o3.operators import _degree, _positive_integer  # noqa: F401
