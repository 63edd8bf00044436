"""MI355X-native ICTC-O3 equivariant operators (drop-in for the reference's ``ictc_o3``).

Public surface follows ictc_o3/__init__.py:19-32 of the reference.  Importing
needs no GPU; calling an operator needs a ROCm device and the in-tree
``_lib/libictc_mi355x.so`` (built by ``csrc/build.py``).
"""
from ictc_o3.operators import (EdgeTensorProduct, GraphMessage, PackedGraphMessage, channel_linear,
                               configure_symmetric_contraction, create_symmetric_contraction,
                               direction_harmonics, normalized_silu)

__version__ = "0.1.0"

__all__ = [
    "EdgeTensorProduct", "GraphMessage", "PackedGraphMessage", "direction_harmonics",
    "create_symmetric_contraction", "configure_symmetric_contraction",
    "channel_linear", "normalized_silu",
]
