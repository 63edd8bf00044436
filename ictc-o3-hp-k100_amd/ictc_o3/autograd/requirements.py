"""Which input gradients does the running backward pass actually consume?

``ctx.needs_input_grad`` only says an input required grad when the forward
ran.  A ``torch.autograd.grad(E, pos)`` call for forces never consumes the
parameter gradients, so adjoints that would produce them (weight-gradient
GEMMs over millions of edges) can be skipped.  Same semantics as the
reference's ``required_gradients`` (ictc_o3/autograd/adjoint_requirements.py:13-27):
ask the engine whether each input's gradient edge will execute, and keep the
declared flag whenever the engine cannot be asked (tracing / functorch).
"""
from __future__ import annotations

import torch


def required_gradients(inputs, declared):
    """Tuple of bools: declared[i] and the engine will run input i's gradient node."""
    from torch.fx.experimental.proxy_tensor import get_proxy_mode
    if (torch.compiler.is_compiling() or get_proxy_mode() is not None
            or torch._C._are_functorch_transforms_active()
            or not hasattr(torch._C, "_will_engine_execute_node")):
        return tuple(bool(d) for d in declared)
    out = []
    for t, d in zip(inputs, declared):
        if not d or t is None:
            out.append(False)
            continue
        try:
            node = torch.autograd.graph.get_gradient_edge(t).node
            out.append(bool(torch._C._will_engine_execute_node(node)))
        except (RuntimeError, AttributeError, AssertionError):
            out.append(True)
    return tuple(out)
