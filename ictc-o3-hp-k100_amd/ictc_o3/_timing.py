"""Optional in-step launch timing: HIP events around named native launches.

Off by default (one ``is None`` test per launch).  ``enable()`` starts
collecting; each instrumented launch records an event before and after itself
on the stream it is launched on (torch's current stream, the one the C-ABI
calls receive), so a span is the device time of that launch inside a real
step, with the step's own operands and cache state.  ``collect()`` waits for
the events and returns {name: [milliseconds, ...]} and switches collection off.
"""
from __future__ import annotations

import torch

_spans = None


def enable() -> None:
    global _spans
    _spans = {}


def begin(name: str):
    if _spans is None:
        return None
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()
    return name, ev


def end(token) -> None:
    if token is None or _spans is None:
        return
    ev = torch.cuda.Event(enable_timing=True)
    ev.record()
    _spans.setdefault(token[0], []).append((token[1], ev))


def collect() -> dict:
    global _spans
    spans, _spans = _spans or {}, None
    out = {}
    for name, pairs in spans.items():
        if pairs:
            pairs[-1][1].synchronize()
        out[name] = [a.elapsed_time(b) for a, b in pairs]
    return out
