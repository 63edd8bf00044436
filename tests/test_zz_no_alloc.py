"""The no-allocation gate-tangent entry point against the workspace entry point it shares its kernels with.

ictc_radial_gates_tangent_fwd_noalloc keeps the split projection matrix in a
static device array; its gates and r tangents must be bitwise those of
ictc_radial_gates_tangent_fwd on the same inputs, on consecutive calls (the
second smaller, so stale scratch contents would show), for the grouped
(704 gates) and the small (192 gates) kernels, and sizes beyond the static
array are rejected.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(E, M, seed, device):
    g = torch.Generator().manual_seed(seed)
    r = (0.5 + 4.0 * torch.rand(E, generator=g)).to(device)
    Ws = [(torch.randn(o, i, generator=g) / math.sqrt(i)).to(device) for i, o in ((8, 64), (64, 64), (64, 64), (64, M))]
    return r, Ws


def _with_workspace(r, Ws, M):
    from ictc_o3 import _native as nat
    E = r.shape[0]
    out, tan = r.new_empty(E, M), r.new_empty(E, M)
    nbytes = int(nat.lib().ictc_radial_gates_workspace_bytes(M))
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=r.device)
    nat.call("ictc_radial_gates_tangent_fwd", nat.ptr(r), E, 8, 64, 4.5, 5, *(nat.ptr(w) for w in Ws), M,
             1.6791767923989418, nat.ptr(out), nat.ptr(tan), nat.ptr(ws), nbytes, nat.stream_of(r))
    return out, tan


def _no_alloc(r, Ws, M):
    from ictc_o3 import _native as nat
    E = r.shape[0]
    out, tan = r.new_empty(E, M), r.new_empty(E, M)
    nat.call("ictc_radial_gates_tangent_fwd_noalloc", nat.ptr(r), E, 8, 64, 4.5, 5, *(nat.ptr(w) for w in Ws), M,
             1.6791767923989418, nat.ptr(out), nat.ptr(tan), nat.stream_of(r))
    return out, tan


@pytest.mark.parametrize("M", [704, 192])
def test_no_alloc_matches_workspace_entry_on_two_calls(device, M):
    for E, seed in ((50000, 1), (3001, 2)):        # second call smaller, different weights
        r, Ws = _inputs(E, M, seed, device)
        ref = _with_workspace(r, Ws, M)
        got = _no_alloc(r, Ws, M)
        torch.cuda.synchronize()
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1]), (M, E)


def test_no_alloc_rejects_sizes_beyond_the_static_scratch(device):
    r, Ws = _inputs(16, 4096 + 16, 3, device)
    with pytest.raises(ValueError, match="static scratch"):
        _no_alloc(r, Ws, 4096 + 16)
