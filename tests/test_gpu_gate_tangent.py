"""Gate-tangent route of the energy-and-forces backward.

ictc_radial_gates_tangent_fwd writes the gates (those of ictc_radial_gates_fwd
within 1e-6) and d gates / dr, checked against float64 forward-mode
autograd of the radial MLP restatement (1e-5 relative, max-norm).
ictc_msg_bwd_tangent returns dfeatures / dharmonics bitwise equal to
ictc_msg_bwd's and dr = sum dgates * gtangent, checked against that sum formed
in float64 from ictc_msg_bwd's gate gradient (itself pinned to the float64
message oracle in test_gpu_message.py), 1e-5 relative.  Whole model:
forces_only=True gives the oracle's energies and forces and, when parameter
gradients are asked for anyway, the same gradients as the ordinary route.
"""
import math

import pytest
import torch

import ictc_oracle as orc
import model_oracle as mo
from helpers import rel_err
from test_gpu_message import _graph
from test_gpu_radial_mlp import _ref_gates

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _fc(out, Ws, device):
    fc = torch.nn.Sequential(torch.nn.Linear(8, 64, bias=False), torch.nn.SiLU(), torch.nn.Linear(64, 64, bias=False),
                             torch.nn.SiLU(), torch.nn.Linear(64, 64, bias=False), torch.nn.SiLU(),
                             torch.nn.Linear(64, out, bias=False)).to(device)
    with torch.no_grad():
        for m, W in zip([m for m in fc if isinstance(m, torch.nn.Linear)], Ws):
            m.weight.copy_(W.float())
    return fc


@pytest.mark.parametrize("E,out", [(1000, 704), (77, 192), (4099, 64), (33, 2176), (40001, 704), (5, 704), (300, 464),
                                   (129, 272)])
def test_radial_gates_tangent(device, E, out):
    from ictc_o3.ops.radial_mlp import radial_gates, radial_gates_tangent
    g = torch.Generator().manual_seed(E + out)
    r = torch.rand(E, generator=g, dtype=torch.float64) * 4.6 + 0.4        # some beyond the 4.5 cutoff
    sizes = [8, 64, 64, 64, out]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    fc = _fc(out, Ws, device)
    rd = r.float().to(device)
    lin = [m.weight for m in fc if isinstance(m, torch.nn.Linear)]
    gates, gdot = radial_gates_tangent(rd, lin, 4.5, 5, mo.SILU)
    # same arithmetic as ictc_radial_gates_fwd, but the compiler may contract the shared code differently
    assert rel_err(gates, radial_gates(rd, fc, 4.5, 5, mo.SILU)) < 1e-6
    ref_g, ref = torch.autograd.functional.jvp(lambda x: _ref_gates(x, Ws, 4.5, 5), r, torch.ones_like(r))
    assert rel_err(gates, ref_g) < TOL
    assert rel_err(gdot, ref) < TOL
    assert torch.count_nonzero(gdot[rd >= 4.5]) == 0


@pytest.mark.parametrize("N,E,C,li,le,lo,mask,need_x", [
    (64, 2000, 64, 2, 2, 2, True, True),     # fused source-owned pass
    (40, 500, 128, 2, 3, 3, True, True),     # two kernels, two channel groups (workspace)
    (33, 400, 64, 0, 2, 2, False, False),    # receiver-owned pass alone (layer-0 shape)
    (30, 300, 128, 0, 3, 3, True, False),
    (20, 150, 17, 1, 2, 2, True, True)])
def test_msg_bwd_tangent_matches_gate_gradient(device, N, E, C, li, le, lo, mask, need_x):
    from ictc_o3 import PackedGraphMessage
    from ictc_o3.ops import tensor_product as tpo
    op = PackedGraphMessage.create(channels=C, input_lmax=li, edge_lmax=le, output_lmax=lo, device=device)
    spec = op.edge._prepare()
    f64, sh64, g64, src, dst, m64 = _graph(N, E, C, li, le, lo, 500 + N, mask=mask)
    src, dst = src.clone(), dst.clone()
    src[::13] = N + 1          # out-of-range ids: no contribution, zero dr
    dst[5::17] = -2
    keep = ((src < N) & (dst >= 0)).to(device)
    x, sh, g = (t.float().to(device) for t in (f64, sh64, g64))
    m = None if m64 is None else m64.float().to(device)
    gen = torch.Generator().manual_seed(N)
    gdot = torch.randn(g.shape, generator=gen).to(device)
    go = torch.randn(N, op.output_width, generator=gen).to(device)
    topo = tpo.Topology(src.to(device), dst.to(device), N)
    dx0, dsh0, dg0 = tpo._msg_bwd_raw(spec, topo, x, sh, g, m, go, (need_x, True, True))
    dx1, dsh1, dr = tpo._msg_bwd_tangent_raw(spec, topo, x, sh, g, gdot, m, go, (need_x, True))
    # the same products as the ordinary adjoint; the two kernels may contract them into FMAs differently
    # (FP32 rounding: measured at most 7e-8 relative)
    assert rel_err(dsh1, dsh0) < 1e-6
    if need_x:
        assert rel_err(dx1, dx0) < 1e-6
    else:
        assert dx1 is None
    ref = (dg0.double() * gdot.double()).sum(1)
    assert rel_err(dr, ref) < TOL
    assert torch.count_nonzero(dr[~keep]) == 0
    # harmonics gradient not asked for
    _, none, dr2 = tpo._msg_bwd_tangent_raw(spec, topo, x, sh, g, gdot, m, go, (need_x, False))
    assert none is None and rel_err(dr2, ref) < TOL


def _model_case(device):
    from model_helpers import build_graph, fcc_cells
    from mace_ictc.hp import create_model
    torch.manual_seed(4)
    zs = (1, 6, 8)
    model = create_model(channels=32, lmax=2, edge_lmax=2, atomic_numbers=zs, cutoff=4.5, avg_num_neighbors=40.0,
                         device=device)
    pos, Z, batch, cell = fcc_cells(2, 0.1, 0.3, 4, 3, cells=1, atomic_numbers=zs)
    src, dst, sh = build_graph(pos, batch, cell, 4.5)
    return model, pos, Z, batch, cell, src, dst, sh


def test_forces_only_model_matches_oracle_and_ordinary_route(device):
    model, pos, Z, batch, cell, src, dst, sh = _model_case(device)
    E0, F0, A0 = mo.energy_and_forces(model.state_dict(), mo.config_of(model), pos, Z, batch, src, dst, sh, cell, 1)
    args = [t.to(device) for t in (Z, batch, src, dst)] + [sh.float().to(device), cell.float().to(device)]
    outs = {}
    params = [q for q in model.parameters() if q.requires_grad]

    def run(fo, wrt_params):
        p = pos.float().to(device).requires_grad_(True)
        atomic = model(p, args[0], args[1], args[2], args[3], args[4], args[5], second_order=False, forces_only=fo)
        E = atomic.double().sum()
        return E.detach(), torch.autograd.grad(E, [p] + (params if wrt_params else []), allow_unused=True)

    for fo in (True, False):
        E, (gp,) = run(fo, False)                 # forces only: the gate-tangent route when fo
        _, grads = run(fo, True)                  # parameter gradients asked for anyway: the ordinary route
        outs[fo] = (E, gp, grads)
    for fo in (True, False):
        E, gp, grads = outs[fo]
        assert abs(E.item() - E0.sum().item()) <= 1e-6 * A0.abs().sum().item()
        assert rel_err(-gp, F0) < TOL
        assert rel_err(grads[0], gp) < TOL
    for a, b in zip(outs[True][2], outs[False][2]):
        if b is None:
            assert a is None or torch.count_nonzero(a) == 0
        else:
            assert rel_err(a, b) < TOL
