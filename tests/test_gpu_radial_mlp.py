"""GPU parity of the fused radial MLP (MFMA hidden layers) vs a float64 torch restatement.

Gates and their first derivatives (d/dr, d/dW) within 1e-5 relative (max-norm).
"""
import math

import pytest
import torch

import model_oracle as mo
from helpers import rel_err

pytestmark = pytest.mark.gpu


def _ref_gates(r, Ws, cutoff, p):
    h = mo.radial(r, cutoff, 8, p)
    for k, W in enumerate(Ws):
        h = h @ W.t()
        if k < 3:
            h = torch.nn.functional.silu(h) * mo.SILU
    return h


@pytest.mark.parametrize("E,out", [(1000, 704), (77, 192), (4099, 64), (40001, 704), (17, 272), (300, 464)])
def test_fused_radial_gates(device, E, out):
    from ictc_o3.ops.radial_mlp import radial_gates
    g = torch.Generator().manual_seed(E)
    r = torch.rand(E, generator=g, dtype=torch.float64) * 4.6 + 0.4        # some beyond the 4.5 cutoff
    sizes = [8, 64, 64, 64, out]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    fc = torch.nn.Sequential(torch.nn.Linear(8, 64, bias=False), torch.nn.SiLU(), torch.nn.Linear(64, 64, bias=False),
                             torch.nn.SiLU(), torch.nn.Linear(64, 64, bias=False), torch.nn.SiLU(),
                             torch.nn.Linear(64, out, bias=False)).to(device)
    with torch.no_grad():
        for m, W in zip([m for m in fc if isinstance(m, torch.nn.Linear)], Ws):
            m.weight.copy_(W.float())
    rr = r.clone().requires_grad_(True)
    Wr = [W.clone().requires_grad_(True) for W in Ws]
    ref = _ref_gates(rr, Wr, 4.5, 5)
    rd = r.float().to(device).requires_grad_(True)
    got = radial_gates(rd, fc, 4.5, 5, mo.SILU)
    assert rel_err(got, ref) < 1e-5
    go = torch.randn(ref.shape, generator=g, dtype=torch.float64)
    torch.autograd.backward(ref, go)
    torch.autograd.backward(got, go.float().to(device))
    assert rel_err(rd.grad, rr.grad) < 1e-5
    for m, W in zip([m for m in fc if isinstance(m, torch.nn.Linear)], Wr):
        assert rel_err(m.weight.grad, W.grad) < 1e-5


@pytest.mark.parametrize("n,offset", [(4096, 0), (1001, 0), (4096, 1)])
def test_normalized_silu_derivatives(device, n, offset):
    """normalized SiLU, its first and second derivatives (16-byte vector path when n % 4 == 0 and the
    operands are aligned, scalar path otherwise) vs float64 autograd, 1e-5 relative."""
    from ictc_o3.ops.activation import normalized_silu
    g = torch.Generator().manual_seed(n + offset)
    x64 = torch.randn(n + offset, generator=g, dtype=torch.float64)[offset:] * 4
    v64 = torch.randn(n, generator=g, dtype=torch.float64)
    w64 = torch.randn(n, generator=g, dtype=torch.float64)

    def run(x, v, w, f):
        x = x.clone().requires_grad_(True)
        y = f(x)
        (d1,) = torch.autograd.grad(y, x, v, create_graph=True)
        (d2,) = torch.autograd.grad(d1, x, w)
        return y, d1, d2

    ref = run(x64, v64, w64, lambda t: torch.nn.functional.silu(t) * mo.SILU)
    xd = torch.randn(n + offset, generator=g).to(device)[offset:]
    xd.copy_(x64.float().to(device))
    got = run(xd, v64.float().to(device), w64.float().to(device), lambda t: normalized_silu(t, mo.SILU))
    for a, b in zip(got, ref):
        assert rel_err(a, b) < 1e-5


def _ref_hidden(r, Ws, cutoff, p):
    h = mo.radial(r, cutoff, 8, p)
    for W in Ws:
        h = torch.nn.functional.silu(h @ W.t()) * mo.SILU
    return h


def _hidden_case(E, seed, device):
    g = torch.Generator().manual_seed(seed)
    r = torch.rand(E, generator=g, dtype=torch.float64) * 4.6 + 0.4        # some beyond the 4.5 cutoff
    sizes = [8, 64, 64, 64]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    u = torch.randn(E, 64, generator=g, dtype=torch.float64)
    v = torch.randn(E, 64, generator=g, dtype=torch.float64)
    rho = torch.randn(E, generator=g, dtype=torch.float64)
    ref = [t.clone() for t in (r, *Ws, u, v, rho)]
    got = [t.float().to(device) for t in (r, *Ws, u, v, rho)]
    return ref, got


def _force_loss_grads(hidden, r, W1, W2, W3, u, v, rho):
    """grad of <v, h> + <rho, d<u, h>/dr> w.r.t. (r, W1, W2, W3, u): the shape of a force-loss step."""
    leaves = [t.clone().requires_grad_(True) for t in (r, W1, W2, W3, u)]
    r, W1, W2, W3, u = leaves
    h = hidden(r, W1, W2, W3)
    (dr,) = torch.autograd.grad(h, r, u, create_graph=True)
    loss = (v * h).sum() + (rho * dr).sum()
    return [h, dr, *torch.autograd.grad(loss, leaves)]


@pytest.mark.parametrize("E,link", [(0, True), (1, True), (77, True), (4099, True), (40001, True), (4099, False)])
def test_radial_hidden_second_derivatives(device, monkeypatch, E, link):
    """radial_hidden: h3, the force-pass d/dr and the gradients of a force-loss-shaped objective (the
    second-derivative kernel ictc_radial_mlp_bwd2 and the first adjoint; with link, both in one launch)
    vs float64 autograd, 1e-5 relative."""
    from ictc_o3.ops import radial_mlp
    from ictc_o3.ops.radial_mlp import radial_hidden
    monkeypatch.setattr(radial_mlp, "LINK_HIDDEN", link)
    (r, W1, W2, W3, u, v, rho), got = _hidden_case(E, 100 + E, device)
    ref = _force_loss_grads(lambda *a: _ref_hidden(a[0], a[1:], 4.5, 5), r, W1, W2, W3, u, v, rho)
    out = _force_loss_grads(lambda *a: radial_hidden(a[0], *a[1:], 4.5, 5, mo.SILU), *got)
    names = ["h3", "dr", "d/dr", "d/dW1", "d/dW2", "d/dW3", "d/du"]
    for name, a, b in zip(names, out, ref):
        assert a.shape == b.shape, name
        if b.numel() and b.abs().max() > 0:
            assert rel_err(a, b) < 1e-5, name
        else:   # no edges: empty per-edge outputs, zero weight gradients
            assert a.numel() == 0 or bool((a == 0).all()), name


def test_radial_hidden_other_orders(device):
    """Cotangents on the first adjoint's weight gradients and a third derivative take the composed torch
    route (_hidden_torch); both against float64 autograd."""
    from ictc_o3.ops.radial_mlp import radial_hidden
    (r, W1, W2, W3, u, v, rho), got = _hidden_case(300, 7, device)

    def run(hidden, r, W1, W2, W3, u, rho):
        leaves = [t.clone().requires_grad_(True) for t in (r, W1, W2, W3, u)]
        r, W1, W2, W3, u = leaves
        h = hidden(r, W1, W2, W3)
        dr, dW2 = torch.autograd.grad(h, (r, W2), u, create_graph=True)
        s = (rho * dr).sum() + (dW2 * W2).sum()
        (sr,) = torch.autograd.grad(s, r, create_graph=True)          # a third derivative follows
        (t,) = torch.autograd.grad((sr * rho).sum(), r)
        return [dr, dW2, sr, t]

    ref = run(lambda *a: _ref_hidden(a[0], a[1:], 4.5, 5), r, W1, W2, W3, u, rho)
    out = run(lambda *a: radial_hidden(a[0], *a[1:], 4.5, 5, mo.SILU), *got[:5], got[6])
    for a, b in zip(out, ref):
        assert rel_err(a, b) < 1e-5


@pytest.mark.parametrize("inputs", [(0, 1, 2, 3, 4), (0,), (2,), (4,), (1, 4)])
def test_radial_hidden_link_partial_inputs_and_retained_graph(device, monkeypatch, inputs):
    """The force-loss-shaped objective of radial_hidden differentiated for a subset of (r, W1, W2, W3, u) and
    twice over one retained graph: float64 gradients (1e-5), the two passes bitwise equal, with the
    second-derivative hand-off (LINK_HIDDEN) on and off."""
    from ictc_o3.ops import radial_mlp
    from ictc_o3.ops.radial_mlp import radial_hidden
    (r, W1, W2, W3, u, v, rho), got_in = _hidden_case(2000, 8, device)

    def objective(hidden, leaves, v, rho):
        r, W1, W2, W3, u = leaves
        h = hidden(r, W1, W2, W3)
        (dr,) = torch.autograd.grad(h, r, u, create_graph=True)
        return (v * h).sum() + (rho * dr).sum()

    ref_leaves = [t.clone().requires_grad_(True) for t in (r, W1, W2, W3, u)]
    L = objective(lambda *a: _ref_hidden(a[0], a[1:], 4.5, 5), ref_leaves, v, rho)
    ref = torch.autograd.grad(L, [ref_leaves[k] for k in inputs])
    for link in (True, False):
        monkeypatch.setattr(radial_mlp, "LINK_HIDDEN", link)
        leaves = [t.clone().requires_grad_(True) for t in got_in[:5]]
        L = objective(lambda *a: radial_hidden(a[0], *a[1:], 4.5, 5, mo.SILU), leaves, got_in[5], got_in[6])
        got = torch.autograd.grad(L, [leaves[k] for k in inputs], retain_graph=True)
        again = torch.autograd.grad(L, [leaves[k] for k in inputs])
        for g1, g2, want in zip(got, again, ref):
            assert torch.equal(g1, g2)
            assert rel_err(g1, want) < 1e-5
