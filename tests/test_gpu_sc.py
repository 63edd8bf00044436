"""GPU parity of the symmetric contraction (fwd, dx, dW, mixed second derivatives) vs the float64 oracle.

Tolerance 1e-5 relative (max-norm).  The oracle's U uses sympy CG and the
reference's bridge-Q fixture; see test_sc_oracle.py for how it is pinned.
"""
import pytest
import torch

import sc_oracle as so
from helpers import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _setup(device, lmax, lt, corr, C, N, S, seed):
    from ictc_o3 import create_symmetric_contraction
    torch.manual_seed(seed)
    mod = create_symmetric_contraction(num_elements=S, lmax=lmax, target_lmax=lt, channels=C, correlation=corr,
                                       device=device)
    g = torch.Generator().manual_seed(seed)
    x64 = torch.randn(N, C, (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    species = torch.randint(0, S, (N,), generator=g)
    return mod, x64, species


def _oracle_weights(mod, device=None):
    W = {}
    for L, c in enumerate(mod.symmetric_contractions.contractions):
        W[L] = {nu: c.weight_for(nu).detach().double().cpu() for nu in range(1, c.correlation + 1)}
    return W


def _packed(x_ncd, lmax):
    """[N, C, dim] (component index l*l+m) -> packed ir_mul [N, dim*C]."""
    return x_ncd.transpose(1, 2).reshape(x_ncd.shape[0], -1)


def _oracle_packed(x_ncd, species, W, lmax, lt, corr, C):
    out = so.symmetric_contraction(x_ncd, species, W, lmax, lt, corr)  # per L [N, C, 2L+1] flattened
    parts, off = [], 0
    for L in range(lt + 1):
        w = C * (2 * L + 1)
        parts.append(out[:, off:off + w].reshape(-1, C, 2 * L + 1).transpose(1, 2).reshape(-1, w))
        off += w
    return torch.cat(parts, -1)


CASES = [(2, 0, 3, 64, 300, 4), (2, 1, 3, 64, 257, 4), (2, 2, 3, 64, 200, 3), (2, 2, 2, 32, 100, 2),
         (2, 0, 1, 17, 50, 3), (1, 1, 3, 128, 90, 5), (3, 2, 3, 128, 64, 10), (3, 0, 3, 128, 80, 10),
         (0, 0, 3, 64, 70, 3)]


@pytest.mark.parametrize("lmax,lt,corr,C,N,S", CASES)
def test_sc_forward_and_first_derivatives(device, lmax, lt, corr, C, N, S):
    mod, x64, species = _setup(device, lmax, lt, corr, C, N, S, 3)
    W = _oracle_weights(mod)
    xr = x64.clone().requires_grad_(True)
    Wr = {L: {nu: w.clone().requires_grad_(True) for nu, w in W[L].items()} for L in W}
    ref = _oracle_packed(xr, species, Wr, lmax, lt, corr, C)
    x = _packed(x64, lmax).float().to(device).requires_grad_(True)
    out = mod.contract(x, species.to(device))
    assert rel_err(out, ref) < TOL
    go = torch.randn(ref.shape, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    torch.autograd.backward(ref, go)
    torch.autograd.backward(out, go.float().to(device))
    assert rel_err(x.grad, _packed(xr.grad, lmax)) < TOL
    for L, c in enumerate(mod.symmetric_contractions.contractions):
        for nu in range(1, corr + 1):
            assert rel_err(c.weight_for(nu).grad, Wr[L][nu].grad) < TOL, (L, nu)


@pytest.mark.parametrize("lmax,lt,corr,C,N,S", [(2, 0, 3, 64, 120, 3), (2, 2, 3, 32, 60, 2), (3, 2, 3, 128, 40, 4)])
def test_sc_mixed_second_derivatives(device, lmax, lt, corr, C, N, S):
    mod, x64, species = _setup(device, lmax, lt, corr, C, N, S, 5)
    W = _oracle_weights(mod)
    gen = torch.Generator().manual_seed(6)
    no = sum(2 * L + 1 for L in range(lt + 1))
    go64 = torch.randn(N, no * C, generator=gen, dtype=torch.float64)
    hx = torch.randn(N, C, (lmax + 1) ** 2, generator=gen, dtype=torch.float64)
    hW = {L: {nu: torch.randn(W[L][nu].shape, generator=gen, dtype=torch.float64) for nu in W[L]} for L in W}

    # oracle: s = <hx, dx> + <hW, dW>, then grads wrt (x, W, go)
    xr = x64.clone().requires_grad_(True)
    Wr = {L: {nu: w.clone().requires_grad_(True) for nu, w in W[L].items()} for L in W}
    gor = go64.clone().requires_grad_(True)
    wl = [Wr[L][nu] for L in Wr for nu in Wr[L]]
    out = _oracle_packed(xr, species, Wr, lmax, lt, corr, C)
    first = torch.autograd.grad(out, [xr] + wl, gor, create_graph=True)
    s = (first[0] * hx).sum() + sum((a * hW[L][nu]).sum() for a, (L, nu) in
                                     zip(first[1:], [(L, nu) for L in Wr for nu in Wr[L]]))
    ref = torch.autograd.grad(s, [xr, gor] + wl)

    x = _packed(x64, lmax).float().to(device).requires_grad_(True)
    params = [mod.symmetric_contractions.contractions[L].weight_for(nu) for L in Wr for nu in Wr[L]]
    gov = go64.float().to(device).requires_grad_(True)
    out = mod.contract(x, species.to(device))
    first = torch.autograd.grad(out, [x] + params, gov, create_graph=True)
    hxp = _packed(hx, lmax).float().to(device)
    s = (first[0] * hxp).sum() + sum((a * hW[L][nu].float().to(device)).sum() for a, (L, nu) in
                                      zip(first[1:], [(L, nu) for L in Wr for nu in Wr[L]]))
    got = torch.autograd.grad(s, [x, gov] + params)
    assert rel_err(got[0], _packed(ref[0], lmax)) < TOL
    assert rel_err(got[1], ref[1]) < TOL
    for a, b in zip(got[2:], ref[2:]):
        assert rel_err(a, b) < TOL


def test_sc_module_reference_layout_and_attrs(device):
    mod, x64, species = _setup(device, 2, 1, 3, 16, 40, 3, 7)
    W = _oracle_weights(mod)
    ref = so.symmetric_contraction(x64, species, W, 2, 1, 3)   # reference flat mul_ir layout
    flat = torch.cat([x64[:, :, l * l:(l + 1) ** 2].reshape(40, -1) for l in range(3)], -1)
    out = mod(flat.float().to(device), node_type_idx=species.to(device))
    assert rel_err(out, ref) < TOL
    attrs = torch.nn.functional.one_hot(species, 3).float().to(device)
    assert torch.equal(mod(flat.float().to(device), attrs), out)


def test_sc_deterministic_weight_gradients(device):
    mod, x64, species = _setup(device, 2, 2, 3, 64, 3000, 4, 8)
    x = _packed(x64, 2).float().to(device)
    go = torch.randn(3000, 9 * 64, device=device)
    res = []
    for _ in range(2):
        mod.zero_grad()
        mod.contract(x, species.to(device)).backward(go)
        res.append([p.grad.clone() for p in mod.parameters()])
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_sc_factory_validation(device):
    from ictc_o3 import configure_symmetric_contraction, create_symmetric_contraction
    with pytest.raises(ValueError, match="correlation"):
        create_symmetric_contraction(num_elements=2, lmax=2, correlation=4, device=device)
    with pytest.raises(ValueError, match="reduced"):
        create_symmetric_contraction(num_elements=2, lmax=2, use_reduced_cg=True, device=device)
    mod = create_symmetric_contraction(num_elements=2, lmax=2, target_lmax=0, channels=8, device=device)
    info = configure_symmetric_contraction(mod, policy="auto")
    assert info["selected"] == "generated" and info["reasons"] == []
    with pytest.raises(ValueError, match="policy"):
        configure_symmetric_contraction(mod, policy="bogus")
    with pytest.raises(TypeError):
        configure_symmetric_contraction(torch.nn.Linear(2, 2))
