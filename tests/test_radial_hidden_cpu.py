"""CPU checks of the composed-torch route of radial_hidden (third and higher derivatives) against the
oracle's radial basis and MLP in float64."""
import math

import torch

import model_oracle as mo
from helpers import rel_err


def test_hidden_torch_matches_oracle():
    from ictc_o3.ops.radial_mlp import _hidden_torch
    g = torch.Generator().manual_seed(3)
    r = torch.rand(257, generator=g, dtype=torch.float64) * 4.6 + 0.4
    sizes = [8, 64, 64, 64]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    h = mo.radial(r, 4.5, 8, 5)
    for W in Ws:
        h = torch.nn.functional.silu(h @ W.t()) * mo.SILU
    assert rel_err(_hidden_torch(r, *Ws, 4.5, 5, mo.SILU), h) < 1e-12


def test_hidden_adjoint_torch_second_derivative():
    """_hidden_adjoint_torch (d of the first adjoint for cotangents on dr and dW2) vs nested autograd."""
    from ictc_o3.ops.radial_mlp import _hidden_adjoint_torch, _hidden_torch
    g = torch.Generator().manual_seed(4)
    E = 65
    r = torch.rand(E, generator=g, dtype=torch.float64) * 4.0 + 0.5
    sizes = [8, 64, 64, 64]
    Ws = [torch.randn(o, i, generator=g, dtype=torch.float64) / math.sqrt(i) for i, o in zip(sizes, sizes[1:])]
    u = torch.randn(E, 64, generator=g, dtype=torch.float64)
    hr = torch.randn(E, generator=g, dtype=torch.float64)
    hW2 = torch.randn(64, 64, generator=g, dtype=torch.float64)
    cfg = (4.5, 5, mo.SILU)
    got = _hidden_adjoint_torch(cfg, (r, *Ws, u), (hr, None, hW2, None), (True,) * 5)
    leaves = [t.clone().requires_grad_(True) for t in (r, *Ws, u)]
    h = _hidden_torch(*leaves[:4], *cfg)
    dr, dW2 = torch.autograd.grad(h, (leaves[0], leaves[2]), leaves[4], create_graph=True)
    want = torch.autograd.grad((hr * dr).sum() + (hW2 * dW2).sum(), leaves)
    for a, b in zip(got, want):
        assert rel_err(a, b) < 1e-12
