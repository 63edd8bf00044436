"""GPU parity of the direction-harmonic kernels (forward, J^T, J, Hessian-vector) vs the float64 oracle."""
import pytest
import torch

import ictc_oracle as orc
from helpers import rel_err, unit_vectors

pytestmark = pytest.mark.gpu
TOL = 1e-5


@pytest.mark.parametrize("lmax", [0, 1, 2, 3])
def test_harmonics_forward_and_derivatives(device, lmax):
    from ictc_o3 import direction_harmonics
    from ictc_o3.ops.harmonics import harmonics_packed
    E = 1000
    g = torch.Generator().manual_seed(lmax)
    n64 = torch.randn(E, 3, generator=g, dtype=torch.float64)   # unnormalised, as callers may pass
    ref = torch.cat(orc.direction_harmonics(n64, lmax), -1)
    n = n64.float().to(device)
    out = direction_harmonics(n, lmax)
    assert [o.shape[1] for o in out] == [2 * l + 1 for l in range(lmax + 1)]
    assert rel_err(torch.cat(out, -1), ref) < TOL
    if lmax == 0:
        return
    gY = torch.randn(E, (lmax + 1) ** 2, generator=g, dtype=torch.float64)
    h = torch.randn(E, 3, generator=g, dtype=torch.float64)
    # first and mixed second derivatives through float64 autograd of the oracle
    nr = n64.clone().requires_grad_(True)
    gr = gY.clone().requires_grad_(True)
    (dn_ref,) = torch.autograd.grad(torch.cat(orc.direction_harmonics(nr, lmax), -1), nr, gr, create_graph=True)
    d2n_ref, d2g_ref = torch.autograd.grad(dn_ref, (nr, gr), h)
    nn = n.clone().requires_grad_(True)
    gg = gY.float().to(device).requires_grad_(True)
    (dn,) = torch.autograd.grad(harmonics_packed(nn, lmax), nn, gg, create_graph=True)
    assert rel_err(dn, dn_ref) < TOL
    d2n, d2g = torch.autograd.grad(dn, (nn, gg), h.float().to(device))
    assert rel_err(d2n, d2n_ref) < TOL
    assert rel_err(d2g, d2g_ref) < TOL
