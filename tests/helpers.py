"""Shared test helpers: seeded inputs, rotations in the ICTC basis, error metrics."""
import math

import numpy as np
import torch

import ictc_oracle as orc


def rel_err(a, b):
    """max|a-b| / max|b| (normwise max relative error; operands float64 on CPU)."""
    a = a.detach().to("cpu", torch.float64)
    b = b.detach().to("cpu", torch.float64)
    den = b.abs().max().item()
    if den == 0:
        return a.abs().max().item()
    return (a - b).abs().max().item() / den


def random_rotation(seed):
    g = np.random.default_rng(seed)
    q, r = np.linalg.qr(g.standard_normal((3, 3)))
    q = q * np.sign(np.diag(r))
    if np.linalg.det(q) < 0:
        q[:, 0] = -q[:, 0]
    return q


def wigner_ictc(R, l, samples=64, seed=0):
    """D_l(R) in the ICTC basis from Y_l(R n) = D_l Y_l(n), least squares over sample directions."""
    g = torch.Generator().manual_seed(seed)
    n = torch.randn(samples, 3, generator=g, dtype=torch.float64)
    n = n / n.norm(dim=1, keepdim=True)
    Rt = torch.tensor(R, dtype=torch.float64)
    Y = orc.direction_harmonics(n, l)[l]
    YR = orc.direction_harmonics(n @ Rt.T, l)[l]
    D = torch.linalg.lstsq(Y, YR).solution.T
    return D


def unit_vectors(E, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(E, 3, generator=g, dtype=dtype)
    return v / v.norm(dim=1, keepdim=True)
