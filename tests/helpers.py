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


# Energies are held to 1e-6 of |E| (the north star's "energies within 1e-6 relative").  Only a system whose
# atomic energies cancel so far that |E| < CANCEL_RATIO * sum |e_i| falls back to 1e-6 of sum |e_i| (fp32
# atomic energies carry ~1e-7 of their own magnitude each, which no summation order removes); the ratio is
# printed either way so a run's log shows which bound held.
CANCEL_RATIO = 1e-2


def assert_energy_close(got, ref, atomic_ref, tag="", tol=1e-6):
    """|got - ref| <= tol * |ref| for one graph's energy (atomic_ref: that graph's oracle atomic energies)."""
    got, ref = float(got), float(ref)
    scale = float(atomic_ref.detach().double().abs().sum())
    ratio = abs(ref) / scale if scale > 0 else 1.0
    err = abs(got - ref)
    print(f"[energy {tag}] |E|={abs(ref):.6g} sum|e_i|={scale:.6g} ratio={ratio:.3g} "
          f"err/|E|={err / max(abs(ref), 1e-300):.3g}", flush=True)
    bound = tol * abs(ref) if ratio >= CANCEL_RATIO else tol * scale
    assert err <= bound, (tag, got, ref, err, bound, ratio)
