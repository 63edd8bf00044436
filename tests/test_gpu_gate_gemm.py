"""GPU accuracy of the split-bf16 MFMA gate projection and its adjoint vs a float64 matmul.

The kernel's error bound is FP32-level: |got - ref| <= 4e-7 * (|h| . |W|^T)
elementwise (the dot product of magnitudes), checked on N(0,1) data, on data
spanning 1e-20 .. 1e20 (bf16 keeps FP32's exponent range), and on ragged
edge counts that end inside a 16-edge tile and inside a 256-edge block.
"""
import pytest
import torch

from helpers import rel_err

pytestmark = pytest.mark.gpu


def _check(device, E, M, scale_h=None, seed=0):
    from ictc_o3.ops.radial_mlp import gate_projection
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(E, 64, generator=g, dtype=torch.float64)
    W = torch.randn(M, 64, generator=g, dtype=torch.float64) / 8
    if scale_h is not None:
        h = h * torch.pow(10.0, torch.randint(-scale_h, scale_h + 1, (E, 1), generator=g).double())
    h32, W32 = h.float(), W.float()
    ref = h32.double() @ W32.double().t()
    bound = h32.double().abs() @ W32.double().abs().t()
    got = gate_projection(h32.to(device), W32.to(device)).double().cpu()
    assert got.shape == (E, M)
    assert bool(((got - ref).abs() <= 4e-7 * bound + 1e-45).all()), float(((got - ref).abs() / bound).max())


@pytest.mark.parametrize("E,M", [(1000, 704), (77, 192), (4099, 64), (16, 16), (257, 2176), (1, 48)])
def test_gate_projection_accuracy(device, E, M):
    _check(device, E, M)


def test_gate_projection_range(device):
    _check(device, 3000, 704, scale_h=20, seed=1)


def test_gate_projection_rejects(device):
    from ictc_o3.ops.radial_mlp import gate_projection
    with pytest.raises(ValueError):
        gate_projection(torch.zeros(4, 64, device=device), torch.zeros(20, 64, device=device))
    with pytest.raises(ValueError):
        gate_projection(torch.zeros(4, 32, device=device), torch.zeros(16, 32, device=device))
    assert gate_projection(torch.zeros(0, 64, device=device), torch.zeros(16, 64, device=device)).shape == (0, 16)


def _check_adjoint(device, E, M, scale=None, seed=0):
    from ictc_o3.ops.radial_mlp import gate_projection_adjoint
    g = torch.Generator().manual_seed(seed)
    dg = torch.randn(E, M, generator=g, dtype=torch.float64)
    W = torch.randn(M, 64, generator=g, dtype=torch.float64) / 8
    if scale is not None:
        dg = dg * torch.pow(10.0, torch.randint(-scale, scale + 1, (E, 1), generator=g).double())
    dg32, W32 = dg.float(), W.float()
    ref = dg32.double() @ W32.double()
    bound = dg32.double().abs() @ W32.double().abs()
    got = gate_projection_adjoint(dg32.to(device), W32.to(device)).double().cpu()
    assert got.shape == (E, 64)
    assert bool(((got - ref).abs() <= 4e-7 * bound + 1e-45).all()), float(((got - ref).abs() / bound).max())
    return got


@pytest.mark.parametrize("E,M", [(1000, 704), (77, 192), (4099, 64), (16, 768), (1, 320), (70001, 704), (90001, 512), (33, 448),
                                 (300, 2176), (50, 48)])
def test_gate_adjoint_accuracy(device, E, M):
    """Kernel for M a multiple of 64 up to 768 (ragged tiles included); library GEMM beyond."""
    _check_adjoint(device, E, M)


def test_gate_adjoint_range_and_determinism(device):
    a = _check_adjoint(device, 5000, 704, scale=20, seed=3)
    b = _check_adjoint(device, 5000, 704, scale=20, seed=3)
    assert torch.equal(a, b)


@pytest.mark.parametrize("E,M", [(5000, 2176), (777, 1600), (300, 832)])
def test_wide_gate_adjoint_column_blocks(device, E, M):
    """Projections wider than 768 gates: the split-bf16 adjoint over column blocks of at most 768, accumulated
    in column order, against float64 (1e-5) and bitwise repeatable."""
    from ictc_o3.ops.radial_mlp import gate_projection_adjoint
    g = torch.Generator().manual_seed(E + M)
    dg = torch.randn(E, M, generator=g, dtype=torch.float64)
    W = torch.randn(M, 64, generator=g, dtype=torch.float64) / 8
    out = gate_projection_adjoint(dg.float().to(device), W.float().to(device))
    assert rel_err(out, dg @ W) < 1e-5
    assert torch.equal(out, gate_projection_adjoint(dg.float().to(device), W.float().to(device)))
