"""GPU parity of the per-edge TP (EdgeTensorProduct) against the float64 oracle.

Tolerance: operator outputs and gradients within 1e-5 relative
(max|gpu - oracle| / max|oracle|), FP32 kernels vs float64 oracle.
"""
import pytest
import torch

import ictc_oracle as orc
from helpers import rel_err, unit_vectors

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _inputs(E, C, li, le, lo, seed, dev, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    P = len(orc.natural_paths(li, le, lo))
    blocks = {l: torch.randn(E, C, 2 * l + 1, generator=g, dtype=dtype) for l in range(li + 1)}
    n = unit_vectors(E, seed + 1)
    sh = torch.cat(orc.direction_harmonics(n, le), -1)
    gates = torch.randn(E, P * C, generator=g, dtype=dtype)
    feats = orc.pack_ir_mul(blocks, li)
    return feats, sh, gates


CONFIGS = [(2, 2, 2, 32, 257), (2, 2, 2, 64, 300), (2, 3, 3, 128, 100), (0, 3, 3, 128, 77), (0, 2, 2, 64, 50),
           (3, 3, 3, 16, 40), (1, 2, 1, 200, 33), (2, 1, 2, 17, 21), (1, 1, 0, 256, 9)]


@pytest.mark.parametrize("li,le,lo,C,E", CONFIGS)
def test_edge_tp_forward_backward(device, li, le, lo, C, E):
    from ictc_o3 import EdgeTensorProduct
    op = EdgeTensorProduct.create(input_lmax=li, edge_lmax=le, output_lmax=lo, channels=C, device=device)
    f64, sh64, g64 = _inputs(E, C, li, le, lo, 100 + C, device)
    ref = orc.edge_tp_packed(f64, sh64, g64, li, le, lo, C)
    f, sh, g = (t.float().to(device).requires_grad_(True) for t in (f64, sh64, g64))
    out = op(f, sh, g)
    assert out.shape == ref.shape
    assert rel_err(out, ref) < TOL
    # backward of loss = mean(out^2) (the cfg1 loss)
    go = torch.randn(ref.shape, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    fr, shr, gr = (t.clone().requires_grad_(True) for t in (f64, sh64, g64))
    torch.autograd.backward(orc.edge_tp_packed(fr, shr, gr, li, le, lo, C), go)
    torch.autograd.backward(out, go.float().to(device))
    assert rel_err(f.grad, fr.grad) < TOL
    assert rel_err(sh.grad, shr.grad) < TOL
    assert rel_err(g.grad, gr.grad) < TOL


@pytest.mark.parametrize("li,le,lo,C,E,which,create", [
    (2, 2, 2, 32, 64, (0, 1, 2), False), (2, 3, 3, 128, 40, (0, 1, 2), False), (1, 1, 1, 64, 30, (0, 1, 2), False),
    (2, 2, 2, 32, 64, (0, 1, 2), True), (2, 3, 3, 128, 40, (0,), False), (2, 2, 2, 64, 50, (1, 2), False),
    (0, 3, 3, 17, 33, (2,), False)])
def test_edge_tp_mixed_second_derivatives(device, li, le, lo, C, E, which, create):
    """Double backward through the TP adjoint vs float64 autograd of the oracle.

    ``which``: the first-order gradients the second-order objective depends on
    (the others give absent tangents); ``create``: keep the graph of the second
    derivative (composed first-order operators) instead of the fused kernel.
    """
    from ictc_o3 import EdgeTensorProduct
    op = EdgeTensorProduct.create(input_lmax=li, edge_lmax=le, output_lmax=lo, channels=C, device=device)
    f64, sh64, g64 = _inputs(E, C, li, le, lo, 7, device)
    gen = torch.Generator().manual_seed(8)
    go64 = torch.randn(E, op.output_width, generator=gen, dtype=torch.float64)
    v = [torch.randn(t.shape, generator=gen, dtype=torch.float64) for t in (f64, sh64, g64)]

    def run(tensors, gov, fn):
        xs = [t.clone().requires_grad_(True) for t in tensors]
        gov = gov.clone().requires_grad_(True)
        out = fn(*xs)
        grads = torch.autograd.grad(out, xs, gov, create_graph=True)
        s = sum((grads[k] * v[k].to(grads[k])).sum() for k in which)
        return torch.autograd.grad(s, xs + [gov], allow_unused=True, create_graph=create)

    ref = run((f64, sh64, g64), go64, lambda a, b, c: orc.edge_tp_packed(a, b, c, li, le, lo, C))
    got = run([t.float().to(device) for t in (f64, sh64, g64)], go64.float().to(device), op)
    for name, a, b in zip(("dx", "dsh", "dg", "dgo"), got, ref):
        if b is None or not b.abs().max() > 0:
            assert a is None or torch.count_nonzero(a) == 0, name
        else:
            assert rel_err(a, b) < TOL, name


def test_edge_tp_mul_ir_layout(device):
    from ictc_o3 import EdgeTensorProduct
    C = 8
    ir = EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, channels=C, device=device)
    mi = EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, channels=C, layout="mul_ir", device=device)
    g = torch.Generator().manual_seed(9)
    blocks = {l: torch.randn(10, C, 2 * l + 1, generator=g).to(device) for l in range(3)}
    sh = torch.cat(orc.direction_harmonics(unit_vectors(10, 3), 2), -1).float().to(device)
    gates = torch.randn(10, ir.gate_width, generator=g).to(device)
    a = ir.unpack_output(ir(ir.pack_input(blocks), sh, gates))
    b = mi.unpack_output(mi(mi.pack_input(blocks), sh, gates))
    for l in a:
        assert rel_err(b[l], a[l]) < 1e-6


def test_edge_tp_empty_and_3d_gates(device):
    from ictc_o3 import EdgeTensorProduct
    op = EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, channels=32, device=device)
    f = torch.zeros(0, 32 * 9, device=device, requires_grad=True)
    out = op(f, torch.zeros(0, 9, device=device), torch.zeros(0, op.gate_width, device=device))
    assert out.shape == (0, op.output_width)
    out.sum().backward()
    assert f.grad.shape == f.shape
    f64, sh64, g64 = _inputs(5, 32, 2, 2, 2, 3, device)
    x = [t.float().to(device) for t in (f64, sh64, g64)]
    a = op(x[0], x[1], x[2])
    b = op(x[0], x[1], x[2].reshape(5, 11, 32))
    assert torch.equal(a, b)


def test_edge_tp_validation(device):
    from ictc_o3 import EdgeTensorProduct
    op = EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, channels=32, device=device)
    with pytest.raises(ValueError, match="features must have shape"):
        op(torch.zeros(3, 5, device=device), torch.zeros(3, 9, device=device), torch.zeros(3, 352, device=device))
    with pytest.raises(ValueError, match="FP32"):
        op(torch.zeros(3, 288, device=device, dtype=torch.float64), torch.zeros(3, 9, device=device),
           torch.zeros(3, 352, device=device))
    with pytest.raises(ValueError, match="ir_mul"):
        EdgeTensorProduct(op.tp, input_lmax=2, edge_lmax=2, layout="bogus")


def test_edge_tp_large_E_properties(device):
    """E = 2^20 at cfg1 shapes: linearity in the gates and agreement with a sampled oracle subset."""
    from ictc_o3 import EdgeTensorProduct
    E, C = 1 << 20, 32
    op = EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, channels=C, device=device)
    g = torch.Generator(device=device).manual_seed(1)
    f = torch.randn(E, C * 9, device=device, generator=g)
    n = torch.nn.functional.normalize(torch.randn(E, 3, device=device, generator=g), dim=1)
    from ictc_o3 import direction_harmonics
    sh = torch.cat(direction_harmonics(n, 2), -1)
    g1 = torch.randn(E, op.gate_width, device=device, generator=g)
    g2 = torch.randn(E, op.gate_width, device=device, generator=g)
    a = op(f, sh, g1) + 2 * op(f, sh, g2)
    b = op(f, sh, g1 + 2 * g2)
    assert rel_err(a, b) < 1e-5
    idx = torch.randint(0, E, (200,), generator=torch.Generator().manual_seed(2))
    ref = orc.edge_tp_packed(f[idx].double().cpu(), sh[idx].double().cpu(), g1[idx].double().cpu(), 2, 2, 2, C)
    assert rel_err(op(f, sh, g1)[idx.to(device)], ref) < 1e-5
