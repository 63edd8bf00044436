"""Public O(3) operators, drop-in for the reference's ``ictc_o3.operators``.

Same names, signatures, validation and error types as
ictc_o3/operators.py of the reference (cited per entry point); the compute
runs on the gfx950 HIP kernels of libictc_mi355x.so.  Nothing here has a CPU
compute path: operators called with non-ROCm tensors raise ``ValueError``.
"""
from __future__ import annotations

import torch

from ictc_o3.basis import tables
from ictc_o3.basis.ictd_irreps import EdgeWeightedPathPreservingTensorProduct
from ictc_o3.ops import tensor_product as tpo
from ictc_o3.ops.harmonics import harmonics_packed

__all__ = [
    "EdgeTensorProduct", "GraphMessage", "PackedGraphMessage", "direction_harmonics",
    "create_symmetric_contraction", "configure_symmetric_contraction",
    "channel_linear", "normalized_silu",
]


def _degree(value, name):
    """operators.py:14-16"""
    if not isinstance(value, int) or isinstance(value, bool) or value < 0:
        raise ValueError(f"{name} must be a nonnegative integer")


def _positive_integer(value, name):
    """operators.py:19-21"""
    if not isinstance(value, int) or isinstance(value, bool) or value < 1:
        raise ValueError(f"{name} must be a positive integer")


def _eager(sample):
    """operators.py:24-32: eager FP32 only, TF32 off."""
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    from torch._subclasses.fake_tensor import is_fake
    from torch.fx.experimental.proxy_tensor import get_proxy_mode
    if (torch.compiler.is_compiling() or get_proxy_mode() is not None or is_fake(sample)
            or torch._C._are_functorch_transforms_active()
            or torch.is_autocast_enabled(sample.device.type)):
        raise ValueError("Standalone generated TP requires eager execution without autocast; "
                         "use whole-model prepared export for AOTI")


def _tp_coverage(tp, input_lmax, edge_lmax):
    """operators.py:35-47, plus the MI355X compiled coverage (degrees <= 3, natural paths)."""
    _degree(input_lmax, "input_lmax")
    _degree(edge_lmax, "edge_lmax")
    if not isinstance(tp, EdgeWeightedPathPreservingTensorProduct):
        raise TypeError("Expected an ICTC EdgeWeightedPathPreservingTensorProduct")
    if (tp.channels < 1 or tp.lmax < 0 or not tp.weight.is_cuda
            or tp.weight.dtype != torch.float32 or tp.internal_compute_dtype != torch.float32):
        raise ValueError("Generated TP requires CUDA FP32, internal FP32 and positive channels")
    if tp.weight.requires_grad:
        raise ValueError("TP base coefficients must already be fixed; HP does not freeze learned weights")
    if not tp.paths or any(l1 > input_lmax or l2 > edge_lmax for l1, l2, _ in tp.paths):
        raise ValueError("TP paths must be nonempty and fit the declared input/edge degrees")
    lo = max(p[2] for p in tp.paths)
    if max(input_lmax, edge_lmax, lo) > 3 or tp.channels > 256:
        raise ValueError("MI355X kernels cover degrees <= 3 and channels <= 256")
    if [tuple(p) for p in tp.paths] != tables.natural_paths(input_lmax, edge_lmax, lo):
        raise ValueError("MI355X kernels cover the natural-parity path set of the declared degrees")


def _operand(value, shape, sample, name):
    """operators.py:50-54"""
    if not isinstance(value, torch.Tensor) or tuple(value.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}")
    if value.device != sample.device or value.dtype != torch.float32:
        raise ValueError(f"{name} must be FP32 on {sample.device}")


def _spec_for(tp, input_lmax, edge_lmax):
    lo = max(p[2] for p in tp.paths)
    unit = bool(torch.all(tp.weight == 1).item())
    return tpo.make_spec(input_lmax, edge_lmax, lo, tp.channels,
                         None if unit else tp.weight.detach().contiguous())


class EdgeTensorProduct(torch.nn.Module):
    """Edge-wise TP with fixed base coefficients and live external gates (operators.py:161-340).

    ir_mul uses [magnetic, channel] within each degree/path; mul_ir uses
    [channel, magnetic].  Output paths stay separate.  First, mixed and higher
    derivatives run on the HIP kernels.  ``execution`` is accepted for API
    compatibility ('direct' / 'legacy' select the same MI355X schedule).
    """

    def __init__(self, tp, *, input_lmax, edge_lmax, layout="ir_mul", execution="direct"):
        super().__init__()
        _tp_coverage(tp, input_lmax, edge_lmax)
        if layout not in ("ir_mul", "mul_ir"):
            raise ValueError("Edge layout must be 'ir_mul' or 'mul_ir'")
        if execution not in ("direct", "legacy"):
            raise ValueError("Edge execution must be 'direct' or 'legacy'")
        self.tp = tp
        self.input_lmax, self.edge_lmax, self.layout, self.execution = input_lmax, edge_lmax, layout, execution
        self._spec, self._weight_version = None, None

    @classmethod
    def create(cls, *, input_lmax, edge_lmax, output_lmax=None, channels=64, layout="ir_mul",
               execution="direct", device="cuda"):
        """Fresh natural-parity FP32 TP with unit fixed coefficients (operators.py:190-215)."""
        _degree(input_lmax, "input_lmax")
        _positive_integer(channels, "channels")
        _degree(edge_lmax, "edge_lmax")
        output_lmax = input_lmax if output_lmax is None else output_lmax
        _degree(output_lmax, "output_lmax")
        if torch.device(device).type != "cuda":
            raise ValueError("Generated edge TP requires a CUDA device")
        paths = tables.natural_paths(input_lmax, edge_lmax, output_lmax)
        tp = EdgeWeightedPathPreservingTensorProduct(
            channels=channels, lmax=max(input_lmax, edge_lmax, output_lmax), allowed_paths=paths,
            path_policy="full", internal_compute_dtype=torch.float32).to(device=device, dtype=torch.float32)
        with torch.no_grad():
            tp.weight.fill_(1.)
        tp.weight.requires_grad_(False)
        return cls(tp, input_lmax=input_lmax, edge_lmax=edge_lmax, layout=layout, execution=execution)

    @property
    def paths(self):
        """Immutable external-gate order: (input_l, edge_l, output_l)."""
        return tuple(tuple(path) for path in self.tp.paths)

    @property
    def gate_width(self):
        return self.tp.num_paths * self.tp.channels

    @property
    def output_width(self):
        return sum(self.tp.channels * count * (2 * l + 1) for l, count in self.tp.path_counts_by_l.items())

    def _prepare(self):
        """Kernel spec; the unit-weight test syncs once per weight version (operators.py:264-271)."""
        _tp_coverage(self.tp, self.input_lmax, self.edge_lmax)
        version = self.tp.weight._version
        if self._spec is None or self._weight_version != version:
            self._spec = _spec_for(self.tp, self.input_lmax, self.edge_lmax)
            self._weight_version = version
        return self._spec

    def pack_input(self, blocks):
        """Pack {l: [E,C,2l+1]} using this operator's layout (operators.py:283-294)."""
        if set(blocks) != set(range(self.input_lmax + 1)):
            raise ValueError("Input blocks must cover every declared degree")
        rows, parts = blocks[0].shape[0], []
        for l in range(self.input_lmax + 1):
            block = blocks[l]
            _operand(block, (rows, self.tp.channels, 2 * l + 1), self.tp.weight, f"blocks[{l}]")
            if self.layout == "ir_mul":
                block = block.transpose(1, 2)
            parts.append(block.reshape(rows, self.tp.channels * (2 * l + 1)))
        return torch.cat(parts, -1).contiguous()

    def unpack_output(self, output):
        """Return {l: [E,C*path_count_l,2l+1]} in the ICTC convention (operators.py:296-308)."""
        rows = output.shape[0]
        _operand(output, (rows, self.output_width), self.tp.weight, "output")
        result, offset = {}, 0
        for l in range(self.tp.lmax + 1):
            count, width = self.tp.path_counts_by_l.get(l, 0), 2 * l + 1
            value = output[:, offset:offset + count * self.tp.channels * width]
            if self.layout == "ir_mul":
                value = value.reshape(rows, count, width, self.tp.channels).transpose(2, 3)
            result[l] = value.reshape(rows, count * self.tp.channels, width)
            offset += count * self.tp.channels * width
        return result

    def _features_to_ir_mul(self, features):
        C, parts, off = self.tp.channels, [], 0
        for l in range(self.input_lmax + 1):
            w = C * (2 * l + 1)
            parts.append(features[:, off:off + w].reshape(-1, C, 2 * l + 1).transpose(1, 2).reshape(-1, w))
            off += w
        return torch.cat(parts, -1)

    def _output_to_mul_ir(self, output):
        C, parts, off = self.tp.channels, [], 0
        for l in range(self.tp.lmax + 1):
            count, width = self.tp.path_counts_by_l.get(l, 0), 2 * l + 1
            w = count * C * width
            if w:
                parts.append(output[:, off:off + w].reshape(-1, count, width, C).transpose(2, 3).reshape(-1, w))
            off += w
        return torch.cat(parts, -1)

    def forward(self, features, harmonics, gates):
        """features [E,C*(L_in+1)^2], harmonics [E,(L_edge+1)^2], gates [E,P*C] or [E,P,C] (operators.py:310-340)."""
        _tp_coverage(self.tp, self.input_lmax, self.edge_lmax)
        _eager(features)
        if features.ndim != 2:
            raise ValueError("features must be a flat two-dimensional row buffer")
        rows = features.shape[0]
        _operand(features, (rows, self.tp.channels * (self.input_lmax + 1) ** 2), self.tp.weight, "features")
        _operand(harmonics, (rows, (self.edge_lmax + 1) ** 2), self.tp.weight, "harmonics")
        _operand(gates, (rows, self.gate_width) if gates.ndim == 2 else (rows, self.tp.num_paths, self.tp.channels),
                 self.tp.weight, "gates")
        if rows == 0:
            empty = features[:, :1] * harmonics[:, :1] * gates.reshape(0, self.gate_width)[:, :1]
            return empty.expand(0, self.output_width)
        spec = self._prepare()
        if self.layout == "mul_ir":
            features = self._features_to_ir_mul(features)
        out = tpo.edge_tp(features, harmonics, gates.reshape(rows, self.gate_width), spec)
        if self.layout == "mul_ir":
            out = self._output_to_mul_ir(out)
        return out


def _index_vector(value, e, device, name, message):
    if (not isinstance(value, torch.Tensor) or value.ndim != 1 or value.numel() != e
            or value.device != device or value.dtype != torch.int64):
        raise ValueError(message.format(name=name))


class PackedGraphMessage(torch.nn.Module):
    """Packed gather/TP/scatter (operators.py:343-409).

    Input/output layout matches EdgeTensorProduct(layout='ir_mul').  The
    reduction is always the deterministic receiver-sorted CSR (the reference's
    'atomic' and 'csr' choices both map onto it); chunking options are accepted
    and validated for compatibility, the MI355X kernels stream all edges in one
    launch.
    """

    def __init__(self, tp, *, input_lmax, edge_lmax, cartesian_schedule='native', reduction='atomic',
                 edge_chunk_size=65536, topology_backend='native', csr_accumulator_limit=None,
                 csr_slice_search=False, geometry_schedule='auto'):
        super().__init__()
        if cartesian_schedule != 'native':
            raise ValueError('Only the original ICTC basis is supported; the experimental STF-coordinate schedule is retired')
        if reduction not in ('atomic', 'csr'):
            raise ValueError('Packed graph reduction must be atomic or csr')
        if topology_backend not in ('native', 'device'):
            raise ValueError('Topology backend must be native or device')
        if csr_accumulator_limit is not None and (not isinstance(csr_accumulator_limit, int)
                                                  or isinstance(csr_accumulator_limit, bool)
                                                  or csr_accumulator_limit < 1):
            raise ValueError('CSR accumulator limit must be a positive integer or None')
        if not isinstance(csr_slice_search, bool):
            raise ValueError('csr_slice_search must be a bool')
        if geometry_schedule not in ('auto', 'native', 'streamed'):
            raise ValueError('geometry_schedule must be auto, native or streamed')
        if not isinstance(edge_chunk_size, int) or isinstance(edge_chunk_size, bool) or edge_chunk_size < 1:
            raise ValueError('edge_chunk_size must be a positive integer')
        self.edge = EdgeTensorProduct(tp, input_lmax=input_lmax, edge_lmax=edge_lmax)
        self.cartesian_schedule, self.reduction, self.edge_chunk_size = cartesian_schedule, reduction, edge_chunk_size

    @classmethod
    def create(cls, *, channels=64, input_lmax=3, edge_lmax=3, output_lmax=None, device='cuda', **kwargs):
        edge = EdgeTensorProduct.create(channels=channels, input_lmax=input_lmax, edge_lmax=edge_lmax,
                                        output_lmax=output_lmax, device=device)
        return cls(edge.tp, input_lmax=input_lmax, edge_lmax=edge_lmax, **kwargs)

    @property
    def tp(self):
        return self.edge.tp

    @property
    def output_width(self):
        return self.edge.output_width

    @property
    def gate_width(self):
        return self.edge.gate_width

    def forward(self, features, harmonics, gates, src, dst, mask=None, topology=None):
        _eager(features)
        _tp_coverage(self.tp, self.edge.input_lmax, self.edge.edge_lmax)
        if features.ndim != 2:
            raise ValueError('Expected a flat two-dimensional packed node buffer')
        n, e = features.shape[0], src.numel()
        _operand(features, (n, self.tp.channels * (self.edge.input_lmax + 1) ** 2), self.tp.weight, 'features')
        _operand(harmonics, (e, (self.edge.edge_lmax + 1) ** 2), self.tp.weight, 'harmonics')
        _operand(gates, (e, self.gate_width) if gates.ndim == 2 else (e, self.tp.num_paths, self.tp.channels),
                 self.tp.weight, 'gates')
        for name, value in (('src', src), ('dst', dst)):
            _index_vector(value, e, features.device, name, '{name} must be an int64 CUDA vector of valid node indices')
        if mask is not None:
            if mask.requires_grad or tuple(mask.shape) not in ((e,), (e, 1)):
                raise ValueError('Mask must be fixed [E] or [E,1]')
            _operand(mask, mask.shape, self.tp.weight, 'mask')
            mask = mask.reshape(e).contiguous()
        spec = self.edge._prepare()
        topo = topology if topology is not None else tpo.Topology(src, dst, n)
        return tpo.message(features, harmonics.contiguous(), gates.reshape(e, self.gate_width), spec, topo, mask)


class GraphMessage(torch.nn.Module):
    """Gather/TP/gate/scatter on degree dictionaries (operators.py:412-468)."""

    def __init__(self, tp, *, input_lmax, edge_lmax, layout="packed", edge_chunk_size=65536,
                 reduction="auto", cartesian_schedule="native"):
        super().__init__()
        _tp_coverage(tp, input_lmax, edge_lmax)
        if layout not in ("packed", "fused_pack", 'canonical'):
            raise ValueError("Graph layout must be packed, fused_pack or canonical")
        if reduction not in ("auto", "atomic", "csr"):
            raise ValueError("Graph reduction must be auto, atomic or csr")
        if cartesian_schedule != 'native':
            raise ValueError('Only the original ICTC basis is supported; the experimental STF-coordinate schedule is retired')
        if not isinstance(edge_chunk_size, int) or isinstance(edge_chunk_size, bool) or edge_chunk_size < 1:
            raise ValueError("edge_chunk_size must be a positive integer")
        self.tp, self.input_lmax, self.edge_lmax = tp, input_lmax, edge_lmax
        self.layout, self.edge_chunk_size = layout, edge_chunk_size
        self._packed = PackedGraphMessage(tp, input_lmax=input_lmax, edge_lmax=edge_lmax)

    def forward(self, features, harmonics, gates, src, dst, mask=None):
        """features {l:[N,C,2l+1]}, harmonics {l:[E,1,2l+1]}, gates [E,P*C]."""
        _tp_coverage(self.tp, self.input_lmax, self.edge_lmax)
        if set(features) != set(range(self.input_lmax + 1)) or set(harmonics) != set(range(self.edge_lmax + 1)):
            raise ValueError("Degree dictionaries must cover declared input/edge degrees")
        _eager(features[0])
        n, e = features[0].shape[0], src.numel()
        for name, indices in (("src", src), ("dst", dst)):
            if (indices.ndim != 1 or indices.numel() != e or indices.dtype != torch.int64
                    or indices.device != self.tp.weight.device):
                raise ValueError(f"{name} must be an int64 CUDA vector of E valid node indices")
        for l, value in features.items():
            _operand(value, (n, self.tp.channels, 2 * l + 1), self.tp.weight, f"features[{l}]")
        for l, value in harmonics.items():
            _operand(value, (e, 1, 2 * l + 1), self.tp.weight, f"harmonics[{l}]")
        _operand(gates, (e, self.tp.num_paths * self.tp.channels), self.tp.weight, "gates")
        if mask is not None:
            if mask.requires_grad or tuple(mask.shape) not in ((e,), (e, 1)):
                raise ValueError("mask must be fixed and have shape [E] or [E,1]")
            _operand(mask, mask.shape, self.tp.weight, "mask")
        edge = self._packed.edge
        packed = edge.pack_input(features)
        sh = torch.cat([harmonics[l].reshape(e, 2 * l + 1) for l in range(self.edge_lmax + 1)], -1)
        out = self._packed(packed, sh, gates, src, dst, mask)
        return edge.unpack_output(out)


def direction_harmonics(directions, lmax, *, policy="auto"):
    """Component-normalized Cartesian harmonics: list of [E,2l+1] blocks (operators.py:471-490)."""
    _degree(lmax, "lmax")
    if directions.ndim != 2 or directions.shape[1] != 3:
        raise ValueError("directions must have shape [E,3]")
    if policy not in ("auto", "generated", "reference"):
        raise ValueError("Harmonic policy must be auto, generated or reference")
    if directions.device.type != "cuda" or directions.dtype != torch.float32:
        raise ValueError("Generated harmonics require eager CUDA FP32 and no autocast")
    if lmax > 3:
        raise ValueError("MI355X harmonic kernels cover lmax <= 3")
    packed = harmonics_packed(directions, lmax)
    return [packed[:, l * l:(l + 1) ** 2] for l in range(lmax + 1)]


def channel_linear(features, weight, bias=None):
    """Shared-weight channel GEMM: [*,Cin,m] x [Cout,Cin] -> [*,Cout,m] (operators.py:609-628)."""
    from ictc_o3.ops.linear import channel_linear as impl
    if features.ndim < 2 or weight.ndim != 2 or features.shape[-2] != weight.shape[1]:
        raise ValueError("Expected features [*,Cin,m] and weight [Cout,Cin]")
    if features.device != weight.device or features.dtype != weight.dtype:
        raise ValueError("Features and weights must share device and dtype")
    if bias is not None:
        if features.shape[-1] != 1:
            raise ValueError("Channel bias is allowed only for the scalar angular block")
        if bias.shape != (weight.shape[0],) or bias.device != weight.device or bias.dtype != weight.dtype:
            raise ValueError("bias must match output channel count, device and dtype")
    return impl(features, weight, bias)


def normalized_silu(features, scale=1.0):
    """SiLU times a fixed scale with first and mixed derivatives (operators.py:631-636)."""
    if not isinstance(scale, (int, float)) or isinstance(scale, bool):
        raise TypeError("scale must be a fixed numeric scalar")
    from ictc_o3.ops.activation import normalized_silu as impl
    return impl(features, float(scale))


def create_symmetric_contraction(*args, **kwargs):
    """operators.py:493-526."""
    from ictc_o3.ops.symmetric_contraction import create_symmetric_contraction as impl
    return impl(*args, **kwargs)


def configure_symmetric_contraction(module, **kwargs):
    """operators.py:529-606."""
    from ictc_o3.ops.symmetric_contraction import configure_symmetric_contraction as impl
    return impl(module, **kwargs)
