"""Bridge-U symmetric contraction (correlation 1..3) on the HIP kernels.

Public surface follows the reference:
  * ``ICTDBridgeUSymmetricContractionSO3`` (ictc_o3/ops/symmetric_contraction.py:8-158):
    ``symmetric_contractions.contractions[L]`` with parameters ``weights_max``
    [S, P_corr, C] and ``weights[j]`` [S, P_{corr-1-j}, C]
    (ictc_o3/ops/_mace_symmetric_contraction.py:140-201) and buffers
    ``U_matrix_{nu}`` (bridge folded in), ``basis_bridge.q_{l}``;
  * ``create_symmetric_contraction`` / ``configure_symmetric_contraction``
    (ictc_o3/operators.py:493-606) with the same validation and info keys.

``forward(node_feats, node_attrs, node_type_idx=None)`` takes the reference's
flat mul_ir layout ([C, 2l+1] per degree) and returns the same layout;
``contract(x, species)`` is the native entry on the packed ir_mul layout
([2l+1, C] per degree) used by the MACE model.
"""
from __future__ import annotations

import ctypes
from typing import Dict, List

import torch
import torch.nn as nn
from torch.autograd.function import once_differentiable

from ictc_o3 import _native as nat
from ictc_o3.autograd import required_gradients
from ictc_o3.basis import e3nn_basis


def sc_shape(lmax, target_lmax, correlation):
    paths = (ctypes.c_int * 12)()
    nw = ctypes.c_int()
    nat.call("ictc_sc_shape", lmax, target_lmax, correlation, paths, ctypes.byref(nw))
    return [[paths[L * 3 + n] for n in range(3)] for L in range(4)], nw.value


class ScSpec:
    def __init__(self, lmax, target_lmax, correlation, channels, num_species):
        self.lmax, self.target_lmax, self.corr = lmax, target_lmax, correlation
        self.channels, self.num_species = channels, num_species
        self.paths, self.num_weights = sc_shape(lmax, target_lmax, correlation)
        self.nx = (lmax + 1) ** 2
        self.no = sum(2 * L + 1 for L in range(target_lmax + 1))
        # flattened (L, nu) slots that carry weights, in table order
        self.slots = [(L, n) for L in range(target_lmax + 1) for n in range(correlation) if self.paths[L][n] > 0]


def _table(spec, tensors):
    """12-entry pointer table (index L*3 + nu-1) from the slot-ordered tensors."""
    arr = (ctypes.c_void_p * 12)()
    for (L, n), t in zip(spec.slots, tensors):
        arr[L * 3 + n] = t.data_ptr() if t is not None else None
    return arr


class _SpeciesCsr:
    def __init__(self, species, num_species):
        from ictc_o3.ops.tensor_product import Csr
        self.csr = Csr(species, num_species)


def _c(t):
    return t if t.is_contiguous() else t.contiguous()


def term_count(spec) -> int:
    """Monomial x weight terms per (node, channel) of the generated forward (2 FLOPs each)."""
    n = int(nat.lib().ictc_sc_terms(spec.lmax, spec.target_lmax, spec.corr))
    if n < 0:
        raise ValueError(nat.lib().ictc_last_error().decode(errors="replace"))
    return n


def _fwd_raw(spec, x, species, ws, tangent=None):
    out = x.new_empty(x.shape[0], spec.no * spec.channels)
    if tangent is None:
        nat.call("ictc_sc_fwd", spec.lmax, spec.target_lmax, spec.corr, spec.channels, nat.ptr(x), nat.ptr(species),
                 spec.num_species, _table(spec, ws), x.shape[0], nat.ptr(out), nat.stream_of(x))
    else:
        nat.call("ictc_sc_jvp", spec.lmax, spec.target_lmax, spec.corr, spec.channels, nat.ptr(x), nat.ptr(species),
                 spec.num_species, _table(spec, ws), x.shape[0], nat.ptr(tangent), nat.ptr(out), nat.stream_of(x))
    return out


def _dx_raw(spec, x, species, ws, go, tangent=None):
    dx = torch.empty_like(x)
    if tangent is None:
        nat.call("ictc_sc_bwd_x", spec.lmax, spec.target_lmax, spec.corr, spec.channels, nat.ptr(x),
                 nat.ptr(species), spec.num_species, _table(spec, ws), x.shape[0], nat.ptr(go), nat.ptr(dx),
                 nat.stream_of(x))
    else:
        nat.call("ictc_sc_hvp", spec.lmax, spec.target_lmax, spec.corr, spec.channels, nat.ptr(x),
                 nat.ptr(species), spec.num_species, _table(spec, ws), x.shape[0], nat.ptr(go), nat.ptr(tangent),
                 nat.ptr(dx), nat.stream_of(x))
    return dx


def _dw_raw(spec, x, species_csr, go, tangent=None):
    N = x.shape[0]
    dws = [x.new_empty(spec.num_species, spec.paths[L][n], spec.channels) for L, n in spec.slots]
    ws_bytes = int(nat.lib().ictc_sc_workspace_bytes(spec.lmax, spec.target_lmax, spec.corr, spec.channels, N,
                                                     spec.num_species))
    work = x.new_empty(max(ws_bytes // 4, 1))
    csr = species_csr.csr
    table = (ctypes.c_void_p * 12)()
    for (L, n), t in zip(spec.slots, dws):
        table[L * 3 + n] = t.data_ptr()
    if tangent is None:
        nat.call("ictc_sc_bwd_w", spec.lmax, spec.target_lmax, spec.corr, spec.channels, nat.ptr(x),
                 spec.num_species, N, nat.ptr(go), nat.ptr(csr.ptr), nat.ptr(csr.order), table, nat.ptr(work),
                 ws_bytes, nat.stream_of(x))
    else:
        nat.call("ictc_sc_bwd_w_jvp", spec.lmax, spec.target_lmax, spec.corr, spec.channels, nat.ptr(x),
                 spec.num_species, N, nat.ptr(go), nat.ptr(tangent), nat.ptr(csr.ptr), nat.ptr(csr.order), table,
                 nat.ptr(work), ws_bytes, nat.stream_of(x))
    return dws


class _SC(torch.autograd.Function):
    @staticmethod
    def forward(ctx, spec, species, holder, x, *ws):
        ctx.set_materialize_grads(False)
        ctx.spec, ctx.species, ctx.holder = spec, species, holder
        x = _c(x)
        ws = tuple(_c(w) for w in ws)
        ctx.save_for_backward(x, *ws)
        return _fwd_raw(spec, x, species, ws)

    @staticmethod
    def backward(ctx, go):
        if go is None:
            return (None,) * (4 + len(ctx.spec.slots))
        x, *ws = ctx.saved_tensors
        needs = required_gradients((x, *ws), ctx.needs_input_grad[3:])
        need_x = needs[0]
        need_w = any(needs[1:])
        grads = _SCAdjoint.apply(ctx.spec, ctx.species, ctx.holder, need_x, need_w, x, _c(go), *ws)
        return (None, None, None, *grads)


class _SCAdjoint(torch.autograd.Function):
    @staticmethod
    def forward(ctx, spec, species, holder, need_x, need_w, x, go, *ws):
        ctx.set_materialize_grads(False)
        ctx.spec, ctx.species, ctx.holder = spec, species, holder
        ctx.save_for_backward(x, go, *ws)
        dx = _dx_raw(spec, x, species, ws, go) if need_x else None
        dws = _dw_raw(spec, x, holder.species_csr(), go) if need_w else [None] * len(ws)
        return (dx, *dws)

    @staticmethod
    @once_differentiable
    def backward(ctx, hdx, *hdws):
        x, go, *ws = ctx.saved_tensors
        spec, species, holder = ctx.spec, ctx.species, ctx.holder
        needs = required_gradients((x, go, *ws), ctx.needs_input_grad[5:])
        n_x, n_go = needs[0], needs[1]
        n_w = needs[2:]
        have_hw = any(h is not None for h in hdws)
        hws = tuple(h if h is not None else torch.zeros_like(w) for h, w in zip(hdws, ws)) if have_hw else None
        dx = dgo = None
        dws = [None] * len(ws)
        if n_go:
            if hdx is not None:
                dgo = _fwd_raw(spec, x, species, ws, tangent=_c(hdx))
            if have_hw:
                t = _fwd_raw(spec, x, species, hws)
                dgo = t if dgo is None else dgo + t
        if n_x:
            if hdx is not None:
                dx = _dx_raw(spec, x, species, ws, go, tangent=_c(hdx))
            if have_hw:
                t = _dx_raw(spec, x, species, hws, go)
                dx = t if dx is None else dx + t
        if any(n_w) and hdx is not None:
            dws = _dw_raw(spec, x, holder.species_csr(), go, tangent=_c(hdx))
        return (None, None, None, None, None, dx, dgo, *dws)


class _SpeciesHolder:
    """Lazily built species-sorted node CSR, shared by the adjoints of one forward call."""

    def __init__(self, species, num_species):
        self.species, self.num_species, self._csr = species, num_species, None

    def species_csr(self):
        if self._csr is None:
            self._csr = _SpeciesCsr(self.species, self.num_species)
        return self._csr


def symmetric_contraction(x, species, weights: List[torch.Tensor], spec: ScSpec):
    """x [N, NX*C] packed ir_mul, species [N] int64, weights in spec.slots order -> [N, NO*C] packed ir_mul."""
    holder = _SpeciesHolder(species, spec.num_species)
    return _SC.apply(spec, species, holder, x, *weights)


# ---------------------------------------------------------------------------
# Modules (parameter names and layouts of the reference)
# ---------------------------------------------------------------------------


class _Contraction(nn.Module):
    """Per-output-irrep holder: weights_max [S, P_corr, C], weights[j] [S, P_{corr-1-j}, C]."""

    def __init__(self, lmax, l_out, correlation, num_elements, channels):
        super().__init__()
        self.correlation, self.output_lmax, self.num_features = correlation, l_out, channels
        for nu in range(1, correlation + 1):
            U = torch.tensor(e3nn_basis.mace_u_ictc(lmax, l_out, nu), dtype=torch.get_default_dtype())
            self.register_buffer(f"U_matrix_{nu}", U)
        P = [getattr(self, f"U_matrix_{nu}").shape[-1] for nu in range(1, correlation + 1)]
        self.weights_max = nn.Parameter(torch.randn(num_elements, P[-1], channels) / max(P[-1], 1))
        self.weights = nn.ParameterList([nn.Parameter(torch.randn(num_elements, P[nu - 1], channels) / max(P[nu - 1], 1))
                                         for nu in range(correlation - 1, 0, -1)])

    def weight_for(self, nu):
        return self.weights_max if nu == self.correlation else self.weights[self.correlation - 1 - nu]


class MaceSymmetricContraction(nn.Module):
    def __init__(self, lmax, target_lmax, correlation, num_elements, channels):
        super().__init__()
        self.contractions = nn.ModuleList([_Contraction(lmax, L, correlation, num_elements, channels)
                                           for L in range(target_lmax + 1)])


class SO3ToE3NNBasisBridge(nn.Module):
    """Fixed per-degree orthogonal bridge buffers q_l (bridge.py:26-62)."""

    def __init__(self, channels, lmax):
        super().__init__()
        self.channels, self.lmax = channels, lmax
        for l in range(lmax + 1):
            self.register_buffer(f"q_{l}", torch.tensor(e3nn_basis.bridge_q(l), dtype=torch.get_default_dtype()))


class ICTDBridgeUSymmetricContractionSO3(nn.Module):
    def __init__(self, *, num_elements, channels, lmax, target_lmax, correlation=3, use_reduced_cg=False):
        super().__init__()
        if use_reduced_cg:
            raise ValueError("The independent HP factory uses native full CG; cuEq reduced-basis generation is not enabled")
        self.channels, self.lmax, self.target_lmax = int(channels), int(lmax), int(target_lmax)
        self.correlation, self.num_elements = int(correlation), int(num_elements)
        self.use_reduced_cg = False
        self.basis_bridge = SO3ToE3NNBasisBridge(self.channels, max(self.lmax, self.target_lmax))
        self.symmetric_contractions = MaceSymmetricContraction(self.lmax, self.target_lmax, self.correlation,
                                                               self.num_elements, self.channels)
        self._spec = None
        self._configured = {}

    def spec(self):
        if self._spec is None:
            self._spec = ScSpec(self.lmax, self.target_lmax, self.correlation, self.channels, self.num_elements)
        return self._spec

    def slot_weights(self):
        spec = self.spec()
        return [self.symmetric_contractions.contractions[L].weight_for(n + 1) for L, n in spec.slots]

    def contract(self, x, species):
        """Native entry: x [N, (lmax+1)^2*C] packed ir_mul -> [N, sum_L (2L+1)*C] packed ir_mul."""
        return symmetric_contraction(x, species, self.slot_weights(), self.spec())

    def forward(self, node_feats, node_attrs=None, node_type_idx=None):
        """Reference layout: flat mul_ir in and out (symmetric_contraction.py:98-147)."""
        N, C = node_feats.shape[0], self.channels
        if node_type_idx is None:
            if node_attrs is None:
                raise ValueError("node_attrs or node_type_idx is required")
            node_type_idx = node_attrs.argmax(-1)
        if (node_type_idx.shape != (N,) or node_type_idx.dtype != torch.int64
                or node_type_idx.device != node_feats.device):
            raise ValueError('Species indices must be int64 [N] on the feature device')
        x = _mul_ir_to_ir_mul(node_feats, C, self.lmax)
        out = self.contract(x, node_type_idx.contiguous())
        return _ir_mul_to_mul_ir(out, C, self.target_lmax)


def _mul_ir_to_ir_mul(x, C, lmax):
    parts, off = [], 0
    for l in range(lmax + 1):
        w = C * (2 * l + 1)
        parts.append(x[:, off:off + w].reshape(-1, C, 2 * l + 1).transpose(1, 2).reshape(-1, w))
        off += w
    return torch.cat(parts, -1).contiguous()


def _ir_mul_to_mul_ir(x, C, lmax):
    parts, off = [], 0
    for l in range(lmax + 1):
        w = C * (2 * l + 1)
        parts.append(x[:, off:off + w].reshape(-1, 2 * l + 1, C).transpose(1, 2).reshape(-1, w))
        off += w
    return torch.cat(parts, -1)


# ---------------------------------------------------------------------------
# Factories (operators.py:493-606)
# ---------------------------------------------------------------------------


def create_symmetric_contraction(*, num_elements, lmax, target_lmax=None, channels=64, correlation=3,
                                 use_reduced_cg=False, device="cuda", policy="generated", high_l_policy="auto",
                                 training=False, reference_buffer_policy="auto", species_schedule="auto",
                                 inference_basis_fusion="auto"):
    from ictc_o3.operators import _degree, _positive_integer
    _degree(lmax, "lmax")
    _positive_integer(channels, "channels")
    _positive_integer(correlation, "correlation")
    if correlation not in (1, 2, 3):
        raise ValueError("HP correlation currently supports 1, 2, 3; cor4/5 experiments are separate")
    if not isinstance(use_reduced_cg, bool):
        raise TypeError("use_reduced_cg must be a boolean")
    if use_reduced_cg:
        raise ValueError("The independent HP factory uses native full CG; cuEq reduced-basis generation is not enabled")
    target_lmax = lmax if target_lmax is None else target_lmax
    _degree(target_lmax, "target_lmax")
    if not isinstance(num_elements, int) or isinstance(num_elements, bool) or num_elements < 1:
        raise ValueError("num_elements must be a positive integer")
    module = ICTDBridgeUSymmetricContractionSO3(num_elements=num_elements, channels=channels, lmax=lmax,
                                                target_lmax=target_lmax, correlation=correlation,
                                                use_reduced_cg=use_reduced_cg).to(device=device, dtype=torch.float32)
    configure_symmetric_contraction(module, policy=policy, high_l_policy=high_l_policy, training=training,
                                    reference_buffer_policy=reference_buffer_policy,
                                    species_schedule=species_schedule, inference_basis_fusion=inference_basis_fusion)
    return module


def configure_symmetric_contraction(module, *, policy="auto", high_l_policy="auto", training=False,
                                    reference_buffer_policy="auto", species_schedule="auto",
                                    inference_basis_fusion="auto"):
    """Validate and report the plan; the MI355X build has one route (the generated circuit)."""
    if not isinstance(module, ICTDBridgeUSymmetricContractionSO3):
        raise TypeError("Expected ICTDBridgeUSymmetricContractionSO3")
    if policy not in ("auto", "generated", "reference"):
        raise ValueError("SC policy must be auto, generated or reference")
    if high_l_policy not in ("auto", "off"):
        raise ValueError("high_l_policy must be auto or off")
    if species_schedule not in ('auto', 'grouped', 'indexed'):
        raise ValueError('species_schedule must be auto, grouped or indexed')
    if not (isinstance(inference_basis_fusion, bool) or inference_basis_fusion == 'auto'):
        raise ValueError('inference_basis_fusion must be auto or a boolean')
    if not isinstance(training, bool):
        raise TypeError("training must be a boolean")
    if reference_buffer_policy not in ('auto', 'device'):
        raise ValueError('reference_buffer_policy must be auto or device')
    parameter = next(module.parameters())
    supported = (parameter.is_cuda and parameter.dtype == torch.float32 and module.channels > 0
                 and module.correlation in (1, 2, 3) and (module.lmax, module.target_lmax) in _COMPILED)
    if policy == "generated" and not supported:
        raise ValueError("Generated SC requires CUDA FP32 and a positive-order bridge-U contraction")
    module._configured = {"policy": policy, "training": training}
    return {"selected": "generated" if supported and policy != "reference" else "reference",
            "high_l_policy": high_l_policy, "species_schedule": species_schedule,
            "indexed_species_active": bool(supported), "inference_basis_fusion": inference_basis_fusion,
            "basis_fusion_active": bool(supported), "reference_buffer_policy": reference_buffer_policy,
            "sc_schedule": "circuit" if supported else "reference",
            "reasons": [] if supported or policy == "reference" else ["outside qualified standalone SC coverage"]}


_COMPILED = {(li, lt) for li in range(3) for lt in range(li + 1)} | {(3, 0), (3, 1), (3, 2)}
