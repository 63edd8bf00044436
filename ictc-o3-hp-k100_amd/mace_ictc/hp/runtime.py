"""Whole-network entry points (reference: mace_ictc/hp/runtime.py:6-310).

create_model builds the bridge-U baseline MACE-ICTC (model.py) with the
reference factory's fixed choices (runtime.py:70-79: bessel radial basis,
polynomial cutoff p=5, no sqrt(num_basis) norm, frozen unit TP coefficients,
first-layer scalar self connection, 16-wide final readout).  configure_model
validates the reference keywords and reports the single MI355X plan.
energy_and_forces evaluates E, F = -dE/dpos and per-atom energies; the
per-graph energy sum is accumulated in FP64.
"""
from __future__ import annotations

import torch

from mace_ictc.hp.model import PureCartesianICTDFix


def create_model(*, channels=64, lmax=3, edge_lmax=None, num_interactions=2, correlation=3, use_reduced_cg=False,
                 atomic_numbers=(1, 6, 8), cutoff=5.0, avg_num_neighbors=50.0, device="cuda", dtype=torch.float32,
                 electrostatics=None):
    """Parameterized bridge-U model with initialized (not trained) weights (runtime.py:6-83)."""
    from ictc_o3.operators import _degree, _positive_integer
    if not isinstance(num_interactions, int) or isinstance(num_interactions, bool) or num_interactions < 1:
        raise ValueError("num_interactions must be a positive integer")
    _positive_integer(channels, "channels")
    _positive_integer(correlation, "correlation")
    if correlation not in (1, 2, 3):
        raise ValueError("HP correlation currently supports 1, 2, 3; cor4/5 experiments are separate")
    if not isinstance(use_reduced_cg, bool):
        raise TypeError("use_reduced_cg must be a boolean")
    if use_reduced_cg:
        raise ValueError("The independent HP factory uses native full CG; cuEq reduced-basis generation is not enabled")
    _degree(lmax, "lmax")
    edge_lmax = lmax if edge_lmax is None else edge_lmax
    _degree(edge_lmax, "edge_lmax")
    if edge_lmax < lmax:
        raise ValueError("edge_lmax must be at least lmax")
    if electrostatics is not None:
        raise ValueError("Long-range electrostatics is outside the MI355X operator build")
    if dtype != torch.float32:
        raise ValueError("The MI355X kernels compute in FP32")
    if max(lmax, edge_lmax) > 3:
        raise ValueError("The MI355X kernels cover lmax and edge_lmax <= 3")
    previous = torch.get_default_dtype()
    try:
        torch.set_default_dtype(torch.float32)
        model = PureCartesianICTDFix(channels=channels, lmax=lmax, edge_lmax=edge_lmax,
                                     num_interactions=num_interactions, correlation=correlation,
                                     atomic_numbers=atomic_numbers, cutoff=cutoff,
                                     avg_num_neighbors=avg_num_neighbors)
    finally:
        torch.set_default_dtype(previous)
    return model.to(device=device)


def energy_and_forces(model, positions, atomic_numbers, batch, edge_src, edge_dst, edge_shifts, cell, *,
                      training=False, owned_mask=None, topology=None):
    """Energy [B], forces [N,3], atomic_energy [N] of a prebuilt graph (runtime.py:86-113).

    training=True keeps the graph for force-loss mixed derivatives; inference
    returns detached results.  ``topology`` optionally reuses a prebuilt CSR
    (ictc_o3.ops.tensor_product.Topology) of the same edge list.
    """
    if torch.is_inference_mode_enabled():
        raise ValueError("Full forces require autograd; use no_grad instead of inference_mode")
    if positions.ndim != 2 or positions.shape[1] != 3 or cell.ndim != 3 or cell.shape[1:] != (3, 3):
        raise ValueError("Expected positions [N,3] and cell [B,3,3]")
    n = positions.shape[0]
    if atomic_numbers.shape != (n,) or batch.shape != (n,):
        raise ValueError("Atomic numbers and graph batch must have shape [N]")
    if owned_mask is not None and (owned_mask.shape != (n,) or owned_mask.requires_grad):
        raise ValueError("owned_mask must be a fixed [N] tensor")
    with torch.enable_grad():
        pos = positions if positions.requires_grad else positions.detach().requires_grad_(True)
        output = model(pos, atomic_numbers, batch, edge_src, edge_dst, edge_shifts, cell, topology=topology,
                       second_order=training, forces_only=not training)
        atomic = (output[0] if isinstance(output, tuple) else output).reshape(n)
        selected = atomic if owned_mask is None else atomic * owned_mask.to(atomic)
        # per-graph sums in FP64 without atomics (deterministic, contention free)
        if cell.shape[0] == 1:
            energy64 = selected.double().sum().reshape(1)
        elif selected.is_cuda and selected.dtype == torch.float32:
            from ictc_o3.ops.linear import graph_sum
            graphs = cell.shape[0]
            # Many small graphs: the contiguous-batch form is O(N + graphs) instead of O(graphs * N); the
            # one host read deciding it is paid only where the quadratic form would cost more.
            ordered = graphs > 64 and n > 1 and bool((batch[1:] >= batch[:-1]).all())
            energy64 = graph_sum(selected, batch, graphs, batch_sorted=ordered)
        else:
            onehot = torch.nn.functional.one_hot(batch, cell.shape[0]).to(torch.float64)
            energy64 = onehot.t() @ selected.double()
        force = -torch.autograd.grad(energy64.sum() + pos.sum() * 0.0, pos, create_graph=training,
                                     retain_graph=training)[0]
        energy = energy64.to(atomic.dtype)
        result = {"energy": energy, "forces": force, "atomic_energy": atomic}
        return result if training else {key: value.detach() for key, value in result.items()}


def check_model(model: torch.nn.Module, *, training=False, capture=False) -> dict:
    """Read-only coverage check (runtime.py:119-133)."""
    reasons = []
    if not isinstance(model, PureCartesianICTDFix):
        reasons.append("model is not an MI355X MACE-ICTC baseline")
    else:
        p = next(model.parameters())
        if not p.is_cuda or p.dtype != torch.float32:
            reasons.append("parameters must be FP32 on a ROCm device")
        if capture:
            reasons.append("graph capture of the whole model is not qualified; run eager")
    return {"supported": not reasons, "reasons": reasons}


_LEGACY_CHOICES = {
    "policy": ("auto", "generated", "reference"),
    "layout": ("packed", "fused_pack"),
    "wide_channel_policy": ("auto", "off"),
    "high_l_policy": ("auto", "off"),
    "reference_buffer_policy": ("auto", "device"),
    "message_schedule": ("native",),
    "graph_reduction": ("auto", "atomic", "csr"),
    "topology_backend": ("native", "device"),
    "geometry_schedule": ("auto", "native", "streamed"),
    "species_schedule": ("grouped", "indexed", "auto"),
    "mixed_geometry_schedule": ("fused", "split"),
    "training_gate_gemm_policy": ("torch", "k100_tiled"),
    "training_message_linear_layout": ("node_component", "einsum"),
    "inference_message_layout": ("native", "degree"),
    "inference_gemm_policy": ("torch", "dtk2604"),
    "species_linear_schedule": ("auto", "grouped", "gather"),
    "electrostatics_backend": ("auto", "hip", "reference"),
}


def configure_model(model: torch.nn.Module, *, training=False, policy="auto", layout="packed", gate_cache_bytes=0,
                    capture=False, wide_channel_policy="auto", high_l_policy="auto", reference_buffer_policy="auto",
                    message_schedule="native", graph_reduction="auto", topology_backend="native",
                    csr_accumulator_limit=None, csr_slice_search=False, geometry_schedule="auto",
                    message_chunk_edges=None, species_schedule="grouped", training_gate_schedule="materialized",
                    mixed_channel_tile=None, mixed_geometry_schedule="fused", training_gate_gemm_policy="torch",
                    training_adjoint_channel_tile=None, training_message_linear_layout="node_component",
                    radial_checkpoint=False, inference_message_layout="native", inference_adjoint_channel_tile="auto",
                    inference_gate_adjoint_rows=0, inference_gemm_policy="torch", inference_message_adjoint_edges=0,
                    inference_basis_fusion=False, species_linear_schedule="auto", electrostatics_backend="auto",
                    plan=None, foundation_config=None) -> dict:
    """Validate the reference's runtime keywords and report the MI355X plan (runtime.py:136-310).

    The MI355X build has one qualified route per operator (receiver-sorted CSR
    message, generated SC circuit, HIP harmonics / radial / SiLU), so the
    schedule keywords are validated and echoed; no parameter, dtype or
    trainability is changed.
    """
    values = dict(policy=policy, layout=layout, wide_channel_policy=wide_channel_policy, high_l_policy=high_l_policy,
                  reference_buffer_policy=reference_buffer_policy, message_schedule=message_schedule,
                  graph_reduction=graph_reduction, topology_backend=topology_backend,
                  geometry_schedule=geometry_schedule, species_schedule=species_schedule,
                  mixed_geometry_schedule=mixed_geometry_schedule, training_gate_gemm_policy=training_gate_gemm_policy,
                  training_message_linear_layout=training_message_linear_layout,
                  inference_message_layout=inference_message_layout, inference_gemm_policy=inference_gemm_policy,
                  species_linear_schedule=species_linear_schedule, electrostatics_backend=electrostatics_backend)
    for key, value in values.items():
        if value not in _LEGACY_CHOICES[key]:
            raise ValueError(f"{key} must be one of {_LEGACY_CHOICES[key]}")
    for key, value in (("training", training), ("capture", capture), ("csr_slice_search", csr_slice_search),
                       ("radial_checkpoint", radial_checkpoint)):
        if not isinstance(value, bool):
            raise TypeError(f"{key} must be a boolean")
    if not isinstance(gate_cache_bytes, int) or isinstance(gate_cache_bytes, bool) or gate_cache_bytes < 0:
        raise ValueError("gate_cache_bytes must be a nonnegative integer")
    if training and gate_cache_bytes:
        raise ValueError("Training requires gate_cache_bytes=0")
    schedules = training_gate_schedule if isinstance(training_gate_schedule, (list, tuple)) else [training_gate_schedule]
    if any(s not in ("materialized", "cached", "recompute") for s in schedules):
        raise ValueError("training_gate_schedule must be materialized, cached or recompute")
    if plan is not None:
        raise ValueError("RuntimePlan objects are not part of the MI355X build; pass keywords")
    if foundation_config is not None:
        raise ValueError("foundation_config requires a FoundationTrainHP model")
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    check = check_model(model, training=training, capture=capture)
    selected = "generated" if check["supported"] and policy != "reference" else "reference"
    if policy == "generated" and not check["supported"]:
        raise ValueError("; ".join(check["reasons"]))
    n_inter = len(getattr(model, "interactions", ()))
    return {
        "selected": selected,
        "reasons": check["reasons"],
        "training": training,
        "layout": layout,
        "message_schedule": message_schedule if selected == "generated" else "reference",
        "graph_reduction": "csr" if selected == "generated" else "reference",
        "topology_backend": "native",
        "species_schedule": species_schedule if selected == "generated" else "reference",
        "species_linear_schedule": species_linear_schedule if selected == "generated" else "reference",
        "training_gate_schedule": "materialized",
        "training_message_linear_layout": training_message_linear_layout if training else "einsum",
        "counts": {"interactions": n_inter, "products": len(getattr(model, "products", ()))},
        "device_adaptations": {
            "target": "gfx950",
            "native_hip": ["direction_harmonics", "radial_basis", "normalized_silu", "tp_csr_forward",
                           "tp_adjoint_receiver", "tp_adjoint_source", "tp_mixed_second", "csr_topology",
                           "species_circuit", "species_circuit_mixed", "species_bank_reduce"],
            "library_gemm": ["radial_mlp", "linear_up", "message_linear", "self_connection", "product_linear"],
        },
    }
