"""Benchmark of the ICTC-O3 MI355X hot path (one JSON line on stdout).

Default workload ``cfg4`` (the config the headline
metric is quoted on): full MACE-ICTC energy + forces, C64 / lmax 2 /
2 interactions / correlation 3 / cutoff 4.5 A / 8 Bessel radial basis,
random-init weights, 3 species uniformly assigned; 131,072 atoms = FCC 32^3
at 0.1 atoms/A^3 (a = 3.420 A) jittered +-0.3 A (seeded).  One step = GPU
neighbour-list rebuild + E + F = -dE/dpos (an MD-style step).  value =
atom-steps/s = atoms / step time.

Workload ``cfg2``: graph message + aggregation,
4,096 atoms uniform in a periodic cube at 0.1 atoms/A^3, cutoff 4.5 A
(~156k directed edges, sorted by receiver), C64 / lmax 2 (11 paths),
radial 8-Bessel x polynomial cutoff (p=5) -> MLP 8-64-64-64-704 (SiLU) gates.
One step = radial MLP -> gates -> CSR message forward -> backward to
(features, harmonics, gates, radial weights), all on the GPU.  Inputs are
resident in HBM before the timed region.

Roofline: the step's layer-1 kernels (radial gates with their r tangents,
message forward, gate-tangent message adjoint) are timed inside five real
steps after the timed ones, with HIP events recorded around each launch on
the stream it runs on (torch's current stream; ictc_o3._timing), averaged
over those launches; the one with the largest time is the roofline kernel: its
algorithmic bytes (compulsory traffic: each operand read once, each output
written once, index arrays included, gathers not counted; the message kernels
counted per edge with one gate row each, the gate kernel per computed row) /
time vs 8 TB/s.  ``frac_shared_gate_rows`` is the same time against the
message kernels' bytes with each gate row shared by an edge and its reverse
counted once.  ``roofline_kernels`` lists all of them.

CPU baseline: the FP32 torch-eager restatement of the reference path
(oracle/: gather, per-path CG einsum, gate, index_add, SC recursion, linears,
autograd backward) on the host cores, timed on a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ictc-o3-hp-k100_amd"))

HBM_PEAK_GBS = 8000.0
FP32_PEAK_TFLOPS = 157.3
METRIC = "atom-steps/s (E+F, 1 GPU) C64/lmax2 MACE; TP edges/s & % HBM roofline"
# HBM bytes per launch of the cfg4 layer-1 message kernels (P11, C64, E=5,262,704; msg_bwd_x in
# the Morton source order the model uses), from rocprofv3 FETCH_SIZE + WRITE_SIZE runs of
# `bench.py --workload probe`, each scaled by the counter's reading for a 1 GiB copy (FETCH x2.0,
# WRITE x1.0); see profiles/msg_cfg4_hbm_traffic.md.  msg_fwd, msg_bwd_tan and gates_tan are the step's
# forms: gates shared by each edge and its reverse (2,631,352 gate rows), measured in the cfg4 step
# (profiles/step_cfg4_hbm_traffic.md).
MEASURED_TRAFFIC = {("msg_fwd", 131072, 5262704, 64): 19.65e9, ("msg_bwd_edge", 131072, 5262704, 64): 37.16e9,
                    ("msg_bwd_x", 131072, 5262704, 64): 31.91e9, ("msg_bwd", 131072, 5262704, 64): 61.18e9,
                    ("msg_bwd_tan", 131072, 5262704, 64): 42.93e9, ("gates_tan", 131072, 5262704, 64): 14.87e9}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def periodic_graph(n_atoms, density, cutoff, seed, device):
    """Uniform random positions in a periodic cube; all directed pairs within cutoff, sorted by receiver."""
    import torch
    L = (n_atoms / density) ** (1.0 / 3.0)
    g = torch.Generator(device="cpu").manual_seed(seed)
    pos = (torch.rand(n_atoms, 3, generator=g, dtype=torch.float64) * L).to(device)
    src_l, dst_l, vec_l = [], [], []
    chunk = 1024
    for s in range(0, n_atoms, chunk):
        d = pos[None, :, :] - pos[s:s + chunk, None, :]          # [c, N, 3]: pos[dst] - pos[src]
        d = d - L * torch.round(d / L)
        r = d.norm(dim=-1)
        src, dst = torch.nonzero((r < cutoff) & (r > 1e-9), as_tuple=True)
        src_l.append(src + s)
        dst_l.append(dst)
        vec_l.append(d[src, dst])
    src, dst, vec = torch.cat(src_l), torch.cat(dst_l), torch.cat(vec_l)
    order = torch.argsort(dst, stable=True)
    return pos, src[order], dst[order], vec[order].float(), L


def radial_basis(r, r_max, n_basis=8, p=5):
    """Bessel sqrt(2/r_max) sin(n pi r / r_max) / r times the MACE polynomial cutoff (radial_basis.py:11-92)."""
    import torch
    n = torch.arange(1, n_basis + 1, device=r.device, dtype=r.dtype)
    emb = math.sqrt(2.0 / r_max) * torch.sin(r[:, None] * n * math.pi / r_max) / r[:, None]
    x = r / r_max
    env = (1.0 - (p + 1) * (p + 2) / 2 * x ** p + p * (p + 2) * x ** (p + 1) - p * (p + 1) / 2 * x ** (p + 2))
    return emb * (env * (r < r_max))[:, None]


def message_bytes(N, E, C, NX, NY, P, NO, G=None):
    """Algorithmic HBM bytes of the message kernels; G = rows of gates shared through gate_rows (None = E, one
    row per edge; otherwise the gate-reading forms read G rows plus the int32 gate_rows map)."""
    idx = E * 8 + (N + 2) * 4 + E * 4
    gread = E * P * C * 4 if G is None else G * P * C * 4 + E * 4
    fwd = N * NX * C * 4 + E * NY * 4 + gread + idx + N * NO * C * 4
    bwd_edge = N * NO * C * 4 + N * NX * C * 4 + E * NY * 4 + E * P * C * 4 + idx + E * NY * 4 + E * P * C * 4
    bwd_x = N * NO * C * 4 + E * NY * 4 + E * P * C * 4 + idx + N * NX * C * 4
    # the complete adjoint (dx, dsh, dg) of one source-owned pass: every operand read once, every output written once
    bwd = N * NO * C * 4 + N * NX * C * 4 + E * NY * 4 + E * P * C * 4 + idx + E * NY * 4 + E * P * C * 4 \
        + N * NX * C * 4
    # gate-tangent form of the complete adjoint (energy + forces): gates and gdot read (G rows each, through one
    # gate_rows map), dr [E] written, no dg
    bwd_tan = bwd - 2 * E * P * C * 4 + (2 * E * P * C * 4 if G is None else 2 * G * P * C * 4 + E * 4) + E * 4
    return {"msg_fwd": fwd, "msg_bwd_edge": bwd_edge, "msg_bwd_x": bwd_x, "msg_bwd": bwd, "msg_bwd_tan": bwd_tan}


def time_launches(fn, reps, stream):
    import torch
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(reps):
        fn()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / reps * 1e-3


def host_cpu():
    """CPU model of the host (first 'model name' of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_cpu(step, warmup=3, runs=5):
    """The reference's CPU protocol: `warmup` untimed steps, then the median of `runs` timed steps (s)."""
    for _ in range(warmup):
        step()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def cpu_record(value, unit, sample):
    import torch
    return {"value": value, "unit": unit, "cores": torch.get_num_threads(), "kind": "port",
            "cpu": host_cpu(), "threads": torch.get_num_threads(),
            "sample": sample + f", {host_cpu()}, {torch.get_num_threads()} torch threads, 3 warm-up steps then "
                               "the median of 5"}


def cpu_baseline(data, budget_s=20.0):
    """Reference-path CPU eager (FP32 torch on host cores) on a bounded sample of receivers."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ictc_oracle as orc
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    x, sh, gates, src, dst, N, C = data
    # bounded sample: the edges of the first K receivers (edges are receiver-sorted)
    E = src.numel()
    take = min(E, 40000)
    xs, shs, gs = x.cpu(), sh[:take].cpu(), gates[:take].cpu()
    ss, ds = src[:take].cpu(), dst[:take].cpu()

    def step():
        a = xs.clone().requires_grad_(True)
        b = shs.clone().requires_grad_(True)
        c = gs.clone().requires_grad_(True)
        out = orc.message_packed(a, b, c, ss, ds, None, 2, 2, 2, C)
        out.backward(torch.ones_like(out))
    med = time_cpu(step)
    return cpu_record(take / med, "edges/s", f"message fwd+bwd (oracle FP32 torch eager) on the first {take} "
                      "receiver-sorted edges of the cfg2 graph")


def run_cfg2(args):
    import torch
    from ictc_o3 import PackedGraphMessage, direction_harmonics
    from ictc_o3.ops import tensor_product as tpo
    dev = torch.device("cuda:0")
    torch.backends.cuda.matmul.allow_tf32 = False
    C, cutoff = 64, 4.5
    pos, src, dst, vec, L = periodic_graph(4096, 0.1, cutoff, 1234, dev)
    N, E = pos.shape[0], src.numel()
    log(f"cfg2: N={N} E={E} box={L:.2f}")
    op = PackedGraphMessage.create(channels=C, input_lmax=2, edge_lmax=2, output_lmax=2, device=dev)
    P, NO = op.tp.num_paths, op.output_width // C
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(N, C * 9, device=dev, generator=g).requires_grad_(True)
    r = vec.norm(dim=1)
    n = vec / r[:, None]
    sh = torch.cat(direction_harmonics(n, 2), -1).detach().requires_grad_(True)
    rb = radial_basis(r, cutoff)
    widths = [8, 64, 64, 64, P * C]
    Ws = [(torch.randn(o, i, device=dev, generator=g) / math.sqrt(i)).requires_grad_(True)
          for i, o in zip(widths[:-1], widths[1:])]
    go = torch.randn(N, op.output_width, device=dev, generator=g)
    topo = tpo.Topology(src, dst, N, positions=pos)

    from ictc_o3.ops.radial_mlp import _RadialGates

    def mlp(_rb):
        # the library's fused radial path: Bessel x cutoff basis, 3 SiLU layers and the gate projection in one
        # kernel; its adjoint gives the MLP weight gradients
        return _RadialGates.apply(r, *Ws, cutoff, 5, 1.6791767923989418)

    def step():
        gates = mlp(rb)
        out = op(x, sh, gates, src, dst, topology=topo)
        torch.autograd.backward(out, go)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps

    # live kernel timing on the stream the kernels run on
    stream = torch.cuda.current_stream(dev)
    gates = mlp(rb).detach()
    spec = op.edge._prepare()
    xd, shd = x.detach(), sh.detach()
    t_fwd = time_launches(lambda: tpo._msg_fwd_raw(spec, topo, xd, shd, gates, None), 20, stream)
    t_bwd_e = time_launches(lambda: tpo._msg_bwd_raw(spec, topo, xd, shd, gates, None, go, (False, True, True)),
                            20, stream)
    topo.by_src
    t_bwd_x = time_launches(lambda: tpo._msg_bwd_raw(spec, topo, xd, shd, gates, None, go, (True, False, False)),
                            20, stream)
    nbytes = message_bytes(N, E, C, 9, 9, P, NO)
    t_bwd = time_launches(lambda: tpo._msg_bwd_raw(spec, topo, xd, shd, gates, None, go, (True, True, True)), 20,
                          stream)
    kern = {"msg_fwd": t_fwd, "msg_bwd_edge": t_bwd_e, "msg_bwd_x": t_bwd_x}
    if t_bwd < 0.9 * (t_bwd_e + t_bwd_x):   # the step's backward: one fused source-owned kernel
        kern["msg_bwd"] = t_bwd
    for k, t in kern.items():
        log(f"  {k}: {t * 1e6:.1f} us  {nbytes[k] / t / 1e9:.0f} GB/s ({nbytes[k] / 1e6:.1f} MB)")
    dom = max(kern, key=kern.get)
    achieved = nbytes[dom] / kern[dom] / 1e9
    result = {
        "metric": METRIC,
        "value": E / dt, "unit": "edges/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": dt * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32", "data": "synthetic (seeded uniform periodic positions, N(0,1) features, random-init MLP)",
        "config": {"workload": "cfg2: graph message + aggregation fwd+bwd, 4096 atoms, 0.1/A^3, rc 4.5 A, "
                               "C64 lmax2 (11 paths), radial MLP 8-64-64-64-704",
                   "atoms": N, "edges": E, "channels": C, "lmax": 2,
                   "atom_steps_per_s": N / dt,
                   "kernel_us": {k: round(t * 1e6, 2) for k, t in kern.items()},
                   "kernel_algorithmic_MB": {k: round(v / 1e6, 2) for k, v in nbytes.items()}},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None},
    }
    return result, (xd, shd, gates, src, dst, N, C)


def fcc_system(n, density, jitter, seed, species_count, device):
    import torch
    g = torch.Generator().manual_seed(seed)
    a = (4.0 / density) ** (1.0 / 3.0)
    base = torch.tensor([[0, 0, 0], [0.5, 0.5, 0], [0.5, 0, 0.5], [0, 0.5, 0.5]], dtype=torch.float64)
    grid = torch.stack(torch.meshgrid(*[torch.arange(n)] * 3, indexing="ij"), -1).reshape(-1, 3).double()
    pos = (grid[:, None, :] + base[None]).reshape(-1, 3) * a
    pos = pos + (torch.rand(pos.shape, generator=g, dtype=torch.float64) * 2 - 1) * jitter
    Z = torch.tensor([1, 6, 8])[torch.randint(0, species_count, (pos.shape[0],), generator=g)]
    cell = (torch.eye(3, dtype=torch.float64) * a * n)[None]
    return pos.float().to(device), Z.to(device), cell.float().to(device), a


def cpu_baseline_model(model, budget_s=25.0):
    """Reference-path CPU eager (FP32 torch on host cores): E+F of a 2,048-atom FCC sample of cfg4."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import model_oracle as mo
    from mace_ictc.hp import radius_graph_pbc
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    pos, Z, cell, _ = fcc_system(8, 0.1, 0.3, 99, 3, "cpu")
    src, dst, sh = radius_graph_pbc(pos, cell[0], 4.5)
    batch = torch.zeros(pos.shape[0], dtype=torch.long)
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    cfg = mo.config_of(model)

    def step():
        s2, d2, sh2 = radius_graph_pbc(pos, cell[0], 4.5)
        mo.energy_and_forces(sd, cfg, pos, Z, batch, s2, d2, sh2, cell, 1, dtype=torch.float32)
    med = time_cpu(step)
    return cpu_record(pos.shape[0] / med, "atom-steps/s", f"cfg4 model (same weights) E+F incl. neighbour list "
                      f"on a 2,048-atom FCC 8^3 sample (E={src.numel()}), oracle FP32 torch eager")


def run_cfg4(args):
    import torch
    from mace_ictc.hp import create_model, energy_and_forces, radius_graph_pbc
    from ictc_o3.ops import tensor_product as tpo
    dev = torch.device("cuda:0")
    torch.manual_seed(2024)
    model = create_model(channels=64, lmax=2, num_interactions=2, correlation=3, atomic_numbers=(1, 6, 8),
                         cutoff=4.5, avg_num_neighbors=42.0, device=dev)
    pos, Z, cell, a = fcc_system(32, 0.1, 0.3, 1234, 3, dev)
    N = pos.shape[0]
    batch = torch.zeros(N, dtype=torch.long, device=dev)

    def step():
        src, dst, sh = radius_graph_pbc(pos, cell[0], 4.5)
        out = energy_and_forces(model, pos, Z, batch, src, dst, sh, cell)
        return out, src.numel()

    for _ in range(args.warmup):
        out, E = step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out, E = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    log(f"cfg4: N={N} E={E} step={dt * 1e3:.2f} ms energy={float(out['energy'][0]):.6f}")

    if args.no_kernel_timing:
        return {"metric": METRIC, "value": N / dt, "unit": "atom-steps/s", "ms_per_step": dt * 1e3}, model
    # the step's own layer-1 launches, timed inside real steps (HIP events on the launching stream around
    # each launch: same operands, same cache state as the timed steps above)
    from ictc_o3 import _timing
    _timing.enable()
    for _ in range(5):
        step()
    spans = _timing.collect()
    src, dst, sh = radius_graph_pbc(pos, cell[0], 4.5)
    kern, nbytes, G = layer_message_kernels(model, src, dst, N, pos, sh)
    # the layer-1 radial gates with their r tangents over the step's gate rows (standalone, for the log)
    kern["gates_tan"], nbytes["gates_tan"] = layer_gate_kernel(model, G)
    standalone = dict(kern)
    M = model.interactions[-1].spec().num_paths * 64
    for k, name in (("msg_fwd", "msg_fwd[222C64]"), ("msg_bwd_tan", "msg_bwd_tan[222C64]"),
                    ("gates_tan", f"gates_tan[M{M}]")):
        if spans.get(name):
            kern[k] = sum(spans[name]) / len(spans[name]) * 1e-3
            log(f"  in-step {k}: {kern[k] * 1e6:.1f} us over {len(spans[name])} launches "
                f"(standalone {standalone[k] * 1e6:.1f} us)")
        else:
            raise RuntimeError(f"no in-step launches of {name} were recorded")
    # the step's own layer-1 kernels (energy + forces: radial gates with tangents, message forward,
    # gate-tangent adjoint); the other adjoint forms are timed for reference only
    in_step = [k for k in ("gates_tan", "msg_fwd", "msg_bwd_tan") if k in kern]
    dom = max(in_step, key=kern.get)   # the step's kernel with the largest time
    # Algorithmic bytes per the per-unit figure of the message kernels: per edge, its gate row
    # (P*C*4 B), harmonics, ids and mask, plus the node rows once (an edge list with one gate row per
    # edge, the layout the reference's message kernels read).  The step shares each gate row between
    # an edge and its reverse; `frac_shared_gate_rows` counts each of the G shared rows once instead.
    # The gate kernel computes and writes G rows, so its unit is the shared row either way.
    per_unit = message_bytes(N, E, 64, 9, 9, 11, 35)
    per_unit["gates_tan"] = nbytes["gates_tan"]
    achieved = per_unit[dom] / kern[dom] / 1e9
    result = {
        "metric": METRIC,
        "value": N / dt, "unit": "atom-steps/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": dt * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded jittered FCC positions, uniform species, random-init weights)",
        "config": {"workload": "cfg4: MACE-ICTC E+F, 131072 atoms FCC 32^3 at 0.1/A^3 +-0.3 A, rc 4.5 A, "
                               "C64 lmax2, 2 interactions, correlation 3, 8 Bessel, neighbour list rebuilt each step",
                   "atoms": N, "edges": E, "gate_rows": G, "channels": 64, "lmax": 2,
                   "tp_edges_per_s": 2 * E / dt,
                   "kernel_us_layer1": {k: round(t * 1e6, 2) for k, t in kern.items()},
                   "kernel_us_layer1_standalone": {k: round(t * 1e6, 2) for k, t in standalone.items()},
                   "kernel_algorithmic_MB_layer1": {k: round(v / 1e6, 2) for k, v in nbytes.items()}},
        "roofline": {"bound": "hbm", "kernel": f"{dom} (layer 1, P11 C64)", "timing": "in-step launches",
                     "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": MEASURED_TRAFFIC.get((dom, N, E, 64)),
                     "algorithmic_GB": round(per_unit[dom] / 1e9, 3),
                     "frac_shared_gate_rows": nbytes[dom] / kern[dom] / 1e9 / HBM_PEAK_GBS},
        # every layer-1 kernel of the step, largest first (the first is the roofline kernel above)
        "roofline_kernels": [{"kernel": k, "time_us": round(kern[k] * 1e6, 1),
                              "algorithmic_GB": round(per_unit[k] / 1e9, 3),
                              "achieved": per_unit[k] / kern[k] / 1e9,
                              "frac": per_unit[k] / kern[k] / 1e9 / HBM_PEAK_GBS,
                              "traffic": MEASURED_TRAFFIC.get((k, N, E, 64)),
                              "frac_shared_gate_rows": nbytes[k] / kern[k] / 1e9 / HBM_PEAK_GBS}
                             for k in sorted(in_step, key=kern.get, reverse=True)],
    }
    return result, model


def layer_gate_kernel(model, E, reps=5):
    """HIP-event time of the layer-1 radial gates with their r tangents (ictc_radial_gates_tangent_fwd: W4
    split, then the MLP, both projections and both stores) and its algorithmic bytes: the edge lengths read,
    gates and tangents [E, M] written (weights: under 0.3 MB).  E = the gate rows of the step (one per
    undirected edge pair)."""
    import torch
    from ictc_o3.ops.radial_mlp import radial_gates_tangent
    inter = model.interactions[-1]
    dev = next(model.parameters()).device
    lin = [m.weight for m in inter.fc if isinstance(m, torch.nn.Linear)]
    M = lin[-1].shape[0]
    r = torch.rand(E, device=dev, generator=torch.Generator(device=dev).manual_seed(4)) * 3 + 1.5
    t = time_launches(lambda: radial_gates_tangent(r, lin, model.max_radius, model.polynomial_cutoff_p,
                                                   1.6791767923989418), reps, torch.cuda.current_stream(dev))
    log(f"  last-layer gates_tan: {t * 1e6:.1f} us  {(E * 4 + 2 * E * M * 4) / t / 1e9:.0f} GB/s")
    return t, E * 4 + 2 * E * M * 4


def layer_message_kernels(model, src, dst, N, pos, shifts=None, pair=True, reps=5):
    """Live HIP-event timing of the last interaction's message kernels (fwd, bwd_edge, bwd_x) at the run's shapes,
    visiting rows in the spatial order the model uses (and, for the log only, in index order).  The step's own
    forms (msg_fwd, msg_bwd_tan) read the gates shared by each edge and its reverse, as the model does; the
    other adjoint forms (timed for reference) read one gate row per edge.  pair=False (the second-order
    training route, which keeps per-edge gates) times every form on per-edge rows.  Returns (times, bytes,
    gate rows)."""
    import torch
    from ictc_o3.ops import tensor_product as tpo
    dev = src.device
    stream = torch.cuda.current_stream(dev)
    topo = tpo.Topology(src, dst, N, positions=pos)
    if pair:
        topo.pair_edges(shifts)
    rows = topo.gate_rows
    G = src.numel() if rows is None else topo.gate_reps.numel()
    inter = model.interactions[-1]
    spec = inter.spec()
    C = spec.channels
    NX, NY = (spec.li + 1) ** 2, (spec.le + 1) ** 2
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(N, NX * C, device=dev, generator=g)
    Y = torch.randn(src.numel(), NY, device=dev, generator=g)
    with torch.no_grad():
        r = torch.rand(src.numel(), device=dev, generator=g) * 3 + 1.5
        gates = inter.fc(model.radial_embedding(r))
    shared = gates[:G]
    go = torch.randn(N, spec.out_components * C, device=dev, generator=g)
    t_fwd = time_launches(lambda: tpo._msg_fwd_raw(spec, topo, x, Y, shared, None, rows), reps, stream)
    t_bwd_e = time_launches(lambda: tpo._msg_bwd_raw(spec, topo, x, Y, gates, None, go, (False, True, True)), reps,
                            stream)
    topo.by_src
    t_bwd_x = time_launches(lambda: tpo._msg_bwd_raw(spec, topo, x, Y, gates, None, go, (True, False, False)), reps,
                            stream)
    # the model's backward asks for dx, dsh and dg together: one fused source-owned kernel where the library fuses
    t_bwd = time_launches(lambda: tpo._msg_bwd_raw(spec, topo, x, Y, gates, None, go, (True, True, True)), reps,
                          stream)
    nbytes = message_bytes(N, src.numel(), C, NX, NY, spec.num_paths, spec.out_components)
    paired = message_bytes(N, src.numel(), C, NX, NY, spec.num_paths, spec.out_components, None if rows is None else G)
    nbytes["msg_fwd"], nbytes["msg_bwd_tan"] = paired["msg_fwd"], paired["msg_bwd_tan"]
    kern = {"msg_fwd": t_fwd, "msg_bwd_edge": t_bwd_e, "msg_bwd_x": t_bwd_x}
    if t_bwd < 0.9 * (t_bwd_e + t_bwd_x):   # fused (one launch); otherwise it is the two kernels above
        kern["msg_bwd"] = t_bwd
        # energy + forces (the model's forces_only route): dx, dsh and dr = sum dg * d gates / dr
        gdot = torch.randn_like(shared)
        kern["msg_bwd_tan"] = time_launches(
            lambda: tpo._msg_bwd_tangent_raw(spec, topo, x, Y, shared, gdot, None, go, (True, True), rows), reps,
            stream)
        del gdot
    else:
        log(f"  last-layer full adjoint {t_bwd * 1e6:.1f} us: the two kernels above (not fused at this shape)")
    for k, t in kern.items():
        log(f"  last-layer {k}: {t * 1e6:.1f} us  {nbytes[k] / t / 1e9:.0f} GB/s ({nbytes[k] / 1e6:.1f} MB)")
    nbytes = {k: v for k, v in nbytes.items() if k in kern}
    plain = tpo.Topology(src, dst, N)
    plain.by_src
    t_idx = [time_launches(lambda: tpo._msg_fwd_raw(spec, plain, x, Y, gates, None), reps, stream),
             time_launches(lambda: tpo._msg_bwd_raw(spec, plain, x, Y, gates, None, go, (False, True, True)), reps,
                           stream),
             time_launches(lambda: tpo._msg_bwd_raw(spec, plain, x, Y, gates, None, go, (True, False, False)), reps,
                           stream)]
    log("  index-order rows (one gate row per edge): " + ", ".join(f"{k} {t * 1e6:.1f} us"
                                                                 for k, t in zip(kern, t_idx)))
    return kern, nbytes, G


def run_cfg1(args):
    """EdgeTensorProduct fwd+bwd, C32 L2 ir_mul, E=257 (launch-latency bound) plus the same shapes at E=2^20."""
    import torch
    from ictc_o3 import EdgeTensorProduct, direction_harmonics
    from ictc_o3.ops import tensor_product as tpo
    dev = torch.device("cuda:0")
    C, E = 32, 257
    op = EdgeTensorProduct.create(input_lmax=2, edge_lmax=2, output_lmax=2, channels=C, device=dev)
    torch.manual_seed(0)
    blocks = {l: torch.randn(E, C, 2 * l + 1) for l in range(3)}
    v = torch.randn(E, 3)
    gates = torch.randn(E, op.gate_width)
    x = op.pack_input({l: b.to(dev) for l, b in blocks.items()}).requires_grad_(True)
    sh = torch.cat(direction_harmonics((v / v.norm(dim=1, keepdim=True)).to(dev), 2), -1).requires_grad_(True)
    g = gates.to(dev).requires_grad_(True)

    def step():
        out = op(x, sh, g)
        (out * out).mean().backward()

    for _ in range(max(args.warmup, 3)):
        step()
    torch.cuda.synchronize()
    steps = max(args.steps, 200)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    log(f"cfg1: E={E} step={dt * 1e6:.1f} us")

    # kernel roofline at E = 2^20 (same shapes)
    spec = op._prepare()
    Eb = 1 << 20
    gb = torch.Generator(device=dev).manual_seed(1)
    xb = torch.randn(Eb, x.shape[1], device=dev, generator=gb)
    shb = torch.randn(Eb, 9, device=dev, generator=gb)
    gbt = torch.randn(Eb, op.gate_width, device=dev, generator=gb)
    gob = torch.randn(Eb, op.output_width, device=dev, generator=gb)
    stream = torch.cuda.current_stream(dev)
    t_f = time_launches(lambda: tpo._edge_fwd_raw(spec, xb, shb, gbt), 20, stream)
    t_b = time_launches(lambda: tpo._edge_bwd_raw(spec, xb, shb, gbt, gob, (True, True, True)), 20, stream)
    per_edge_f = (x.shape[1] + 9 + op.gate_width + op.output_width) * 4
    per_edge_b = (x.shape[1] + 9 + op.gate_width + op.output_width) * 4 + (x.shape[1] + 9 + op.gate_width) * 4
    ach_f, ach_b = Eb * per_edge_f / t_f / 1e9, Eb * per_edge_b / t_b / 1e9
    log(f"  E=2^20 tp_fwd {t_f * 1e6:.1f} us {ach_f:.0f} GB/s; tp_bwd {t_b * 1e6:.1f} us {ach_b:.0f} GB/s")
    result = {
        "metric": METRIC, "value": E / dt, "unit": "edges/s", "n_gpus": 1, "steps": steps,
        "warmup": max(args.warmup, 3), "ms_per_step": dt * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic (seeded N(0,1) blocks, directions, gates)",
        "config": {"workload": "cfg1: EdgeTensorProduct fwd+bwd (loss mean(out^2)), C32 lmax2 ir_mul, E=257; "
                               "kernel roofline at the same shapes with E=2^20",
                   "edges": E, "channels": C, "lmax": 2, "us_per_step": dt * 1e6,
                   "kernel_us_E2^20": {"tp_fwd": round(t_f * 1e6, 2), "tp_bwd": round(t_b * 1e6, 2)},
                   "algorithmic_bytes_per_edge": {"tp_fwd": per_edge_f, "tp_bwd": per_edge_b},
                   "tp_bwd_frac": ach_b / HBM_PEAK_GBS},
        "roofline": {"bound": "hbm", "kernel": "tp_fwd (E=2^20, C32, P11)", "achieved": ach_f,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": ach_f / HBM_PEAK_GBS, "traffic": None},
    }
    return result, (blocks, v, gates, C)


def cpu_baseline_tp(data, budget_s=15.0):
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ictc_oracle as orc
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    blocks, v, gates, C = data
    E = v.shape[0]
    feats = torch.cat([blocks[l].transpose(1, 2).reshape(E, -1) for l in range(3)], -1)
    sh = torch.cat(orc.direction_harmonics((v / v.norm(dim=1, keepdim=True)).double(), 2), -1).float()

    def step():
        a = feats.clone().requires_grad_(True)
        b = sh.clone().requires_grad_(True)
        c = gates.clone().requires_grad_(True)
        out = orc.edge_tp_packed(a, b, c, 2, 2, 2, C)
        (out * out).mean().backward()
    med = time_cpu(step)
    return cpu_record(E / med, "edges/s", "cfg1 in full (E=257, C32), oracle FP32 torch eager fwd+bwd")


def run_cfg3(args):
    """Symmetric contraction corr 3, fwd + dx: 32,768 nodes, C64, lmax 2 -> L<=1, 4 species."""
    import torch
    from ictc_o3 import create_symmetric_contraction
    from ictc_o3.ops import symmetric_contraction as sco
    dev = torch.device("cuda:0")
    N, C, S = 32768, 64, 4
    torch.manual_seed(11)
    mod = create_symmetric_contraction(num_elements=S, lmax=2, target_lmax=1, channels=C, correlation=3,
                                       device=dev)
    for p in mod.parameters():
        p.requires_grad_(False)
    g = torch.Generator(device=dev).manual_seed(12)
    x = torch.randn(N, 9 * C, device=dev, generator=g).requires_grad_(True)
    species = torch.randint(0, S, (N,), device=dev, generator=g)
    go = torch.randn(N, 4 * C, device=dev, generator=g)

    def step():   # SC forward + feature adjoint (dx returned, not accumulated into x.grad)
        out = mod.contract(x, species)
        return torch.autograd.grad(out, x, go)

    for _ in range(max(args.warmup, 3)):
        step()
    torch.cuda.synchronize()
    steps = max(args.steps, 50)
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    spec = mod.spec()
    ws = mod.slot_weights()
    stream = torch.cuda.current_stream(dev)
    xd = x.detach()
    t_f = time_launches(lambda: sco._fwd_raw(spec, xd, species, ws), 50, stream)
    t_x = time_launches(lambda: sco._dx_raw(spec, xd, species, ws, go), 50, stream)
    fwd_bytes = N * 9 * C * 4 + N * 8 + N * 4 * C * 4
    dx_bytes = N * 9 * C * 4 + N * 4 * C * 4 + N * 8 + N * 9 * C * 4
    terms = sco.term_count(spec)
    fwd_flops = 2.0 * terms * N * C
    ach_f = fwd_bytes / t_f / 1e9
    log(f"cfg3: step {dt * 1e6:.1f} us; sc_fwd {t_f * 1e6:.1f} us {ach_f:.0f} GB/s "
        f"{fwd_flops / t_f / 1e12:.1f} TFLOP/s; sc_dx {t_x * 1e6:.1f} us {dx_bytes / t_x / 1e9:.0f} GB/s")
    result = {
        "metric": METRIC, "value": N / dt, "unit": "node-steps/s", "n_gpus": 1, "steps": steps,
        "warmup": max(args.warmup, 3), "ms_per_step": dt * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic (seeded N(0,1) features, uniform species)",
        "config": {"workload": "cfg3: symmetric contraction corr 3 fwd + dx, 32768 nodes, C64, lmax2 -> L<=1, "
                               "4 species", "nodes": N, "channels": C,
                   "kernel_us": {"sc_fwd": round(t_f * 1e6, 2), "sc_dx": round(t_x * 1e6, 2)},
                   "algorithmic_bytes": {"sc_fwd": fwd_bytes, "sc_dx": dx_bytes},
                   "fwd_flops": fwd_flops, "fwd_flops_per_byte": fwd_flops / fwd_bytes,
                   "fwd_fp32_frac": fwd_flops / t_f / 1e12 / FP32_PEAK_TFLOPS,
                   "dx_hbm_frac": dx_bytes / t_x / 1e9 / HBM_PEAK_GBS},
        "roofline": {"bound": "hbm", "kernel": "sc_fwd (corr 3, C64, L2 -> L<=1)", "achieved": ach_f,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": ach_f / HBM_PEAK_GBS, "traffic": None},
    }
    return result, (mod, x.detach().cpu(), species.cpu(), go.cpu())


def cpu_baseline_sc(data, budget_s=15.0):
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import sc_oracle as so
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    mod, x, species, go = data
    take = 2048
    W = {L: {nu: c.weight_for(nu).detach().float().cpu() for nu in range(1, c.correlation + 1)}
         for L, c in enumerate(mod.symmetric_contractions.contractions)}
    C = mod.channels
    xs = x[:take].reshape(take, 9, C).transpose(1, 2).contiguous()
    sp = species[:take]
    gos = go[:take]

    def step():
        a = xs.clone().requires_grad_(True)
        out = so.symmetric_contraction(a, sp, W, 2, 1, 3)
        out.backward(gos[:, :out.shape[1]])
    med = time_cpu(step)
    return cpu_record(take / med, "node-steps/s", f"first {take} nodes of cfg3, oracle FP32 torch eager SC fwd + dx")


def batched_cells(cells, n, density, jitter, seed, species, cutoff, device):
    """`cells` independent periodic FCC n^3 cells as one batch with per-cell neighbour lists (a data set)."""
    import torch
    from mace_ictc.hp import radius_graph_pbc
    P, Zs, B, S, D, SH, cellv = [], [], [], [], [], [], []
    off = 0
    for b in range(cells):
        pos, _, cell, _ = fcc_system(n, density, jitter, seed + b, 3, device)
        g = torch.Generator().manual_seed(seed + 1000 + b)
        Z = torch.tensor(species)[torch.randint(0, len(species), (pos.shape[0],), generator=g)].to(device)
        src, dst, sh = radius_graph_pbc(pos, cell[0], cutoff)
        P.append(pos), Zs.append(Z), B.append(torch.full((pos.shape[0],), b, dtype=torch.long, device=device))
        S.append(src + off), D.append(dst + off), SH.append(sh), cellv.append(cell)
        off += pos.shape[0]
    cat = torch.cat
    return cat(P), cat(Zs), cat(B), cat(S), cat(D), cat(SH), cat(cellv)


def run_cfg5(args):
    """Force-loss training step: C128, edge L3, hidden L2, 10 species, 32 cells x 256 atoms, cutoff 5 A."""
    import torch
    from mace_ictc.hp import create_model, energy_and_forces
    from ictc_o3.ops import tensor_product as tpo
    dev = torch.device("cuda:0")
    torch.manual_seed(55)
    species = tuple(range(1, 11))
    model = create_model(channels=128, lmax=2, edge_lmax=3, num_interactions=2, correlation=3,
                         atomic_numbers=species, cutoff=5.0, device=dev)
    pos, Z, batch, src, dst, sh, cell = batched_cells(32, 4, 0.1, 0.3, 500, species, 5.0, dev)
    N, E, B = pos.shape[0], src.numel(), cell.shape[0]
    g = torch.Generator(device=dev).manual_seed(56)
    E_t = torch.randn(B, device=dev, generator=g) * math.sqrt(256)
    F_t = torch.randn(N, 3, device=dev, generator=g) * 0.5
    topo = tpo.Topology(src, dst, N)   # 32 graphs: index order (atoms contiguous per graph)
    opt = torch.optim.Adam(model.parameters(), lr=1e-4)

    def step():
        opt.zero_grad(set_to_none=True)
        out = energy_and_forces(model, pos, Z, batch, src, dst, sh, cell, training=True, topology=topo)
        loss = ((out["energy"] - E_t) ** 2).mean() + ((out["forces"] - F_t) ** 2).mean()
        loss.backward()
        opt.step()
        return loss

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    log(f"cfg5: N={N} E={E} step={dt * 1e3:.2f} ms loss={float(loss.detach()):.4f}")
    if args.no_kernel_timing:
        return {"metric": METRIC, "value": N / dt, "unit": "atom-steps/s", "ms_per_step": dt * 1e3}, model
    kern, nbytes, _ = layer_message_kernels(model, src, dst, N, None, pair=False, reps=10)
    dom = max(kern, key=kern.get)   # the layer-1 message kernel with the largest time
    achieved = nbytes[dom] / kern[dom] / 1e9
    result = {
        "metric": METRIC, "value": N / dt, "unit": "atom-steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": dt * 1e3, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (32 seeded jittered FCC 4^3 cells, uniform species 1..10, N(0,1) per-atom energy and "
                "N(0,0.5) force targets, random-init weights; neighbour lists built once like a data set)",
        "config": {"workload": "cfg5: force-loss training step (E+F MSE backward through mixed second "
                               "derivatives + Adam), C128, edge L3, hidden L2, 2 interactions, corr 3, rc 5 A, "
                               "10 species, 32 cells x 256 atoms",
                   "atoms": N, "edges": E, "channels": 128,
                   "kernel_us_layer1": {k: round(t * 1e6, 2) for k, t in kern.items()},
                   "kernel_algorithmic_MB_layer1": {k: round(v / 1e6, 2) for k, v in nbytes.items()}},
        "roofline": {"bound": "hbm", "kernel": f"{dom} (layer 1, P17 C128)",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "traffic": None},
    }
    return result, model


def cpu_baseline_train(model, budget_s=25.0):
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import model_oracle as mo
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    species = tuple(range(1, 11))
    pos, Z, batch, src, dst, sh, cell = batched_cells(1, 4, 0.1, 0.3, 500, species, 5.0, "cpu")
    sd = {k: v.detach().float().cpu().clone() for k, v in model.state_dict().items()}
    names = [k for k, p in model.named_parameters() if p.requires_grad]
    cfg = mo.config_of(model)
    E_t = torch.zeros(1)
    F_t = torch.zeros_like(pos)

    def step():
        for k in names:
            sd[k] = sd[k].detach().requires_grad_(True)
        p = pos.clone().requires_grad_(True)
        atomic = mo.forward(sd, cfg, p, Z, batch, src, dst, sh, cell, dtype=torch.float32)
        En = atomic.sum().reshape(1)
        (gp,) = torch.autograd.grad(En.sum(), p, create_graph=True)
        loss = ((En - E_t) ** 2).mean() + ((-gp - F_t) ** 2).mean()
        torch.autograd.grad(loss, [sd[k] for k in names], allow_unused=True)
    med = time_cpu(step)
    return cpu_record(pos.shape[0] / med, "atom-steps/s", f"one 256-atom cell of cfg5 (E={src.numel()}), oracle "
                      "FP32 torch eager E+F+force-loss parameter gradients")



def run_layers(args):
    """Fused against materialised radial gates, per cfg4 layer: one message forward + energy-and-forces adjoint
    (features, harmonics, edge lengths) including the layer's radial gates, HIP-event timed (ms per pass)."""
    import torch
    from mace_ictc.hp import create_model, radius_graph_pbc
    from ictc_o3.ops import tensor_product as tpo
    dev = torch.device("cuda:0")
    torch.manual_seed(2024)
    model = create_model(channels=64, lmax=2, num_interactions=2, correlation=3, atomic_numbers=(1, 6, 8),
                         cutoff=4.5, avg_num_neighbors=42.0, device=dev)
    pos, Z, cell, a = fcc_system(32, 0.1, 0.3, 1234, 3, dev)
    N = pos.shape[0]
    src, dst, _ = radius_graph_pbc(pos, cell[0], 4.5)
    E = src.numel()
    topo = tpo.Topology(src, dst, N, positions=pos)
    topo.by_src
    g = torch.Generator(device=dev).manual_seed(3)
    r = (torch.rand(E, device=dev, generator=g) * 3 + 1.5).requires_grad_(True)
    Y = torch.randn(E, 9, device=dev, generator=g).requires_grad_(True)
    cfg = (4.5, 5, 1.6791767923989418)
    stream = torch.cuda.current_stream(dev)
    out = {}
    for li, inter in ((0, model.interactions[0]), (2, model.interactions[1])):
        spec = inter.spec()
        x = torch.randn(N, (li + 1) ** 2 * 64, device=dev, generator=g).requires_grad_(li > 0)
        go = torch.randn(N, spec.out_components * 64, device=dev, generator=g)
        wrt = [t for t in (x, Y, r) if t.requires_grad]
        for mode in ("always", "never"):
            tpo.FUSED_GATES = mode

            def step():
                o = tpo.radial_message(x, Y, r, inter.fc, spec, topo, None, cfg)
                torch.autograd.grad(o, wrt, go)
            t = time_launches(step, args.steps, stream)
            out[f"layer{li}_{'fused' if mode == 'always' else 'materialised'}_ms"] = round(t * 1e3, 3)
            log(f"  input degree {li}, {mode}: {t * 1e3:.2f} ms")
    tpo.FUSED_GATES = "auto"
    print(json.dumps({"workload": "cfg4 layers: radial gates + message forward + energy-and-forces adjoint",
                      "atoms": N, "edges": E, **out}), flush=True)
    return None, None


def run_probe(args):
    """Counter-collection workload: the cfg4 layer-1 message kernels and gate kernels, then a 1 GiB copy.

    Run under ``rocprofv3 --pmc FETCH_SIZE`` (and separately ``WRITE_SIZE``): the
    copy (1 GiB read, 1 GiB written) calibrates the counters, the message
    kernels give HBM bytes per dispatch.  Prints nothing but a short log.
    """
    import torch
    from mace_ictc.hp import create_model, radius_graph_pbc
    from ictc_o3.ops import tensor_product as tpo
    dev = torch.device("cuda:0")
    torch.manual_seed(2024)
    model = create_model(channels=64, lmax=2, num_interactions=2, correlation=3, atomic_numbers=(1, 6, 8),
                         cutoff=4.5, avg_num_neighbors=42.0, device=dev)
    pos, Z, cell, a = fcc_system(32, 0.1, 0.3, 1234, 3, dev)
    N = pos.shape[0]
    src, dst, sh = radius_graph_pbc(pos, cell[0], 4.5)
    topo = tpo.Topology(src, dst, N, positions=pos)
    inter = model.interactions[-1]
    spec = inter.spec()
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(N, 9 * 64, device=dev, generator=g)
    Y = torch.randn(src.numel(), 9, device=dev, generator=g)
    with torch.no_grad():
        r = torch.rand(src.numel(), device=dev, generator=g) * 3 + 1.5
        gates = inter.fc(model.radial_embedding(r))
    go = torch.randn(N, spec.out_components * 64, device=dev, generator=g)
    topo.by_src
    for _ in range(args.steps):
        tpo._msg_fwd_raw(spec, topo, x, Y, gates, None)
        tpo._msg_bwd_raw(spec, topo, x, Y, gates, None, go, (False, True, True))
        tpo._msg_bwd_raw(spec, topo, x, Y, gates, None, go, (True, False, False))
        tpo._msg_bwd_raw(spec, topo, x, Y, gates, None, go, (True, True, True))
    # the energy + forces step's forms: gates (and gdot) shared by each edge and its reverse
    paired = tpo.Topology(src, dst, N, positions=pos)
    paired.pair_edges(sh)
    G = paired.gate_reps.numel() if paired.gate_rows is not None else src.numel()
    shared = gates[:G]
    gdot = torch.randn_like(shared)
    paired.by_src
    for _ in range(args.steps):
        tpo._msg_fwd_raw(spec, paired, x, Y, shared, None, paired.gate_rows)
        tpo._msg_bwd_tangent_raw(spec, paired, x, Y, shared, gdot, None, go, (True, True), paired.gate_rows)
    del gdot
    from ictc_o3.ops.radial_mlp import gate_projection_adjoint, radial_gates, radial_gates_tangent
    lin = [m for m in inter.fc if isinstance(m, torch.nn.Linear)]
    with torch.no_grad():
        for _ in range(args.steps):
            radial_gates(r, inter.fc, model.max_radius, model.polynomial_cutoff_p, 1.6791767923989418)
            gate_projection_adjoint(gates, lin[-1].weight.detach())
            radial_gates_tangent(r[:G], [m.weight for m in lin], model.max_radius, model.polynomial_cutoff_p,
                                 1.6791767923989418)
    a = torch.empty(1 << 28, device=dev)
    b = torch.randn(1 << 28, device=dev)
    for _ in range(args.steps):
        a.copy_(b)
    torch.cuda.synchronize()
    nbytes = message_bytes(N, src.numel(), 64, 9, 9, spec.num_paths, spec.out_components)
    pb = message_bytes(N, src.numel(), 64, 9, 9, spec.num_paths, spec.out_components, G)
    log(f"probe: N={N} E={src.numel()} gate rows {G} algorithmic bytes {nbytes}; paired msg_fwd "
        f"{pb['msg_fwd']} msg_bwd_tan {pb['msg_bwd_tan']}; copy {4 << 28} bytes each way")
    return None, None



def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="cfg4", choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5", "probe", "layers"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-timing", action="store_true",
                    help="skip the per-kernel HIP-event timings after the timed steps (clean profiles of the step)")
    ap.add_argument("--no-cfg5", action="store_true", help="cfg4 only: skip the cfg5 training-step line")
    ap.add_argument("--cfg5-steps", type=int, default=10)
    ap.add_argument("--cfg5-warmup", type=int, default=3)
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one-GPU hot path by design); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    runners = {"cfg1": (run_cfg1, cpu_baseline_tp), "cfg2": (run_cfg2, cpu_baseline),
               "cfg3": (run_cfg3, cpu_baseline_sc), "cfg4": (run_cfg4, cpu_baseline_model),
               "cfg5": (run_cfg5, cpu_baseline_train)}
    if args.workload == "probe":
        run_probe(args)
        return
    if args.workload == "layers":
        run_layers(args)
        return
    run, cpu = runners[args.workload]
    result, data = run(args)
    if args.workload == "cfg4" and not args.no_cfg5:
        # the force-loss training step timed in the same run, beside the headline
        sub = argparse.Namespace(**{**vars(args), "no_kernel_timing": True, "steps": args.cfg5_steps,
                                    "warmup": args.cfg5_warmup})
        r5, _ = run_cfg5(sub)
        result["cfg5"] = {"workload": "cfg5: force-loss training step (E+F MSE backward through mixed second "
                                      "derivatives + Adam), C128, edge L3, hidden L2, 10 species, 32 cells x 256 "
                                      "atoms, rc 5 A",
                          "metric": "atom-steps/s", "value": r5["value"], "ms_per_step": r5["ms_per_step"],
                          "steps": sub.steps, "warmup": sub.warmup}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu(data)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
