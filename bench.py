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

Roofline: the dominant message kernel is timed live with HIP events on the
stream it runs on (torch's current stream), averaged over repeated launches;
its algorithmic bytes (compulsory traffic: each operand read once, each output
written once, index arrays included, gathers not counted) / time vs 8 TB/s.

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


def message_bytes(N, E, C, NX, NY, P, NO):
    idx = E * 8 + (N + 2) * 4 + E * 4
    fwd = N * NX * C * 4 + E * NY * 4 + E * P * C * 4 + idx + N * NO * C * 4
    bwd_edge = N * NO * C * 4 + N * NX * C * 4 + E * NY * 4 + E * P * C * 4 + idx + E * NY * 4 + E * P * C * 4
    bwd_x = N * NO * C * 4 + E * NY * 4 + E * P * C * 4 + idx + N * NX * C * 4
    return {"msg_fwd": fwd, "msg_bwd_edge": bwd_edge, "msg_bwd_x": bwd_x}


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
    step()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 and (time.perf_counter() < t_end or len(times) < 1):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"value": take / med, "unit": "edges/s", "cores": threads, "kind": "port",
            "sample": f"message fwd+bwd (oracle FP32 torch eager) on the first {take} receiver-sorted edges "
                      f"of the cfg2 graph, median of {len(times)} runs, {torch.get_num_threads()} threads"}


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
    topo = tpo.Topology(src, dst, N)

    def mlp(h):
        for k, W in enumerate(Ws):
            h = torch.nn.functional.linear(h, W)
            if k < len(Ws) - 1:
                h = torch.nn.functional.silu(h) * 1.6791767923989418
        return h

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
    kern = {"msg_fwd": t_fwd, "msg_bwd_edge": t_bwd_e, "msg_bwd_x": t_bwd_x}
    for k, t in kern.items():
        log(f"  {k}: {t * 1e6:.1f} us  {nbytes[k] / t / 1e9:.0f} GB/s ({nbytes[k] / 1e6:.1f} MB)")
    dom = max(kern, key=kern.get)
    achieved = nbytes[dom] / kern[dom] / 1e9
    result = {
        "metric": "atom-steps/s (E+F, 1 GPU) C64/lmax2 MACE; TP edges/s & % HBM roofline",
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
    step()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 and (time.perf_counter() < t_end or not times):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = sorted(times)[len(times) // 2]
    return {"value": pos.shape[0] / med, "unit": "atom-steps/s", "cores": threads, "kind": "port",
            "sample": f"cfg4 model (same weights) E+F incl. neighbour list on a 2,048-atom FCC 8^3 sample "
                      f"(E={src.numel()}), oracle FP32 torch eager, median of {len(times)} steps, "
                      f"{torch.get_num_threads()} threads"}


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

    # live timing of the dominant message kernels at layer-1 shapes (P11, C64)
    stream = torch.cuda.current_stream(dev)
    src, dst, sh = radius_graph_pbc(pos, cell[0], 4.5)
    topo = tpo.Topology(src, dst, N)
    inter = model.interactions[1]
    spec = inter.spec()
    g = torch.Generator(device=dev).manual_seed(3)
    x = torch.randn(N, 9 * 64, device=dev, generator=g)
    Y = torch.randn(E, 9, device=dev, generator=g)
    with torch.no_grad():
        r = torch.rand(E, device=dev, generator=g) * 3 + 1.5
        gates = inter.fc(model.radial_embedding(r))
    go = torch.randn(N, spec.out_components * 64, device=dev, generator=g)
    t_fwd = time_launches(lambda: tpo._msg_fwd_raw(spec, topo, x, Y, gates, None), 5, stream)
    t_bwd_e = time_launches(lambda: tpo._msg_bwd_raw(spec, topo, x, Y, gates, None, go, (False, True, True)), 5,
                            stream)
    topo.by_src
    t_bwd_x = time_launches(lambda: tpo._msg_bwd_raw(spec, topo, x, Y, gates, None, go, (True, False, False)), 5,
                            stream)
    nbytes = message_bytes(N, E, 64, 9, 9, spec.num_paths, spec.out_components)
    kern = {"msg_fwd": t_fwd, "msg_bwd_edge": t_bwd_e, "msg_bwd_x": t_bwd_x}
    for k, t in kern.items():
        log(f"  layer-1 {k}: {t * 1e6:.1f} us  {nbytes[k] / t / 1e9:.0f} GB/s ({nbytes[k] / 1e6:.1f} MB)")
    dom = "msg_fwd"
    achieved = nbytes[dom] / kern[dom] / 1e9
    result = {
        "metric": "atom-steps/s (E+F, 1 GPU) C64/lmax2 MACE; TP edges/s & % HBM roofline",
        "value": N / dt, "unit": "atom-steps/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": dt * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded jittered FCC positions, uniform species, random-init weights)",
        "config": {"workload": "cfg4: MACE-ICTC E+F, 131072 atoms FCC 32^3 at 0.1/A^3 +-0.3 A, rc 4.5 A, "
                               "C64 lmax2, 2 interactions, correlation 3, 8 Bessel, neighbour list rebuilt each step",
                   "atoms": N, "edges": E, "channels": 64, "lmax": 2,
                   "tp_edges_per_s": 2 * E / dt,
                   "kernel_us_layer1": {k: round(t * 1e6, 2) for k, t in kern.items()},
                   "kernel_algorithmic_MB_layer1": {k: round(v / 1e6, 2) for k, v in nbytes.items()}},
        "roofline": {"bound": "hbm", "kernel": "msg_fwd (layer 1, P11 C64)", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None},
    }
    return result, model


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="cfg4", choices=["cfg4", "cfg2"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one-GPU hot path by design); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.workload == "cfg4":
        result, model = run_cfg4(args)
        if not args.no_cpu_baseline:
            result["cpu_baseline"] = cpu_baseline_model(model)
    else:
        result, data = run_cfg2(args)
        if not args.no_cpu_baseline:
            result["cpu_baseline"] = cpu_baseline(data)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
