"""Periodic radius graph on the GPU (receiver-sorted), for MD-style steps.

The reference delegates neighbour search to ASE / matscipy / torch_cluster
(examples/predict.py:62, data/preprocessing.py:11, utils/graph_utils.py:217-297).
This builds the same directed edge list on the device: a cell list when every
periodic direction holds >= 3 cells (the HIP kernels ictc_neighbors_count /
_fill for FP32 ROCm positions, the torch formulation below for CPU tensors,
both emitting the same edges in the same order), else an image-enumerating
all-pairs search.
Edge convention (backbone.py:940-944): vec = pos[dst] - pos[src] + shift @ cell,
with every pair at distance < cutoff (self-images included when in range).
Edges come out sorted by receiver (dst).
"""
from __future__ import annotations

import itertools
import math
import weakref

import torch


def _ncell(cell_cpu: torch.Tensor, cutoff: float):
    c = cell_cpu.double()
    vol = abs(float(torch.det(c)))
    widths = [vol / float(torch.linalg.cross(c[(d + 1) % 3], c[(d + 2) % 3]).norm()) for d in range(3)]
    return [max(1, int(math.floor(w / cutoff))) for w in widths], widths


_fill_capacity = {}   # (atoms, cells, cutoff, device) -> edge capacity for the next fill (from the last count)


def _cell_list_hip(pos, cell_cpu, cutoff, ncell):
    """The HIP cell list.  The edge count must reach the host to size the edge arrays; where an earlier call
    on the same kind of system left a capacity estimate, the fill is launched into arrays of that capacity
    before the count is read (only the count's copy is waited for, the fill runs meanwhile), and the arrays
    are trimmed to the count; a count above the capacity refills arrays of the exact size."""
    import ctypes
    from ictc_o3 import _native as nat
    pos = pos.contiguous()
    N, dev = pos.shape[0], pos.device
    nc = (ctypes.c_int * 3)(*ncell)
    cellh = (ctypes.c_double * 9)(*cell_cpu.double().reshape(-1).tolist())
    ws_bytes = int(nat.lib().ictc_neighbors_workspace_bytes(N, nc))
    if ws_bytes < 0:
        raise ValueError("radius_graph_pbc: system too large for the int32 cell list")
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    count = torch.zeros(1, dtype=torch.int64, device=dev)
    stream = nat.stream_of(pos)
    nat.call("ictc_neighbors_count", nat.ptr(pos), N, cellh, float(cutoff), nc, nat.ptr(ws), ws_bytes,
             nat.ptr(count), stream)
    key = (N, tuple(ncell), float(cutoff), str(dev))
    cap = _fill_capacity.get(key, 0)
    E = -1
    if cap > 0:
        host = torch.empty(1, dtype=torch.int64, pin_memory=True)
        host.copy_(count, non_blocking=True)
        ready = torch.cuda.Event()
        ready.record(torch.cuda.current_stream(dev))
        src = torch.empty(cap, dtype=torch.int64, device=dev)
        dst = torch.empty(cap, dtype=torch.int64, device=dev)
        shifts = torch.empty(cap, 3, dtype=torch.float32, device=dev)
        nat.call("ictc_neighbors_fill_capacity", nat.ptr(pos), N, cellh, float(cutoff), nc, nat.ptr(ws), ws_bytes,
                 nat.ptr(src), nat.ptr(dst), nat.ptr(shifts), cap, stream)
        ready.synchronize()
        E = int(host[0])
        if E <= cap:
            src, dst, shifts = src[:E], dst[:E], shifts[:E]
    if not 0 <= E <= cap:
        if E < 0:
            E = int(count.item())
        src = torch.empty(E, dtype=torch.int64, device=dev)
        dst = torch.empty(E, dtype=torch.int64, device=dev)
        shifts = torch.empty(E, 3, dtype=torch.float32, device=dev)
        if E:
            nat.call("ictc_neighbors_fill", nat.ptr(pos), N, cellh, float(cutoff), nc, nat.ptr(ws), ws_bytes,
                     nat.ptr(src), nat.ptr(dst), nat.ptr(shifts), stream)
    if len(_fill_capacity) > 64:
        _fill_capacity.clear()
    _fill_capacity[key] = E + E // 32 + 1024   # room for the next step's fluctuation in the count
    from ictc_o3.ops.tensor_product import mark_receiver_sorted
    mark_receiver_sorted(dst, N)    # emitted receiver by receiver, ids in [0, N): Topology skips the sort
    return src, dst, shifts


_cell_seen = None   # (weakref to the cell's base tensor, view geometry + version, host copy)


def _host_cell(cell: torch.Tensor) -> torch.Tensor:
    """The cell on the host in float64.  A device cell costs a host sync per copy, which stalls the launch
    queue at every step of an MD loop; the same live storage owner, seen through the same view (offset,
    shape, strides) with an unchanged version counter (an in-place update bumps it, views share it),
    reuses the copy made for it.  Keyed on the base tensor, so `cell[0]` taken anew each step still hits."""
    global _cell_seen
    if not cell.is_cuda:
        return cell.detach().to(torch.float64)
    base = cell._base if cell._base is not None else cell
    key = (cell.storage_offset(), tuple(cell.shape), tuple(cell.stride()), cell.dtype, cell._version)
    seen = _cell_seen
    if seen is not None and seen[0]() is base and seen[1] == key:
        return seen[2]
    host = cell.detach().to("cpu", torch.float64)
    _cell_seen = (weakref.ref(base), key, host)
    return host


def radius_graph_pbc(pos: torch.Tensor, cell: torch.Tensor, cutoff: float):
    """pos [N,3], cell [3,3] (rows = lattice vectors) -> (src, dst, shifts[E,3] float)."""
    cell_cpu = _host_cell(cell)
    ncell, widths = _ncell(cell_cpu, cutoff)
    if pos.is_cuda and pos.dtype == torch.float32 and all(n >= 3 for n in ncell):
        return _cell_list_hip(pos.detach(), cell_cpu, cutoff, ncell)
    return _radius_graph_torch(pos, cell, cutoff)


def _mat3(x: torch.Tensor, m: torch.Tensor) -> torch.Tensor:
    """x [..., 3] . m [3, 3] as broadcast products (no library GEMM for these thin shapes)."""
    return (x.unsqueeze(-1) * m).sum(-2)


def _radius_graph_torch(pos: torch.Tensor, cell: torch.Tensor, cutoff: float):
    """The same edge list with torch device ops (CPU tensors, non-FP32 positions, few cells)."""
    dev = pos.device
    inv = torch.linalg.inv(cell.double())
    frac = _mat3(pos.double(), inv)
    k = torch.floor(frac)
    fw = frac - k
    lengths = cell.double().norm(dim=1)
    # perpendicular widths of the cell
    vol = torch.abs(torch.det(cell.double()))
    widths = torch.stack([vol / torch.linalg.cross(cell[1].double(), cell[2].double()).norm(),
                          vol / torch.linalg.cross(cell[2].double(), cell[0].double()).norm(),
                          vol / torch.linalg.cross(cell[0].double(), cell[1].double()).norm()])
    ncell = torch.floor(widths / cutoff).long().clamp(min=1)
    if bool((ncell >= 3).all()):
        return _cell_list(pos, cell, cutoff, fw, k, ncell)
    return _all_pairs(pos, cell, cutoff, fw, k, widths)


def _cell_list(pos, cell, cutoff, fw, k, ncell):
    dev = pos.device
    N = pos.shape[0]
    nc = ncell.tolist()
    cidx = torch.minimum((fw * ncell.double()).long(), ncell - 1)            # [N,3]
    flat = (cidx[:, 0] * nc[1] + cidx[:, 1]) * nc[2] + cidx[:, 2]
    total = nc[0] * nc[1] * nc[2]
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=total)
    M = int(counts.max().item())
    start = torch.cumsum(counts, 0) - counts
    slot = torch.arange(N, device=dev) - start[flat[order]]
    table = torch.full((total, M), -1, dtype=torch.long, device=dev)
    table[flat[order], slot] = order
    offs = torch.tensor(list(itertools.product((-1, 0, 1), repeat=3)), device=dev)      # [27,3]
    nb = cidx[:, None, :] + offs[None]                                                 # [N,27,3]
    wrap = torch.div(nb, ncell, rounding_mode="floor")                                 # image of the cell
    nbw = nb - wrap * ncell
    nflat = (nbw[..., 0] * nc[1] + nbw[..., 1]) * nc[2] + nbw[..., 2]                 # [N,27]
    cand = table[nflat]                                                                # [N,27,M]
    valid = cand >= 0
    j = cand.clamp(min=0)
    cellf = cell.double()
    posw = _mat3(fw, cellf)                                                            # wrapped positions
    img = _mat3(wrap.double(), cellf)                                                  # [N,27,3]
    # vec = pos_w[i] - (pos_w[j] + img)
    vec = posw[:, None, None, :] - (posw[j] + img[:, :, None, :])
    r2 = (vec * vec).sum(-1)
    keep = valid & (r2 < cutoff * cutoff) & (r2 > 1e-20)
    i_idx, o_idx, m_idx = torch.nonzero(keep, as_tuple=True)
    src = j[i_idx, o_idx, m_idx]
    dst = i_idx
    # shift = k_j - k_i - image  (vec = pos[dst] - pos[src] + shift @ cell)
    shifts = (k[src] - k[dst] - wrap[i_idx, o_idx].double())
    return src, dst, shifts.to(pos.dtype)


def _all_pairs(pos, cell, cutoff, fw, k, widths):
    dev = pos.device
    reps = torch.ceil(cutoff / widths).long().tolist()
    imgs = torch.tensor(list(itertools.product(*[range(-r, r + 1) for r in reps])), device=dev, dtype=torch.double)
    cellf = cell.double()
    posw = _mat3(fw, cellf)
    src_l, dst_l, sh_l = [], [], []
    N = pos.shape[0]
    chunk = max(1, int(4e7 // max(1, N * imgs.shape[0])))
    for s in range(0, N, chunk):
        i = torch.arange(s, min(N, s + chunk), device=dev)
        vec = posw[i, None, None, :] - (posw[None, :, None, :] + _mat3(imgs, cellf)[None, None])
        r2 = (vec * vec).sum(-1)
        keep = (r2 < cutoff * cutoff) & (r2 > 1e-20)
        a, b, c = torch.nonzero(keep, as_tuple=True)
        dst_l.append(i[a])
        src_l.append(b)
        sh_l.append(k[b] - k[i[a]] - imgs[c])
    return torch.cat(src_l), torch.cat(dst_l), torch.cat(sh_l).to(pos.dtype)
