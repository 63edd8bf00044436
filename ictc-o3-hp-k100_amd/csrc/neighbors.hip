// Periodic radius graph (cell list) on the GPU, receiver-sorted and deterministic.
//
// The reference delegates neighbour search to ASE / matscipy / torch_cluster
// (examples/predict.py:62, data/preprocessing.py:11, utils/graph_utils.py:217-297);
// the model consumes edges with vec = pos[dst] - pos[src] + shift @ cell
// (backbone.py:940-944).  Every directed pair (including periodic self-images)
// with 1e-20 < |vec|^2 < cutoff^2 is emitted once.
//
// Steps: (1) per atom, fractional coordinates in FP64, image k = floor(frac),
// wrapped position, cell index; (2) atoms grouped by cell with the stable CSR
// build (ictc_csr_build); (3) each receiver counts its neighbours
// over the 27 surrounding cells (one wave per receiver); (4) exclusive scan of the counts; (5) the same
// walk writes src / dst / shift at the receiver's offset.  Candidates are
// visited in a fixed order (cell offsets, then atoms in index order within a
// cell), so the edge list is receiver-sorted and identical run to run.
// Requires at least 3 cells per periodic direction (cell width >= cutoff).
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ictc_mi355x.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

constexpr int kBlock = 256;

struct Geometry {
  double cell[9];  // rows = lattice vectors
  double inv[9];   // inverse of cell (frac = pos @ inv)
  double cut2;
  int nc[3];
};

__global__ __launch_bounds__(kBlock) void nl_prepare_kernel(const float* __restrict__ pos, int64_t N, Geometry g,
                                                           int64_t* __restrict__ cell_key, double* __restrict__ posw,
                                                           int32_t* __restrict__ kimg, int32_t* __restrict__ cidx) {
  const int64_t a = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (a >= N) return;
  const double p[3] = {pos[3 * a], pos[3 * a + 1], pos[3 * a + 2]};
  double fw[3];
  int ci[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    const double f = p[0] * g.inv[0 * 3 + d] + p[1] * g.inv[1 * 3 + d] + p[2] * g.inv[2 * 3 + d];
    const double k = floor(f);
    fw[d] = f - k;
    kimg[3 * a + d] = (int32_t)k;
    int c = (int)(fw[d] * g.nc[d]);
    ci[d] = c < g.nc[d] - 1 ? c : g.nc[d] - 1;
    cidx[3 * a + d] = ci[d];
  }
#pragma unroll
  for (int d = 0; d < 3; ++d) posw[3 * a + d] = fw[0] * g.cell[0 * 3 + d] + fw[1] * g.cell[1 * 3 + d] + fw[2] * g.cell[2 * 3 + d];
  cell_key[a] = ((int64_t)ci[0] * g.nc[1] + ci[1]) * g.nc[2] + ci[2];
}

// Walk the candidates of receiver i; FILL = false counts, FILL = true writes.  One wave per receiver: the
// candidates of its 27 cells (cell offsets in a fixed order, atoms in index order within a cell) are numbered
// 0 .. total-1 in that order and tested 64 at a time, one per lane; the hits of a chunk are compacted in lane
// order (ballot + prefix count), so the edges come out in the same order as a sequential walk.  Lanes 0..26
// hold one cell each (its first candidate and the inclusive prefix of the candidate counts), and a lane finds
// the cell of its candidate against those prefixes, read as wave-uniform scalars.
constexpr int kWalkWaves = kBlock / 64;

template <bool FILL>
__global__ __launch_bounds__(kBlock) void nl_walk_kernel(int64_t N, Geometry g, const double* __restrict__ posw,
                                                        const int32_t* __restrict__ kimg,
                                                        const int32_t* __restrict__ cidx,
                                                        const int32_t* __restrict__ cptr,
                                                        const int32_t* __restrict__ corder,
                                                        int32_t* __restrict__ count, const int64_t* __restrict__ row,
                                                        int64_t* __restrict__ src, int64_t* __restrict__ dst,
                                                        float* __restrict__ shift, int64_t capacity) {
  const int lane = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * kWalkWaves + (threadIdx.x >> 6);
  if (i >= N) return;   // whole waves leave together
  const double pi[3] = {posw[3 * i], posw[3 * i + 1], posw[3 * i + 2]};
  const int ci[3] = {cidx[3 * i], cidx[3 * i + 1], cidx[3 * i + 2]};
  // lane o < 27: cell offset o, its first candidate and candidate count
  int32_t first = 0, cnt = 0;
  if (lane < 27) {
    const int off[3] = {lane / 9 - 1, (lane / 3) % 3 - 1, lane % 3 - 1};
    int nb[3];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const int c = ci[d] + off[d];
      nb[d] = c - (c < 0 ? -1 : (c >= g.nc[d] ? 1 : 0)) * g.nc[d];
    }
    const int64_t cell = ((int64_t)nb[0] * g.nc[1] + nb[1]) * g.nc[2] + nb[2];
    first = cptr[cell];
    cnt = cptr[cell + 1] - first;
  }
  int32_t incl = cnt;   // inclusive prefix over lanes
#pragma unroll
  for (int k = 1; k < 32; k <<= 1) {
    const int32_t v = __shfl_up(incl, k, 64);
    if (lane >= k) incl += v;
  }
  int32_t bound[27];
#pragma unroll
  for (int k = 0; k < 27; ++k) bound[k] = __builtin_amdgcn_readlane(incl, k);
  const int32_t total = bound[26];
  int64_t out = FILL ? row[i] : 0;
  int32_t n = 0;
  for (int32_t t0 = 0; t0 < total; t0 += 64) {
    const int32_t t = t0 + lane;
    int o = 0;
#pragma unroll
    for (int k = 0; k < 26; ++k) o += t >= bound[k];
    const int32_t excl = __shfl(incl - cnt, o, 64);
    const int32_t q = __shfl(first, o, 64) + (t - excl);
    bool hit = false;
    int32_t j = 0;
    int wrap[3] = {0, 0, 0};
    if (t < total) {
      const int off[3] = {o / 9 - 1, (o / 3) % 3 - 1, o % 3 - 1};
#pragma unroll
      for (int d = 0; d < 3; ++d) {
        const int c = ci[d] + off[d];
        wrap[d] = c < 0 ? -1 : (c >= g.nc[d] ? 1 : 0);
      }
      double img[3];
#pragma unroll
      for (int d = 0; d < 3; ++d)
        img[d] = wrap[0] * g.cell[0 * 3 + d] + wrap[1] * g.cell[1 * 3 + d] + wrap[2] * g.cell[2 * 3 + d];
      j = corder[q];
      double r2 = 0.0;
#pragma unroll
      for (int d = 0; d < 3; ++d) {
        const double v = pi[d] - (posw[3 * j + d] + img[d]);
        r2 += v * v;
      }
      hit = r2 < g.cut2 && r2 > 1e-20;
    }
    const uint64_t mask = __ballot(hit);
    if (FILL) {
      const int64_t at = out + __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
      if (hit && at < capacity) {   // edges past the caller's capacity are counted, not written
        src[at] = j;
        dst[at] = i;
#pragma unroll
        for (int d = 0; d < 3; ++d) shift[3 * at + d] = (float)(kimg[3 * j + d] - kimg[3 * i + d] - wrap[d]);
      }
      out += __popcll(mask);
    } else {
      n += __popcll(mask);
    }
  }
  if (!FILL && lane == 0) count[i] = n;
}

// count != nullptr: count[atoms] = 0 (scan tail); else edges[0] = row[atoms].
__global__ void nl_finish_kernel(int32_t* __restrict__ count, int64_t atoms, const int64_t* __restrict__ row,
                                 int64_t* __restrict__ edges) {
  if (threadIdx.x != 0) return;
  if (count) count[atoms] = 0;
  else edges[0] = row[atoms];
}

struct Layout {
  size_t key, posw, kimg, cidx, cptr, corder, count, row, csr_ws, scan_ws, total;
  int64_t csr_ws_bytes;
  size_t scan_ws_bytes;
};

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

bool layout_for(int64_t N, int64_t ncells, Layout* L) {
  const int64_t csr = ictc_csr_workspace_bytes(N, ncells);
  if (csr < 0) return false;
  // the scan's temporary-storage query asks the runtime for device properties: kept per thread for the
  // last (device, size)
  thread_local int memo_dev = -1;
  thread_local int64_t memo_n = -1;
  thread_local size_t memo_scan = 0;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  size_t scan = 0;
  if (dev == memo_dev && N == memo_n) {
    scan = memo_scan;
  } else {
    (void)hipcub::DeviceScan::ExclusiveSum(nullptr, scan, (const int32_t*)nullptr, (int64_t*)nullptr, (int)(N + 1));
    memo_dev = dev, memo_n = N, memo_scan = scan;
  }
  size_t o = 0;
  L->key = o;    o += align256(sizeof(int64_t) * N);
  L->posw = o;   o += align256(sizeof(double) * 3 * N);
  L->kimg = o;   o += align256(sizeof(int32_t) * 3 * N);
  L->cidx = o;   o += align256(sizeof(int32_t) * 3 * N);
  L->cptr = o;   o += align256(sizeof(int32_t) * (ncells + 2));
  L->corder = o; o += align256(sizeof(int32_t) * (N > 0 ? N : 1));
  L->count = o;  o += align256(sizeof(int32_t) * (N + 1));
  L->row = o;    o += align256(sizeof(int64_t) * (N + 1));
  L->csr_ws = o; o += align256((size_t)(csr > 0 ? csr : 1));
  L->scan_ws = o; o += align256(scan > 0 ? scan : 1);
  L->csr_ws_bytes = csr;
  L->scan_ws_bytes = scan;
  L->total = o;
  return true;
}

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return ICTC_OK;
  char buf[256];
  snprintf(buf, sizeof(buf), "%s: %s", what, hipGetErrorString(e));
  return fail(ICTC_ERR_RUNTIME, buf);
}

int make_geometry(const double* cell, double cutoff, const int* ncell, Geometry* g) {
  if (!cell || !ncell || !(cutoff > 0.0)) return fail(ICTC_ERR_ARGUMENT, "neighbours: invalid cell / cutoff");
  for (int d = 0; d < 3; ++d)
    if (ncell[d] < 3) return fail(ICTC_ERR_UNSUPPORTED, "neighbours: the cell list needs >= 3 cells per direction");
  const double* c = cell;
  const double det = c[0] * (c[4] * c[8] - c[5] * c[7]) - c[1] * (c[3] * c[8] - c[5] * c[6]) +
                     c[2] * (c[3] * c[7] - c[4] * c[6]);
  if (!(det != 0.0)) return fail(ICTC_ERR_ARGUMENT, "neighbours: singular cell");
  const double id = 1.0 / det;
  double* v = g->inv;
  v[0] = (c[4] * c[8] - c[5] * c[7]) * id;
  v[1] = (c[2] * c[7] - c[1] * c[8]) * id;
  v[2] = (c[1] * c[5] - c[2] * c[4]) * id;
  v[3] = (c[5] * c[6] - c[3] * c[8]) * id;
  v[4] = (c[0] * c[8] - c[2] * c[6]) * id;
  v[5] = (c[2] * c[3] - c[0] * c[5]) * id;
  v[6] = (c[3] * c[7] - c[4] * c[6]) * id;
  v[7] = (c[1] * c[6] - c[0] * c[7]) * id;
  v[8] = (c[0] * c[4] - c[1] * c[3]) * id;
  for (int k = 0; k < 9; ++k) g->cell[k] = c[k];
  g->cut2 = cutoff * cutoff;
  for (int d = 0; d < 3; ++d) g->nc[d] = ncell[d];
  return ICTC_OK;
}

}  // namespace

extern "C" {

int64_t ictc_neighbors_workspace_bytes(int64_t atoms, const int* ncell) {
  if (atoms < 0 || !ncell || ncell[0] < 1 || ncell[1] < 1 || ncell[2] < 1) return -1;
  Layout L;
  if (!layout_for(atoms, (int64_t)ncell[0] * ncell[1] * ncell[2], &L)) return -1;
  return (int64_t)L.total;
}

int ictc_neighbors_count(const float* pos, int64_t atoms, const double* cell, double cutoff, const int* ncell,
                         void* workspace, int64_t workspace_bytes, int64_t* edges, void* stream) {
  Geometry g;
  if (int rc = make_geometry(cell, cutoff, ncell, &g)) return rc;
  if (atoms < 0 || !edges || !workspace || (atoms > 0 && !pos))
    return fail(ICTC_ERR_ARGUMENT, "neighbours: null operand");
  const int64_t ncells = (int64_t)ncell[0] * ncell[1] * ncell[2];
  Layout L;
  if (!layout_for(atoms, ncells, &L) || workspace_bytes < (int64_t)L.total)
    return fail(ICTC_ERR_ARGUMENT, "neighbours: workspace too small");
  char* w = (char*)workspace;
  hipStream_t st = (hipStream_t)stream;
  const unsigned blocks = (unsigned)((atoms + kBlock - 1) / kBlock);
  if (atoms > 0) {
    hipLaunchKernelGGL(nl_prepare_kernel, dim3(blocks), dim3(kBlock), 0, st, pos, atoms, g, (int64_t*)(w + L.key),
                       (double*)(w + L.posw), (int32_t*)(w + L.kimg), (int32_t*)(w + L.cidx));
    if (int rc = check_launch("neighbours prepare")) return rc;
  }
  if (int rc = ictc_csr_build((const int64_t*)(w + L.key), atoms, ncells, (int32_t*)(w + L.cptr),
                              (int32_t*)(w + L.corder), w + L.csr_ws, L.csr_ws_bytes, stream))
    return rc;
  int32_t* count = (int32_t*)(w + L.count);
  if (atoms > 0) {
    const unsigned walk_blocks = (unsigned)((atoms + kWalkWaves - 1) / kWalkWaves);
    hipLaunchKernelGGL((nl_walk_kernel<false>), dim3(walk_blocks), dim3(kBlock), 0, st, atoms, g, (const double*)(w + L.posw),
                       (const int32_t*)(w + L.kimg), (const int32_t*)(w + L.cidx), (const int32_t*)(w + L.cptr),
                       (const int32_t*)(w + L.corder), count, nullptr, nullptr, nullptr, nullptr, (int64_t)0);
    if (int rc = check_launch("neighbours count")) return rc;
  }
  // count[atoms] = 0, so the exclusive scan's last entry row[atoms] is the edge count.
  hipLaunchKernelGGL(nl_finish_kernel, dim3(1), dim3(64), 0, st, count, atoms, (const int64_t*)nullptr, edges);
  if (int rc = check_launch("neighbours scan setup")) return rc;
  size_t scan_bytes = L.scan_ws_bytes;
  if (hipcub::DeviceScan::ExclusiveSum(w + L.scan_ws, scan_bytes, count, (int64_t*)(w + L.row), (int)(atoms + 1),
                                       st) != hipSuccess)
    return fail(ICTC_ERR_RUNTIME, "neighbours: scan failed");
  hipLaunchKernelGGL(nl_finish_kernel, dim3(1), dim3(64), 0, st, (int32_t*)nullptr, atoms,
                     (const int64_t*)(w + L.row), edges);
  return check_launch("neighbours total");
}

int ictc_neighbors_fill_capacity(const float* pos, int64_t atoms, const double* cell, double cutoff,
                                 const int* ncell, const void* workspace, int64_t workspace_bytes, int64_t* src,
                                 int64_t* dst, float* shifts, int64_t capacity, void* stream) {
  Geometry g;
  if (int rc = make_geometry(cell, cutoff, ncell, &g)) return rc;
  (void)pos;
  const int64_t ncells = (int64_t)ncell[0] * ncell[1] * ncell[2];
  Layout L;
  if (atoms < 0 || !workspace || !layout_for(atoms, ncells, &L) || workspace_bytes < (int64_t)L.total)
    return fail(ICTC_ERR_ARGUMENT, "neighbours: workspace too small");
  if (capacity < 0) return fail(ICTC_ERR_ARGUMENT, "neighbours: negative capacity");
  if (atoms == 0 || capacity == 0) return ICTC_OK;
  if (!src || !dst || !shifts) return fail(ICTC_ERR_ARGUMENT, "neighbours: null output");
  const char* w = (const char*)workspace;
  const unsigned blocks = (unsigned)((atoms + kWalkWaves - 1) / kWalkWaves);
  hipLaunchKernelGGL((nl_walk_kernel<true>), dim3(blocks), dim3(kBlock), 0, (hipStream_t)stream, atoms, g,
                     (const double*)(w + L.posw), (const int32_t*)(w + L.kimg), (const int32_t*)(w + L.cidx),
                     (const int32_t*)(w + L.cptr), (const int32_t*)(w + L.corder), (int32_t*)nullptr,
                     (const int64_t*)(w + L.row), src, dst, shifts, capacity);
  return check_launch("neighbours fill");
}

int ictc_neighbors_fill(const float* pos, int64_t atoms, const double* cell, double cutoff, const int* ncell,
                        const void* workspace, int64_t workspace_bytes, int64_t* src, int64_t* dst, float* shifts,
                        void* stream) {
  return ictc_neighbors_fill_capacity(pos, atoms, cell, cutoff, ncell, workspace, workspace_bytes, src, dst, shifts,
                                      INT64_MAX, stream);
}

}  // extern "C"
