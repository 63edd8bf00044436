// Edge pairs for the radial gates.
//
// The radial gates of an edge depend on its length only (the radial basis
// and MLP `fc`, layers.py:826-835), and a directed edge (s -> d, shift S) and
// its reverse (d -> s, -S) have bitwise-equal lengths: vec(reverse) =
// pos[s] - pos[d] - S.cell is exactly -vec in FP32 (negation and
// round-to-nearest are symmetric), so |vec| is the same float.  Their gates
// and gate tangents are therefore the same numbers, and one gate row can
// serve both edges: the gate kernels run over the canonical edge of every
// pair (half the edges of a symmetric neighbour list) and the message
// kernels read row gate_rows[e].
//
// Owners and readers: an edge whose source is below its receiver (or, with
// source == receiver, whose shift is zero or lexicographically positive)
// owns a gate row.  Every other edge looks up its reverse -- the first edge,
// in receiver-CSR order of the segment of src[e], with source dst[e] and
// shift -S -- which is an owner by the same rule, and reads the owner's row;
// without a reverse (a one-sided list, ids out of range) it owns a row.
// Duplicated edges may share an owner's row with its reverse: their lengths
// are bitwise equal too, and no kernel accumulates into gate rows.  Owners
// are numbered by a prefix sum in edge order (deterministic), so half of a
// symmetric list searches and half owns.
//
// Source CSR (ictc_edge_pairs_src_csr): when the lookup pairs every edge
// with its reverse one-to-one, the edges leaving node n are exactly the
// reverses of the edges entering it, so the source CSR has the receiver CSR's
// ptr and its order is those reverses ranked into edge order per node: the
// stable sort over src without sorting.
#include <hipcub/hipcub.hpp>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ictc_mi355x.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// Each wave takes kPerWave consecutive edges (two per lane), finds which of them are readers and hands the
// readers out to its lanes in edge order (ballot + prefix count through LDS), so every lane scans for one
// reader's reverse: owners cost no lane time in the scans.
constexpr int kPerWave = 128;
constexpr int kPartnerWaves = 4;

// true when the edge (s -> d, shift (x, y, z)) reads the row of its reverse rather than owning one
__device__ __forceinline__ bool reader(int64_t s, int64_t d, float x, float y, float z) {
  if (s != d) return s > d;
  return x != 0.f ? x < 0.f : (y != 0.f ? y < 0.f : z < 0.f);
}

// sorted_src[q] = src[order[q]] as int32 (receiver-CSR order; ids out of range as -1), so that the
// segment scans below read one contiguous 4-byte stream
__global__ void sorted_src_kernel(const int64_t* __restrict__ src, int64_t N, int64_t E,
                                  const int32_t* __restrict__ order, int32_t* __restrict__ sorted_src) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= E) return;
  const int64_t s = src[order ? order[q] : q];
  sorted_src[q] = (s >= 0 && s < N) ? (int32_t)s : -1;
}

struct ReaderSlot {
  int32_t e, s, d;
  float x, y, z;
};

__global__ __launch_bounds__(kPartnerWaves * 64) void partner_kernel(
    const int64_t* __restrict__ src, const int64_t* __restrict__ dst, const float* __restrict__ shifts, int64_t N,
    int64_t E, const int32_t* __restrict__ ptr, const int32_t* __restrict__ order,
    const int32_t* __restrict__ sorted_src, int32_t* __restrict__ partner, int32_t* __restrict__ rev) {
  __shared__ ReaderSlot slots[kPartnerWaves][kPerWave];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t base = ((int64_t)blockIdx.x * kPartnerWaves + w) * kPerWave;
  ReaderSlot* sl = slots[w];
  int total = 0;
#pragma unroll
  for (int h = 0; h < kPerWave / 64; ++h) {
    const int64_t e = base + 64 * h + lane;
    bool rd = false;
    int64_t s = -1, d = -1;
    float x = 0.f, y = 0.f, z = 0.f;
    if (e < E) {
      s = src[e];
      d = dst[e];
      if (shifts) {
        x = shifts[3 * e];
        y = shifts[3 * e + 1];
        z = shifts[3 * e + 2];
      }
      rd = s >= 0 && s < N && d >= 0 && d < N && reader(s, d, x, y, z);
      if (!rd) partner[e] = -1;   // owners and edges with ids out of range
    }
    const uint64_t m = __ballot(rd);
    if (rd) {
      const int k = total + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
      sl[k] = ReaderSlot{(int32_t)e, (int32_t)s, (int32_t)d, x, y, z};
    }
    total += __popcll(m);
  }
  __syncthreads();
  for (int k = lane; k < total; k += 64) {
    const ReaderSlot r = sl[k];
    const int32_t beg = ptr[r.s], end = ptr[r.s + 1];
    int32_t best = INT32_MAX;
    // the first reverse in CSR order: sources d among the edges into s, read as 16-byte quads of 4-aligned
    // positions (the sorted_src slab is padded to 256 bytes, so a quad past the last edge stays inside it)
#pragma unroll 4
    for (int32_t q4 = beg & ~3; q4 < end && best == INT32_MAX; q4 += 4) {
      const int4 v = *reinterpret_cast<const int4*>(sorted_src + q4);
      const int32_t cand[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int32_t q = q4 + c;
        bool hit = cand[c] == r.d && q >= beg && q < end && best == INT32_MAX;
        if (hit) {
          const int32_t e2 = order ? order[q] : q;
          hit = e2 != r.e && (!shifts || (shifts[3 * (int64_t)e2] == -r.x && shifts[3 * (int64_t)e2 + 1] == -r.y &&
                                          shifts[3 * (int64_t)e2 + 2] == -r.z));
        }
        if (hit) best = q;
      }
    }
    const int32_t p = best == INT32_MAX ? -1 : (order ? order[best] : best);
    partner[r.e] = p;
    if (rev && p >= 0) rev[p] = r.e;   // the reverse of p, for the source CSR (a second claimant races)
  }
}

__global__ void canonical_kernel(const int32_t* __restrict__ partner, int64_t E, int32_t* __restrict__ flag) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  flag[e] = partner[e] < 0;   // owners and readers without a reverse
}

__global__ void rows_kernel(const int32_t* __restrict__ partner, const int32_t* __restrict__ flag,
                            const int32_t* __restrict__ idx, int64_t E, int32_t* __restrict__ gate_rows,
                            int32_t* __restrict__ reps, int32_t* __restrict__ count) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const bool canon = flag[e] != 0;
  gate_rows[e] = idx[canon ? e : partner[e]];
  if (canon) reps[idx[e]] = (int32_t)e;
  if (e == E - 1) count[0] = idx[e] + flag[e];
}

__global__ void zero_count_kernel(int32_t* count) { count[0] = 0; }

// The reverse map for the source CSR: reverse(e) = partner[e] for a reader, rev[e] (written by the reader
// that found e, -1 before) for a row owner.  It is one-to-one when every reader's reverse names it back and
// every owner was found: two readers finding one owner (duplicated edges) leave one of them unnamed.
__global__ void fill_kernel(int32_t* __restrict__ a, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) a[i] = v;
}

__device__ __forceinline__ int32_t reverse_of(const int32_t* __restrict__ partner, const int32_t* __restrict__ rev,
                                              int32_t e) {
  const int32_t p = partner[e];
  return p >= 0 ? p : rev[e];
}

__global__ void check_kernel(const int32_t* __restrict__ partner, const int32_t* __restrict__ rev, int64_t E,
                             int32_t* __restrict__ bad) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int32_t p = partner[e];
  const bool ok = p >= 0 ? rev[p] == (int32_t)e : rev[e] >= 0;
  if (!ok) atomicOr(bad, 1);
}

__global__ void ok_kernel(const int32_t* __restrict__ bad, int32_t* __restrict__ src_ok) {
  src_ok[0] = bad[0] == 0 ? 1 : 0;
}

// One wave per node s: the edges leaving s are the reverses of the edges entering s (segment s of the
// receiver CSR), and they are written in edge order (a stable sort by source) by ranking each value against
// the whole segment.  Ranks stay in [0, segment length), so a map that is not one-to-one still writes
// inside the segment (the host then does not use the result).
__global__ __launch_bounds__(256) void src_order_kernel(const int32_t* __restrict__ ptr,
                                                        const int32_t* __restrict__ order,
                                                        const int32_t* __restrict__ partner,
                                                        const int32_t* __restrict__ rev, int64_t N,
                                                        int32_t* __restrict__ src_order) {
  const int lane = threadIdx.x & 63;
  const int64_t s = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (s >= N) return;   // whole waves leave together
  const int32_t beg = ptr[s], k = ptr[s + 1] - beg;
  for (int32_t t0 = 0; t0 < k; t0 += 64) {
    const bool mine = t0 + lane < k;
    const int32_t v = mine ? reverse_of(partner, rev, order ? order[beg + t0 + lane] : beg + t0 + lane) : 0;
    int32_t rank = 0;
    for (int32_t u0 = 0; u0 < k; u0 += 64) {
      const int32_t x = u0 == t0 ? v
                        : u0 + lane < k ? reverse_of(partner, rev, order ? order[beg + u0 + lane] : beg + u0 + lane)
                                        : 0;
      const int32_t n = min(64, k - u0);
      for (int32_t u = 0; u < n; ++u) rank += __builtin_amdgcn_readlane(x, u) < v;
    }
    if (mine) src_order[beg + rank] = v;
  }
}

// The scan's temporary-storage query asks the runtime for device properties; its answer is kept per
// thread for the last (device, size).
size_t scan_temp_bytes(int64_t E) {
  thread_local int memo_dev = -1;
  thread_local int64_t memo_e = -1;
  thread_local size_t memo_bytes = 0;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) dev = -1;
  if (dev == memo_dev && E == memo_e) return memo_bytes;
  size_t bytes = 0;
  hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, (const int32_t*)nullptr, (int32_t*)nullptr, (int)(E > 0 ? E : 1));
  memo_dev = dev, memo_e = E, memo_bytes = bytes;
  return bytes;
}

}  // namespace

extern "C" {

int64_t ictc_edge_pairs_workspace_bytes(int64_t E) {
  if (E < 0 || E >= (int64_t(1) << 30)) return -1;   // int32 edge ids
  return (int64_t)(5 * align256(sizeof(int32_t) * (size_t)(E > 0 ? E : 1)) + align256(sizeof(int32_t)) +
                   align256(scan_temp_bytes(E)));
}

}  // extern "C"

namespace {

int edge_pairs(const int64_t* src, const int64_t* dst, const float* shifts, int64_t N, int64_t E,
               const int32_t* dst_ptr, const int32_t* dst_order, int32_t* gate_rows, int32_t* reps, int32_t* count,
               int32_t* src_order, int32_t* src_ok, void* workspace, int64_t workspace_bytes, void* stream) {
  if (N < 0 || E < 0) return fail(ICTC_ERR_ARGUMENT, "edge pairs: negative size");
  if (E >= (int64_t(1) << 30) || N >= (int64_t(1) << 31) - 2)
    return fail(ICTC_ERR_UNSUPPORTED, "edge pairs: 2^30 edges or more, or more than 2^31 nodes");
  if (!count) return fail(ICTC_ERR_ARGUMENT, "edge pairs: null count");
  hipStream_t st = (hipStream_t)stream;
  if (E == 0) {   // no pairs: count = 0 (a fill kernel, so the call stays graph-capturable)
    hipLaunchKernelGGL(zero_count_kernel, dim3(1), dim3(1), 0, st, count);
    if (src_ok) hipLaunchKernelGGL(zero_count_kernel, dim3(1), dim3(1), 0, st, src_ok);
    const hipError_t z = hipGetLastError();
    return z == hipSuccess ? ICTC_OK : fail(ICTC_ERR_RUNTIME, "ictc_edge_pairs launch");
  }
  if (!src || !dst || !dst_ptr || !gate_rows || !reps || !workspace)
    return fail(ICTC_ERR_ARGUMENT, "edge pairs: null operand");
  if (workspace_bytes < ictc_edge_pairs_workspace_bytes(E))
    return fail(ICTC_ERR_ARGUMENT, "edge pairs: workspace smaller than ictc_edge_pairs_workspace_bytes");
  char* ws = static_cast<char*>(workspace);
  const size_t slab = align256(sizeof(int32_t) * (size_t)E);
  int32_t* partner = (int32_t*)ws;
  int32_t* flag = (int32_t*)(ws + slab);
  int32_t* idx = (int32_t*)(ws + 2 * slab);
  int32_t* sorted_src = (int32_t*)(ws + 3 * slab);
  int32_t* rev = (int32_t*)(ws + 4 * slab);
  int32_t* bad = (int32_t*)(ws + 5 * slab);
  void* temp = ws + 5 * slab + align256(sizeof(int32_t));
  size_t temp_bytes = scan_temp_bytes(E);
  const unsigned blocks = (unsigned)((E + 255) / 256);
  const unsigned partner_blocks = (unsigned)((E + kPerWave * kPartnerWaves - 1) / (kPerWave * kPartnerWaves));
  hipLaunchKernelGGL(sorted_src_kernel, dim3(blocks), dim3(256), 0, st, src, N, E, dst_order, sorted_src);
  if (src_order) hipLaunchKernelGGL(fill_kernel, dim3(blocks), dim3(256), 0, st, rev, E, -1);
  hipLaunchKernelGGL(partner_kernel, dim3(partner_blocks), dim3(kPartnerWaves * 64), 0, st, src, dst, shifts, N, E, dst_ptr,
                     dst_order, sorted_src, partner, src_order ? rev : nullptr);
  hipLaunchKernelGGL(canonical_kernel, dim3(blocks), dim3(256), 0, st, partner, E, flag);
  if (hipcub::DeviceScan::ExclusiveSum(temp, temp_bytes, flag, idx, (int)E, st) != hipSuccess)
    return fail(ICTC_ERR_RUNTIME, "edge pairs: scan");
  hipLaunchKernelGGL(rows_kernel, dim3(blocks), dim3(256), 0, st, partner, flag, idx, E, gate_rows, reps, count);
  if (src_order) {
    hipLaunchKernelGGL(fill_kernel, dim3(1), dim3(64), 0, st, bad, (int64_t)1, 0);
    hipLaunchKernelGGL(check_kernel, dim3(blocks), dim3(256), 0, st, partner, rev, E, bad);
    hipLaunchKernelGGL(ok_kernel, dim3(1), dim3(1), 0, st, bad, src_ok);
    if (N > 0)
      hipLaunchKernelGGL(src_order_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, dst_ptr, dst_order,
                         partner, rev, N, src_order);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof(buf), "ictc_edge_pairs launch: %s", hipGetErrorString(e));
    return fail(ICTC_ERR_RUNTIME, buf);
  }
  return ICTC_OK;
}

}  // namespace

extern "C" {

int ictc_edge_pairs(const int64_t* src, const int64_t* dst, const float* shifts, int64_t N, int64_t E,
                    const int32_t* dst_ptr, const int32_t* dst_order, int32_t* gate_rows, int32_t* reps,
                    int32_t* count, void* workspace, int64_t workspace_bytes, void* stream) {
  return edge_pairs(src, dst, shifts, N, E, dst_ptr, dst_order, gate_rows, reps, count, nullptr, nullptr,
                    workspace, workspace_bytes, stream);
}

int ictc_edge_pairs_src_csr(const int64_t* src, const int64_t* dst, const float* shifts, int64_t N, int64_t E,
                            const int32_t* dst_ptr, const int32_t* dst_order, int32_t* gate_rows, int32_t* reps,
                            int32_t* count, int32_t* src_order, int32_t* src_ok, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  if (!src_order || !src_ok) return fail(ICTC_ERR_ARGUMENT, "edge pairs: null source order");
  return edge_pairs(src, dst, shifts, N, E, dst_ptr, dst_order, gate_rows, reps, count, src_order, src_ok,
                    workspace, workspace_bytes, stream);
}

}  // extern "C"
