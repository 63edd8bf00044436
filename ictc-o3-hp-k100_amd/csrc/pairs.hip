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

// kLanes lanes per edge scan the receiver segment of src[e] in strides of kLanes and keep the smallest CSR
// position that matches (the first match in CSR order), reduced across the group (2 lanes measured
// fastest against 4, 8 and 16 on the cfg4 graph: more edges in flight per wave, loads unrolled).
constexpr int kLanes = 2;

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

__global__ __launch_bounds__(256) void partner_kernel(const int64_t* __restrict__ src, const int64_t* __restrict__ dst,
                                                      const float* __restrict__ shifts, int64_t N, int64_t E,
                                                      const int32_t* __restrict__ ptr,
                                                      const int32_t* __restrict__ order,
                                                      const int32_t* __restrict__ sorted_src,
                                                      int32_t* __restrict__ partner) {
  const int64_t e = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kLanes;
  const int sub = threadIdx.x % kLanes;
  if (e >= E) return;   // whole groups leave together (E * kLanes lanes, groups aligned)
  const int64_t s = src[e], d = dst[e];
  int32_t best = INT32_MAX;
  const float sx = shifts ? shifts[3 * e] : 0.f, sy = shifts ? shifts[3 * e + 1] : 0.f,
              sz = shifts ? shifts[3 * e + 2] : 0.f;
  if (s >= 0 && s < N && d >= 0 && d < N && reader(s, d, sx, sy, sz)) {
    const int32_t end = ptr[s + 1];
    // every lane runs its whole strided scan (no early exit before the cross-lane reduction) and keeps
    // its first match
#pragma unroll 16
    for (int32_t q = ptr[s] + sub; q < end; q += kLanes) {
      bool hit = sorted_src[q] == (int32_t)d && best == INT32_MAX;
      if (hit) {
        const int32_t e2 = order ? order[q] : q;
        hit = e2 != e && (!shifts || (shifts[3 * (int64_t)e2] == -sx && shifts[3 * (int64_t)e2 + 1] == -sy &&
                                      shifts[3 * (int64_t)e2 + 2] == -sz));
      }
      if (hit) best = q;
    }
  }
#pragma unroll
  for (int m = kLanes / 2; m > 0; m >>= 1) best = min(best, __shfl_xor(best, m, kLanes));
  if (sub == 0) partner[e] = best == INT32_MAX ? -1 : (order ? order[best] : best);
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

size_t scan_temp_bytes(int64_t E) {
  size_t bytes = 0;
  hipcub::DeviceScan::ExclusiveSum(nullptr, bytes, (const int32_t*)nullptr, (int32_t*)nullptr, (int)(E > 0 ? E : 1));
  return bytes;
}

}  // namespace

extern "C" {

int64_t ictc_edge_pairs_workspace_bytes(int64_t E) {
  if (E < 0 || E >= (int64_t(1) << 30)) return -1;   // E * kLanes threads under 2^31
  return (int64_t)(4 * align256(sizeof(int32_t) * (size_t)(E > 0 ? E : 1)) + align256(scan_temp_bytes(E)));
}

int ictc_edge_pairs(const int64_t* src, const int64_t* dst, const float* shifts, int64_t N, int64_t E,
                    const int32_t* dst_ptr, const int32_t* dst_order, int32_t* gate_rows, int32_t* reps,
                    int32_t* count, void* workspace, int64_t workspace_bytes, void* stream) {
  if (N < 0 || E < 0) return fail(ICTC_ERR_ARGUMENT, "edge pairs: negative size");
  if (E >= (int64_t(1) << 30) || N >= (int64_t(1) << 31) - 2)
    return fail(ICTC_ERR_UNSUPPORTED, "edge pairs: 2^30 edges or more, or more than 2^31 nodes");
  if (!count) return fail(ICTC_ERR_ARGUMENT, "edge pairs: null count");
  hipStream_t st = (hipStream_t)stream;
  if (E == 0) {   // no pairs: count = 0 (a fill kernel, so the call stays graph-capturable)
    hipLaunchKernelGGL(zero_count_kernel, dim3(1), dim3(1), 0, st, count);
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
  void* temp = ws + 4 * slab;
  size_t temp_bytes = scan_temp_bytes(E);
  const unsigned blocks = (unsigned)((E + 255) / 256);
  const unsigned partner_blocks = (unsigned)((E * kLanes + 255) / 256);
  hipLaunchKernelGGL(sorted_src_kernel, dim3(blocks), dim3(256), 0, st, src, N, E, dst_order, sorted_src);
  hipLaunchKernelGGL(partner_kernel, dim3(partner_blocks), dim3(256), 0, st, src, dst, shifts, N, E, dst_ptr,
                     dst_order, sorted_src, partner);
  hipLaunchKernelGGL(canonical_kernel, dim3(blocks), dim3(256), 0, st, partner, E, flag);
  if (hipcub::DeviceScan::ExclusiveSum(temp, temp_bytes, flag, idx, (int)E, st) != hipSuccess)
    return fail(ICTC_ERR_RUNTIME, "edge pairs: scan");
  hipLaunchKernelGGL(rows_kernel, dim3(blocks), dim3(256), 0, st, partner, flag, idx, E, gate_rows, reps, count);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof(buf), "ictc_edge_pairs launch: %s", hipGetErrorString(e));
    return fail(ICTC_ERR_RUNTIME, buf);
  }
  return ICTC_OK;
}

}  // extern "C"
