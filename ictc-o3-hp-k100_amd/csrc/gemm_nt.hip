// General channel-linear GEMM and the per-graph energy sum.
//
// C[M, N] (+)= A[M, K] . B[N, K]^T, row-major operands with leading
// dimensions, FP32 in and out, products and sums on FP32 MFMA
// (v_mfma_f32_16x16x4f32: the precision of an FP32 library GEMM with TF32
// off).  This is every `x W^T` / `u W` of the training path's channel
// linears and readouts that the wider kernels (gate_gemm.hip: 64-wide inputs;
// gemm_tn.hip: weight gradients) do not take: the per-degree and
// per-path channel maps (layers.py:317-355, ictd_irreps.py:207-227), the
// species-selected self connection (layers.py:21-87) and the readouts
// (heads.py:12-27), forward and input adjoint.
//
// Tiling: a block of 4 waves computes a 128 x 64 output tile; each K step
// stages a 128 x 32 slab of A and a 64 x 32 slab of B through LDS (reduction
// index outer, so every MFMA operand is one LDS read; 16-byte global loads
// along K where pitch and alignment allow), and wave w multiplies its rows
// 32 w .. 32 w + 31 (two 16-row blocks) against the four 16-column blocks:
// 8 MFMAs per 6 LDS reads.  Thin shapes (N = 1 readouts) are HBM-bound and
// read A once.
//
// Per-graph energy sum: out[b] = sum over atoms n with batch[n] == b of
// values[n] in FP64, one block per graph scanning the atoms in index order and
// adding the thread sums in a fixed tree: deterministic without atomics.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ictc_mi355x.h"
#include "split_bf16.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kTM = 128;  // output tile rows (4 waves x 32)
constexpr int kTN = 64;   // output tile columns
constexpr int kK = 32;    // K per LDS stage

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

// Row r of an operand starts at (r / group) * gstride + (r % group) * ld: rows in groups of `group`
// consecutive rows `ld` apart, groups `gstride` apart (group = 1: plain row pitch gstride).
struct RowMap {
  int64_t ld, group, gstride;
  __device__ __forceinline__ int64_t off(int64_t r) const {
    if (group == 1) return r * gstride;
    const uint32_t g = (uint32_t)r / (uint32_t)group;
    return (int64_t)g * gstride + (int64_t)((uint32_t)r - g * (uint32_t)group) * ld;
  }
};

// Stage rows [r0, r0 + R) x k [k0, k0 + kK) of a row-major operand into lds[k][row] (zero outside).
// Thread t covers (R * kK / 256) entries as float4 runs along k when the pitch and base allow it.
template <int R, bool VEC>
__device__ __forceinline__ void stage(const float* __restrict__ X, int64_t rows, int64_t K, RowMap map, int64_t r0,
                                      int64_t k0, float (*lds)[R + 4]) {
  constexpr int per = R * kK / 256;   // entries per thread (16 for R = 128, 8 for R = 64)
  constexpr int runs = per / 4;
#pragma unroll
  for (int q = 0; q < runs; ++q) {
    const int idx = threadIdx.x + 256 * q;      // run index: row = idx / (kK / 4), k = 4 (idx % (kK / 4))
    const int row = idx / (kK / 4), kq = 4 * (idx % (kK / 4));
    const int64_t r = r0 + row, k = k0 + kq;
    float v[4];
    const int64_t base = r < rows ? map.off(r) : 0;
    if (VEC && r < rows && k + 3 < K) {
      const v4f x = *reinterpret_cast<const v4f*>(X + base + k);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = x[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (r < rows && k + e < K) ? X[base + k + e] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) lds[kq + e][row] = v[e];
  }
}

template <bool VEC>
__global__ __launch_bounds__(256) void gemm_nt_kernel(const float* __restrict__ A, int64_t M, int64_t K, RowMap amap,
                                                      const float* __restrict__ B, int64_t N, int64_t ldb,
                                                      float* __restrict__ C, RowMap cmap, int accumulate,
                                                      int64_t n_tiles) {
  __shared__ float As[kK][kTM + 4];
  __shared__ float Bs[kK][kTN + 4];
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t bm = blockIdx.x / n_tiles, bn = blockIdx.x % n_tiles;
  const int64_t m0 = bm * kTM, n0 = bn * kTN;
  v4f acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int64_t k0 = 0; k0 < K; k0 += kK) {
    stage<kTM, VEC>(A, M, K, amap, m0, k0, As);
    stage<kTN, VEC>(B, N, K, RowMap{ldb, 1, ldb}, n0, k0, Bs);
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kK; kk += 4) {
      const int k = kk + (l >> 4);
      const float a0 = As[k][32 * w + (l & 15)], a1 = As[k][32 * w + 16 + (l & 15)];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float b = Bs[k][16 * j + (l & 15)];
        acc[0][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b, acc[0][j], 0, 0, 0);
        acc[1][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b, acc[1][j], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // D: lane holds rows 4 (l/16) + r of each 16-row block, column l % 16 of each 16-column block
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = n0 + 16 * j + (l & 15);
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + 32 * w + 16 * i + 4 * (l >> 4) + r;
        if (m < M) {
          float* c = C + cmap.off(m) + n;
          *c = accumulate ? *c + acc[i][j][r] : acc[i][j][r];
        }
      }
  }
}


// Split-bf16 form of the same product (FP32-level accuracy: each operand written as hi + mid + lo bf16
// parts, six products kept per pair, split_bf16.h) on v_mfma_f32_16x16x32_bf16 for K a multiple of 32:
// six 16x16x32 bf16 MFMAs replace eight 16x16x4 FP32 ones per 16x16x32 block, about 2.7x fewer MFMA
// cycles, for the large projections that are MFMA-bound in FP32.  Slabs are staged row-major
// ([row][k], float4 runs) and split in registers after the LDS read.
constexpr int kXK = 32;

__device__ __forceinline__ v4f mfma_bf16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ Split lds_split8(const float* p) {
  const v4f x0 = *reinterpret_cast<const v4f*>(p), x1 = *reinterpret_cast<const v4f*>(p + 4);
  float v[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = x0[e];
    v[4 + e] = x1[e];
  }
  return split8(v);
}

__global__ __launch_bounds__(256) void gemm_nt_x3_kernel(const float* __restrict__ A, int64_t M, int64_t K, RowMap amap,
                                                         const float* __restrict__ B, int64_t N, int64_t ldb,
                                                         float* __restrict__ C, RowMap cmap, int accumulate,
                                                         int64_t n_tiles) {
  __shared__ float As[kTM][kXK + 4];
  __shared__ float Bs[kTN][kXK + 4];
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t bm = blockIdx.x / n_tiles, bn = blockIdx.x % n_tiles;
  const int64_t m0 = bm * kTM, n0 = bn * kTN;
  v4f acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int64_t k0 = 0; k0 < K; k0 += kXK) {
#pragma unroll
    for (int q = 0; q < kTM * kXK / 4 / 256; ++q) {
      const int idx = threadIdx.x + 256 * q, row = idx / (kXK / 4), kq = 4 * (idx % (kXK / 4));
      const int64_t r = m0 + row;
      v4f v = v4f{0.f, 0.f, 0.f, 0.f};
      if (r < M) v = *reinterpret_cast<const v4f*>(A + amap.off(r) + k0 + kq);
      *reinterpret_cast<v4f*>(&As[row][kq]) = v;
    }
#pragma unroll
    for (int q = 0; q < kTN * kXK / 4 / 256; ++q) {
      const int idx = threadIdx.x + 256 * q, row = idx / (kXK / 4), kq = 4 * (idx % (kXK / 4));
      const int64_t r = n0 + row;
      v4f v = v4f{0.f, 0.f, 0.f, 0.f};
      if (r < N) v = *reinterpret_cast<const v4f*>(B + r * ldb + k0 + kq);
      *reinterpret_cast<v4f*>(&Bs[row][kq]) = v;
    }
    __syncthreads();
    // operands: lane l holds row / column l % 16 and k = 8 (l / 16) .. + 7 of the slab
    Split a[2], b[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) a[i] = lds_split8(&As[32 * w + 16 * i + (l & 15)][8 * (l >> 4)]);
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = lds_split8(&Bs[16 * j + (l & 15)][8 * (l >> 4)]);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // smallest products first: lo*hi, hi*lo, mid*mid, mid*hi, hi*mid, hi*hi
        acc[i][j] = mfma_bf16(a[i].lo, b[j].hi, acc[i][j]);
        acc[i][j] = mfma_bf16(a[i].hi, b[j].lo, acc[i][j]);
        acc[i][j] = mfma_bf16(a[i].mid, b[j].mid, acc[i][j]);
        acc[i][j] = mfma_bf16(a[i].mid, b[j].hi, acc[i][j]);
        acc[i][j] = mfma_bf16(a[i].hi, b[j].mid, acc[i][j]);
        acc[i][j] = mfma_bf16(a[i].hi, b[j].hi, acc[i][j]);
      }
    __syncthreads();
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t n = n0 + 16 * j + (l & 15);
    if (n >= N) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + 32 * w + 16 * i + 4 * (l >> 4) + r;
        if (m < M) {
          float* c = C + cmap.off(m) + n;
          *c = accumulate ? *c + acc[i][j][r] : acc[i][j][r];
        }
      }
  }
}

constexpr int kSumThreads = 256;

// First index i in [0, n) with batch[i] >= g (batch ascending).
__device__ int64_t lower_bound_graph(const int64_t* __restrict__ batch, int64_t n, int64_t g) {
  int64_t lo = 0, hi = n;
  while (lo < hi) {
    const int64_t mid = lo + ((hi - lo) >> 1);
    if (batch[mid] < g) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// One block per graph. Sorted batch: the block sums its own [begin, end) range, O(n + graphs) in all;
// unsorted batch: the block filters all n atoms, O(graphs * n). Same fixed summation order per thread
// slot in both (atom index ascending), then a fixed tree.
template <bool kSorted>
__global__ __launch_bounds__(kSumThreads) void graph_sum_kernel(const float* __restrict__ values,
                                                                const int64_t* __restrict__ batch, int64_t n,
                                                                double* __restrict__ out) {
  __shared__ double part[kSumThreads];
  __shared__ int64_t range[2];
  const int64_t b = blockIdx.x;
  int64_t begin = 0, end = n;
  if (kSorted) {
    if (threadIdx.x < 2) range[threadIdx.x] = lower_bound_graph(batch, n, b + threadIdx.x);
    __syncthreads();
    begin = range[0];
    end = range[1];
  }
  double s = 0.0;
  for (int64_t i = begin + threadIdx.x; i < end; i += kSumThreads)
    if (kSorted || batch[i] == b) s += (double)values[i];
  part[threadIdx.x] = s;
  __syncthreads();
  for (int h = kSumThreads / 2; h > 0; h >>= 1) {
    if ((int)threadIdx.x < h) part[threadIdx.x] += part[threadIdx.x + h];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[b] = part[0];
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return ICTC_OK;
  char buf[256];
  snprintf(buf, sizeof(buf), "%s: %s", what, hipGetErrorString(e));
  return fail(ICTC_ERR_RUNTIME, buf);
}

}  // namespace

namespace ictc {

// C (+)= A . B^T with A's and C's rows in groups (RowMap): row r of A at (r / a_group) * a_gstride +
// (r % a_group) * lda, likewise for C.  split != 0 takes the split-bf16 MFMA form where K is a multiple of
// 32 and the operands allow 16-byte loads.  Internal to the library (the species message's per-degree GEMMs).
int gemm_nt_grouped(const float* a, int64_t m, int64_t k, int64_t lda, int64_t a_group, int64_t a_gstride,
                    const float* b, int64_t n, int64_t ldb, float* c, int64_t ldc, int64_t c_group,
                    int64_t c_gstride, int accumulate, void* stream, int split) {
  if (m < 0 || n < 0 || k < 0 || lda < k || ldb < k || ldc < n || a_group < 1 || c_group < 1 || a_gstride < k ||
      c_gstride < n)
    return fail(ICTC_ERR_ARGUMENT, "gemm_nt: need m, n, k >= 0, lda >= k, ldb >= k, ldc >= n, groups >= 1");
  if ((a_group > 1 || c_group > 1) && m > INT32_MAX) return fail(ICTC_ERR_ARGUMENT, "gemm_nt: too many rows");
  if (m == 0 || n == 0) return ICTC_OK;
  if (!c || (k > 0 && (!a || !b))) return fail(ICTC_ERR_ARGUMENT, "gemm_nt: null operand");
  const int64_t mt = (m + kTM - 1) / kTM, nt = (n + kTN - 1) / kTN;
  if (mt * nt > INT32_MAX) return fail(ICTC_ERR_ARGUMENT, "gemm_nt: too many output tiles");
  const bool vec = lda % 4 == 0 && ldb % 4 == 0 && (a_group == 1 || a_gstride % 4 == 0) &&
                   ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
  const RowMap am{lda, a_group, a_gstride}, cm{ldc, c_group, c_gstride};
  if (split && vec && k % kXK == 0) {
    hipLaunchKernelGGL(gemm_nt_x3_kernel, dim3((unsigned)(mt * nt)), dim3(256), 0, (hipStream_t)stream, a, m, k, am, b,
                       n, ldb, c, cm, accumulate, nt);
    return launch_status("ictc_gemm_nt launch");
  }
  if (vec)
    hipLaunchKernelGGL(gemm_nt_kernel<true>, dim3((unsigned)(mt * nt)), dim3(256), 0, (hipStream_t)stream, a, m, k,
                       am, b, n, ldb, c, cm, accumulate, nt);
  else
    hipLaunchKernelGGL(gemm_nt_kernel<false>, dim3((unsigned)(mt * nt)), dim3(256), 0, (hipStream_t)stream, a, m, k,
                       am, b, n, ldb, c, cm, accumulate, nt);
  return launch_status("ictc_gemm_nt launch");
}

}  // namespace ictc

extern "C" {

int ictc_gemm_nt(const float* a, int64_t m, int64_t k, int64_t lda, const float* b, int64_t n, int64_t ldb, float* c,
                 int64_t ldc, int accumulate, void* stream) {
  if (m < 0 || n < 0 || k < 0 || lda < k || ldb < k || ldc < n)
    return fail(ICTC_ERR_ARGUMENT, "gemm_nt: need m, n, k >= 0, lda >= k, ldb >= k, ldc >= n");
  return ictc::gemm_nt_grouped(a, m, k, lda, 1, lda, b, n, ldb, c, ldc, 1, ldc, accumulate, stream, 0);
}

int ictc_graph_sum(const float* values, const int64_t* batch, int64_t n, int64_t graphs, int batch_sorted, double* out,
                   void* stream) {
  if (n < 0 || graphs < 0) return fail(ICTC_ERR_ARGUMENT, "graph_sum: negative size");
  if (graphs == 0) return ICTC_OK;
  if (!out || (n > 0 && (!values || !batch))) return fail(ICTC_ERR_ARGUMENT, "graph_sum: null operand");
  if (graphs > INT32_MAX) return fail(ICTC_ERR_ARGUMENT, "graph_sum: too many graphs");
  if (batch_sorted)
    hipLaunchKernelGGL(graph_sum_kernel<true>, dim3((unsigned)graphs), dim3(kSumThreads), 0, (hipStream_t)stream,
                       values, batch, n, out);
  else
    hipLaunchKernelGGL(graph_sum_kernel<false>, dim3((unsigned)graphs), dim3(kSumThreads), 0, (hipStream_t)stream,
                       values, batch, n, out);
  return launch_status("ictc_graph_sum launch");
}

}  // extern "C"
