// Element-conditioned self connection (ElementConditionedLinearSO3, layers.py:21-87) over species-sorted
// node tiles: out[n] = M_s x[n] with s = species[n] and M_s = W[s] ([C, C], output by input) or its
// transpose (the input adjoint), and the weight gradient dW[s] = sum over the nodes of species s of
// a[n] b[n]^T.
//
// The caller passes the nodes in species order (perm: node ids sorted by species, stable; off[s] ..
// off[s + 1] the sorted range of species s; group S, the last, holds nodes whose species is outside
// [0, S)).  A tile is a run of sorted rows of ONE species, so a block stages that species' weights in LDS
// once and every row of the tile uses them: each product is formed once per node, where one GEMM over all
// species' weights followed by a gather forms S of them.  The tile list is implicit: block b walks the
// group sizes to find its (species, first row), so no host sync is needed to size anything.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ictc_mi355x.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kRows = 64;   // sorted rows per tile of the product kernel (4 waves x 16)
constexpr int kCols = 64;   // output columns per block
constexpr int kKs = 32;     // rows per LDS stage of the outer-product kernel

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

// Tile `b` of groups 0..G-1 cut into runs of `rows`: its group, first sorted row and row count.  Returns
// false past the last tile.
__device__ __forceinline__ bool find_tile(const int* __restrict__ off, int G, int rows, int b, int& grp, int& start,
                                          int& cnt) {
  int t = b;
  for (int s = 0; s < G; ++s) {
    const int lo = off[s], n = off[s + 1] - lo;
    const int tiles = (n + rows - 1) / rows;
    if (t < tiles) {
      grp = s;
      start = lo + t * rows;
      cnt = min(rows, n - t * rows);
      return true;
    }
    t -= tiles;
  }
  return false;
}

// out[perm[r]] (columns c0 .. c0 + 64) = M_s x[perm[r]] for the tile's rows; wave w takes rows 16w ..
// 16w + 15 on FP32 MFMA with reduction index b = (lane / 16) * C / 4 + ks, so each lane reads one
// contiguous run of its node's row and of the LDS weight row.
template <int C, bool TRANS>
__global__ __launch_bounds__(256) void species_apply_kernel(const float* __restrict__ x, int64_t ldx,
                                                            const float* __restrict__ W, int S,
                                                            const int* __restrict__ perm, const int* __restrict__ off,
                                                            float* __restrict__ out, int64_t ldo) {
  constexpr int KR = C / 4;
  constexpr int NB = kCols / 16;
  __shared__ float Ms[kCols][C + 4];
  int s, start, cnt;
  if (!find_tile(off, S + 1, kRows, blockIdx.x, s, start, cnt)) return;
  const int c0 = blockIdx.y * kCols;
  const int l = threadIdx.x & 63, li = l & 15, g = l >> 4, w = threadIdx.x >> 6;
  if (s == S) {   // species outside [0, S): zero rows
    for (int i = threadIdx.x; i < cnt * kCols; i += 256) {
      const int r = i / kCols, c = i % kCols;
      out[(int64_t)perm[start + r] * ldo + c0 + c] = 0.f;
    }
    return;
  }
  const float* Wb = W + (int64_t)s * C * C;
  for (int i = threadIdx.x; i < kCols * C; i += 256) {
    if (!TRANS) {
      const int a = i / C, k = i % C;
      Ms[a][k] = Wb[(int64_t)(c0 + a) * C + k];
    } else {
      const int k = i / kCols, a = i % kCols;
      Ms[a][k] = Wb[(int64_t)k * C + c0 + a];
    }
  }
  __syncthreads();
  if (16 * w >= cnt) return;
  const int row = 16 * w + li;
  const bool ok = row < cnt;
  const int64_t node = ok ? perm[start + row] : 0;
  float xa[KR];
  const float* xp = x + node * ldx + g * KR;
#pragma unroll
  for (int q = 0; q < KR / 4; ++q) {
    const v4f v = ok ? *reinterpret_cast<const v4f*>(xp + 4 * q) : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) xa[4 * q + e] = v[e];
  }
  v4f acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    acc[nb] = v4f{0.f, 0.f, 0.f, 0.f};
    const float* mp = &Ms[16 * nb + li][g * KR];
#pragma unroll
    for (int q = 0; q < KR / 4; ++q) {
      const v4f m = *reinterpret_cast<const v4f*>(mp + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[4 * q + e], m[e], acc[nb], 0, 0, 0);
    }
  }
  // lane holds tile rows 16w + 4g + r, column 16 nb + li of each block
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int tr = 16 * w + 4 * g + r;
    if (tr < cnt) {
      float* op = out + (int64_t)perm[start + tr] * ldo + c0 + li;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) op[16 * nb] = acc[nb][r];
    }
  }
}

// Partial of dW[s] (rows a0 .. a0 + 64, columns b0 .. b0 + 64) over one tile of species-s rows:
// ws[tile][a][b] = sum_r A[perm[r]][a] B[perm[r]][b], rows staged 32 at a time in LDS; wave w owns the
// 32 x 32 quarter (w / 2, w % 2) as 2 x 2 MFMA blocks.
template <int C>
__global__ __launch_bounds__(256) void species_outer_partial_kernel(const float* __restrict__ A, int64_t lda,
                                                                    const float* __restrict__ B, int64_t ldb, int S,
                                                                    const int* __restrict__ perm,
                                                                    const int* __restrict__ off, int rows,
                                                                    float* __restrict__ ws) {
  constexpr int OT = C / kCols;   // output tiles per side
  __shared__ float As[kKs][kCols + 4];
  __shared__ float Bs[kKs][kCols + 4];
  int s, start, cnt;
  if (!find_tile(off, S, rows, blockIdx.x, s, start, cnt)) return;
  const int a0 = (blockIdx.y / OT) * kCols, b0 = (blockIdx.y % OT) * kCols;
  const int l = threadIdx.x & 63, li = l & 15, g = l >> 4, w = threadIdx.x >> 6;
  const int wa = (w >> 1) * 32, wb = (w & 1) * 32;
  v4f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int k0 = 0; k0 < cnt; k0 += kKs) {
    // 32 rows x 64 columns of each operand: thread t stages two float4 runs of each
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int idx = threadIdx.x + 256 * q;
      const int kr = idx / (kCols / 4), c = 4 * (idx % (kCols / 4));
      v4f va = v4f{0.f, 0.f, 0.f, 0.f}, vb = va;
      if (k0 + kr < cnt) {
        const int64_t node = perm[start + k0 + kr];
        va = *reinterpret_cast<const v4f*>(A + node * lda + a0 + c);
        vb = *reinterpret_cast<const v4f*>(B + node * ldb + b0 + c);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        As[kr][c + e] = va[e];
        Bs[kr][c + e] = vb[e];
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kKs; kk += 4) {
      const int k = kk + g;
      const float x0 = As[k][wa + li], x1 = As[k][wa + 16 + li];
      const float y0 = Bs[k][wb + li], y1 = Bs[k][wb + 16 + li];
      acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0, y0, acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(x0, y1, acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1, y0, acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(x1, y1, acc[1][1], 0, 0, 0);
    }
    __syncthreads();
  }
  float* wp = ws + (int64_t)blockIdx.x * C * C;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        wp[(int64_t)(a0 + wa + 16 * i + 4 * g + r) * C + b0 + wb + 16 * j + li] = acc[i][j][r];
}

// out[s][e] = sum of ws[t][e] over species s's tiles in tile order (zero for a species with no nodes).
__global__ __launch_bounds__(256) void species_outer_sum_kernel(const float* __restrict__ ws, int64_t CC,
                                                                const int* __restrict__ off, int rows,
                                                                float* __restrict__ out) {
  const int s = blockIdx.y;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= CC) return;
  int t0 = 0;
  for (int q = 0; q < s; ++q) t0 += (off[q + 1] - off[q] + rows - 1) / rows;
  const int nt = (off[s + 1] - off[s] + rows - 1) / rows;
  float acc = 0.f;
  for (int t = 0; t < nt; ++t) acc += ws[(int64_t)(t0 + t) * CC + e];
  out[(int64_t)s * CC + e] = acc;
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return ICTC_OK;
  return fail(ICTC_ERR_RUNTIME, what);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int64_t outer_tiles(int64_t nodes, int species_count, int rows) { return (nodes + rows - 1) / rows + species_count; }

}  // namespace

extern "C" {

int ictc_species_linear(const float* x, int64_t ldx, int64_t nodes, int channels, const float* W, int species_count,
                        const int32_t* perm, const int32_t* offsets, int transpose, float* out, int64_t ldo,
                        void* stream) {
  if (nodes < 0 || nodes > INT32_MAX || species_count <= 0 || ldx < channels || ldo < channels || ldx % 4)
    return fail(ICTC_ERR_ARGUMENT, "species_linear: invalid sizes (row pitches >= channels, input pitch a multiple of 4)");
  if (channels != 64 && channels != 128)
    return fail(ICTC_ERR_UNSUPPORTED, "species_linear: compiled for 64 and 128 channels");
  if (nodes == 0) return ICTC_OK;
  if (!x || !W || !perm || !offsets || !out) return fail(ICTC_ERR_ARGUMENT, "species_linear: null operand");
  if (!aligned16(x) || !aligned16(W)) return fail(ICTC_ERR_ARGUMENT, "species_linear: x and W must be 16-byte aligned");
  const dim3 grid((unsigned)((nodes + kRows - 1) / kRows + species_count + 1), (unsigned)(channels / kCols));
  hipStream_t st = (hipStream_t)stream;
  const int* p = reinterpret_cast<const int*>(perm);
  const int* o = reinterpret_cast<const int*>(offsets);
  if (channels == 64) {
    if (transpose)
      hipLaunchKernelGGL((species_apply_kernel<64, true>), grid, dim3(256), 0, st, x, ldx, W, species_count, p, o, out, ldo);
    else
      hipLaunchKernelGGL((species_apply_kernel<64, false>), grid, dim3(256), 0, st, x, ldx, W, species_count, p, o, out, ldo);
  } else {
    if (transpose)
      hipLaunchKernelGGL((species_apply_kernel<128, true>), grid, dim3(256), 0, st, x, ldx, W, species_count, p, o, out, ldo);
    else
      hipLaunchKernelGGL((species_apply_kernel<128, false>), grid, dim3(256), 0, st, x, ldx, W, species_count, p, o, out, ldo);
  }
  return launch_status("ictc_species_linear launch");
}

int64_t ictc_species_outer_workspace_bytes(int64_t nodes, int channels, int species_count, int rows_per_tile) {
  if (nodes < 0 || species_count <= 0 || rows_per_tile <= 0 || rows_per_tile % kKs) return -1;
  return outer_tiles(nodes, species_count, rows_per_tile) * channels * channels * (int64_t)sizeof(float);
}

int ictc_species_outer(const float* a, int64_t lda, const float* b, int64_t ldb, int64_t nodes, int channels,
                       int species_count, const int32_t* perm, const int32_t* offsets, int rows_per_tile, float* out,
                       void* workspace, int64_t workspace_bytes, void* stream) {
  if (nodes < 0 || nodes > INT32_MAX || species_count <= 0 || lda < channels || ldb < channels || lda % 4 || ldb % 4)
    return fail(ICTC_ERR_ARGUMENT, "species_outer: invalid sizes (row pitches >= channels, multiples of 4)");
  if (channels != 64 && channels != 128)
    return fail(ICTC_ERR_UNSUPPORTED, "species_outer: compiled for 64 and 128 channels");
  if (rows_per_tile <= 0 || rows_per_tile % kKs)
    return fail(ICTC_ERR_ARGUMENT, "species_outer: rows_per_tile must be a positive multiple of 32");
  if (!a || !b || !perm || !offsets || !out) return fail(ICTC_ERR_ARGUMENT, "species_outer: null operand");
  if (!aligned16(a) || !aligned16(b)) return fail(ICTC_ERR_ARGUMENT, "species_outer: a and b must be 16-byte aligned");
  const int64_t tiles = outer_tiles(nodes, species_count, rows_per_tile);
  if (!workspace || workspace_bytes < tiles * channels * channels * (int64_t)sizeof(float))
    return fail(ICTC_ERR_ARGUMENT, "species_outer: workspace smaller than ictc_species_outer_workspace_bytes");
  hipStream_t st = (hipStream_t)stream;
  const int* p = reinterpret_cast<const int*>(perm);
  const int* o = reinterpret_cast<const int*>(offsets);
  float* ws = static_cast<float*>(workspace);
  const int ot = channels / kCols;
  const dim3 grid((unsigned)tiles, (unsigned)(ot * ot));
  if (channels == 64)
    hipLaunchKernelGGL(species_outer_partial_kernel<64>, grid, dim3(256), 0, st, a, lda, b, ldb, species_count, p, o,
                       rows_per_tile, ws);
  else
    hipLaunchKernelGGL(species_outer_partial_kernel<128>, grid, dim3(256), 0, st, a, lda, b, ldb, species_count, p, o,
                       rows_per_tile, ws);
  const int64_t cc = (int64_t)channels * channels;
  hipLaunchKernelGGL(species_outer_sum_kernel, dim3((unsigned)((cc + 255) / 256), (unsigned)species_count), dim3(256),
                     0, st, ws, cc, o, rows_per_tile, out);
  return launch_status("ictc_species_outer launch");
}

}  // extern "C"
