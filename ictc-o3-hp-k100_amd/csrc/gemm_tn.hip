// Weight gradients of the per-edge linears: out[M, N] = A^T B, A [K, M] and
// B [K, N] row-major with K = edges (hundreds of thousands) and M, N the layer
// widths (8 .. a few thousand).  This is the dW = dy^T x of every Linear of
// the radial MLP `fc` (mace_ictc/models/mace/layers.py:826-835) in the
// force-loss training step, where autograd runs it through the library GEMM.
// With a 64 x 64 output the library tiles the output only (two workgroups
// for 424k reduction rows); here the reduction rows are split instead.
//
// Grid: (output tile of 64 x 64) x (chunk of reduction rows).  A block of 4
// waves stages 32-row slabs of A and B (64 columns each) through LDS with
// 256-byte coalesced loads, prefetching the next slab into registers while
// the MFMAs run on the current one.  The products run on bf16 MFMA with the
// three-way operand split (six v_mfma_f32_16x16x32_bf16 per 16x16x32 step,
// FP32-level accuracy): each slab is split once while it is staged, into
// hi / mid / lo planes stored reduction-index-contiguous, so every operand is
// one 16-byte LDS read.  Wave w owns output rows 16w .. 16w+15 of the tile and
// all four 16-column blocks.  (An FP32-MFMA form, v_mfma_f32_16x16x4_f32,
// measured 18-22 % slower even on single-tile 64 x 64 and 64 x 8 outputs over
// 848k rows, and 65 TFLOP/s on the wide ones.)  Each block writes its partial
// tile to the workspace; a second kernel adds the chunks of every output in a
// fixed order (chunks interleaved over 16 waves, the 16 wave sums combined in
// wave order), so the result does not depend on scheduling.
//
// Block order: the tiles of one chunk are consecutive logical blocks, and the
// logical range is split contiguously over the 8 XCDs, so the chunk's rows of
// the shared operand are fetched into one XCD's L2 and reused by its tiles.
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

constexpr int kTile = 64;
constexpr int kXcds = 8;
constexpr int kSumWaves = 16;

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

struct Plan {
  int mt, nt, chunks;
  int64_t rows;      // reduction rows per chunk (multiple of 32)
  int64_t blocks;    // launched blocks (logical count rounded up to a multiple of kXcds)
};

Plan plan_for(int64_t K, int M, int N) {
  Plan p;
  p.mt = (M + kTile - 1) / kTile;
  p.nt = (N + kTile - 1) / kTile;
  const int64_t tiles = (int64_t)p.mt * p.nt;
  const int64_t want = (int64_t)cu_count() * 8;          // about 8 blocks (32 waves) per CU
  int64_t chunks = (want + tiles - 1) / tiles;
  // Wide outputs: every tile of a chunk re-reads the chunk's rows of B, so keep the chunks an XCD runs at
  // once (about 160 blocks, i.e. 160 / tiles chunks) within its 4 MB L2: about 2,048 rows per chunk.
  if (tiles > 16 && chunks < (K + 2047) / 2048) chunks = (K + 2047) / 2048;
  const int64_t max_chunks = (K + 63) / 64;               // at least 64 rows per chunk
  if (chunks > max_chunks) chunks = max_chunks;
  if (chunks > 1024) chunks = 1024;
  if (chunks < 1) chunks = 1;
  int64_t rows = (K + chunks - 1) / chunks;
  rows = (rows + 31) / 32 * 32;   // whole 32-row slabs
  if (rows < 32) rows = 32;
  chunks = K > 0 ? (K + rows - 1) / rows : 1;
  p.chunks = (int)chunks;
  p.rows = rows;
  const int64_t logical = tiles * chunks;
  p.blocks = (logical + kXcds - 1) / kXcds * kXcds;
  return p;
}

// Operand addressing.  Dense row-major: element (r, c) at r * ldg + c.  With
// STRIDED, rows are (group, member) pairs and columns (block, offset) pairs:
// element (r, c) at (r / rg) * ldg + (r % rg) * ldr + (c / cg) * ldc + c % cg,
// e.g. the (node, component) rows and (path, channel) columns of one degree of
// a packed feature array.
struct Layout {
  int64_t ldg, ldr, ldc;
  int rg, cg;
};

template <bool STRIDED>
__device__ __forceinline__ int64_t col_offset(const Layout& L, int c) {
  return STRIDED ? (int64_t)(c / L.cg) * L.ldc + c % L.cg : c;
}

constexpr int kSlabB = 32;     // reduction rows per stage (one MFMA K)
constexpr int kPlanePitch = 40;  // bf16 per plane row: 32 + 8 (80 bytes: 16-byte reads of 8 rows hit distinct banks)

__device__ __forceinline__ v4f mfma16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// NJ: 16-column blocks of the tile computed (1 for outputs at most 16 wide, such as the 64 x 8 gradient of a
// radial MLP's first layer: the other three blocks would multiply zero columns).
template <bool STRIDED, int NJ>
__global__ __launch_bounds__(256) void gemm_tn_bf16_partial_kernel(const float* __restrict__ A, int64_t K, int M,
    Layout la, const float* __restrict__ B, int N, Layout lb, float* __restrict__ part, int mt,
                                                                   int nt, int chunks, int64_t rows, int64_t blocks) {
  const int64_t per = blocks / kXcds;
  const int64_t logical = (int64_t)(blockIdx.x % kXcds) * per + blockIdx.x / kXcds;
  const int64_t tiles = (int64_t)mt * nt;
  if (logical >= tiles * chunks) return;
  const int tile = (int)(logical % tiles);
  const int chunk = (int)(logical / tiles);
  const int m0 = (tile % mt) * kTile, n0 = (tile / mt) * kTile;
  const int64_t k0 = (int64_t)chunk * rows;
  const int64_t k1 = k0 + rows < K ? k0 + rows : K;

  // planes[operand][part][column][k]: column = m (A) or n (B) within the tile
  __shared__ __attribute__((aligned(16))) __bf16 planes[2][3][kTile][kPlanePitch];
  const int t = threadIdx.x, col = t & 63, r0 = t >> 6;   // staging: column col, slab rows 8 r0 .. 8 r0 + 7
  const int lane = t & 63, wave = t >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const bool a_col = m0 + col < M, b_col = n0 + col < N;
  const float* __restrict__ Ap = A + (a_col ? col_offset<STRIDED>(la, m0 + col) : 0);
  const float* __restrict__ Bp = B + (b_col ? col_offset<STRIDED>(lb, n0 + col) : 0);

  float ra[8], rb[8];
  auto load = [&](int64_t k) {
    // grouped rows: one division for the first row, then (group, member) steps (both operands share rg)
    uint32_t g = 0, i = 0;
    if (STRIDED) {
      const uint32_t u = (uint32_t)(k + 8 * r0);
      g = u / (uint32_t)la.rg;
      i = u - g * (uint32_t)la.rg;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t kr = k + 8 * r0 + e;
      const bool in = kr < k1;
      const int64_t oa = STRIDED ? (int64_t)g * la.ldg + (int64_t)i * la.ldr : kr * la.ldg;
      const int64_t ob = STRIDED ? (int64_t)g * lb.ldg + (int64_t)i * lb.ldr : kr * lb.ldg;
      ra[e] = (in && a_col) ? Ap[oa] : 0.f;
      rb[e] = (in && b_col) ? Bp[ob] : 0.f;
      if (STRIDED && ++i == (uint32_t)la.rg) {
        i = 0;
        ++g;
      }
    }
  };

  v4f acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
  if (k0 < k1) load(k0);
  for (int64_t k = k0; k < k1; k += kSlabB) {
    const Split sa = split8(ra), sb = split8(rb);
    __syncthreads();
    *reinterpret_cast<bf16x8*>(&planes[0][0][col][8 * r0]) = sa.hi;
    *reinterpret_cast<bf16x8*>(&planes[0][1][col][8 * r0]) = sa.mid;
    *reinterpret_cast<bf16x8*>(&planes[0][2][col][8 * r0]) = sa.lo;
    *reinterpret_cast<bf16x8*>(&planes[1][0][col][8 * r0]) = sb.hi;
    *reinterpret_cast<bf16x8*>(&planes[1][1][col][8 * r0]) = sb.mid;
    *reinterpret_cast<bf16x8*>(&planes[1][2][col][8 * r0]) = sb.lo;
    __syncthreads();
    if (k + kSlabB < k1) load(k + kSlabB);
    // A operand: row m = 16 wave + li, reduction rows 8 lg .. 8 lg + 7 of the slab
    const int am = 16 * wave + li;
    const bf16x8 ahi = *reinterpret_cast<const bf16x8*>(&planes[0][0][am][8 * lg]);
    const bf16x8 amid = *reinterpret_cast<const bf16x8*>(&planes[0][1][am][8 * lg]);
    const bf16x8 alo = *reinterpret_cast<const bf16x8*>(&planes[0][2][am][8 * lg]);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int bn = 16 * j + li;
      const bf16x8 bhi = *reinterpret_cast<const bf16x8*>(&planes[1][0][bn][8 * lg]);
      const bf16x8 bmid = *reinterpret_cast<const bf16x8*>(&planes[1][1][bn][8 * lg]);
      const bf16x8 blo = *reinterpret_cast<const bf16x8*>(&planes[1][2][bn][8 * lg]);
      acc[j] = mfma16(alo, bhi, acc[j]);
      acc[j] = mfma16(ahi, blo, acc[j]);
      acc[j] = mfma16(amid, bmid, acc[j]);
      acc[j] = mfma16(amid, bhi, acc[j]);
      acc[j] = mfma16(ahi, bmid, acc[j]);
      acc[j] = mfma16(ahi, bhi, acc[j]);
    }
  }

  float* __restrict__ P = part + (int64_t)chunk * M * N;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int n = n0 + 16 * j + li;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 16 * wave + 4 * lg + r;
      if (m < M && n < N) P[(int64_t)m * N + n] = acc[j][r];
    }
  }
}

// out[i] = sum over chunks of part[c][i]: wave w of a block adds chunks
// w, w + 16, ... for 64 consecutive outputs; the wave sums meet in LDS and
// are added in wave order.
__global__ __launch_bounds__(64 * kSumWaves) void gemm_tn_sum_kernel(const float* __restrict__ part, int64_t n,
                                                                     int chunks, float* __restrict__ out) {
  __shared__ float red[kSumWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t i = (int64_t)blockIdx.x * 64 + lane;
  // four independent partial sums (chunks w + 64 q + 16 j go to sum j), added in a fixed order, so four
  // loads are in flight per lane instead of one
  float v = 0.f;
  if (i < n) {
    float v0 = 0.f, v1 = 0.f, v2 = 0.f, v3 = 0.f;
    const float* __restrict__ p = part + i;
    int c = wave;
    for (; c + 3 * kSumWaves < chunks; c += 4 * kSumWaves) {
      v0 += p[(int64_t)c * n];
      v1 += p[(int64_t)(c + kSumWaves) * n];
      v2 += p[(int64_t)(c + 2 * kSumWaves) * n];
      v3 += p[(int64_t)(c + 3 * kSumWaves) * n];
    }
    for (; c < chunks; c += kSumWaves) v0 += p[(int64_t)c * n];
    v = (v0 + v1) + (v2 + v3);
  }
  red[wave][lane] = v;
  __syncthreads();
  if (wave == 0 && i < n) {
    float s = red[0][lane];
#pragma unroll
    for (int w = 1; w < kSumWaves; ++w) s += red[w][lane];
    out[i] = s;
  }
}

int gemm_tn_launch(const float* a, const Layout& la, int64_t k, int64_t m, const float* b, const Layout& lb,
                   int64_t n, bool strided, float* out, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!out || (k > 0 && (!a || !b))) return fail(ICTC_ERR_ARGUMENT, "gemm_tn: null operand");
  const Plan p = plan_for(k, (int)m, (int)n);
  const int64_t need = (int64_t)p.chunks * m * n * (int64_t)sizeof(float);
  if (!workspace || workspace_bytes < need)
    return fail(ICTC_ERR_ARGUMENT, "gemm_tn: workspace smaller than ictc_gemm_tn_workspace_bytes");
  float* part = static_cast<float*>(workspace);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)p.blocks), block(256);
#define ICTC_TN_LAUNCH(S, NJ)                                                                                \
  hipLaunchKernelGGL((gemm_tn_bf16_partial_kernel<S, NJ>), grid, block, 0, st, a, k, (int)m, la, b, (int)n, lb, part, \
                     p.mt, p.nt, p.chunks, p.rows, p.blocks)
  if (strided && n <= 16)
    ICTC_TN_LAUNCH(true, 1);
  else if (strided)
    ICTC_TN_LAUNCH(true, 4);
  else if (n <= 16)
    ICTC_TN_LAUNCH(false, 1);
  else
    ICTC_TN_LAUNCH(false, 4);
#undef ICTC_TN_LAUNCH
  const int64_t total = m * n;
  hipLaunchKernelGGL(gemm_tn_sum_kernel, dim3((unsigned)((total + 63) / 64)), dim3(64 * kSumWaves), 0, st, part,
                     total, p.chunks, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof(buf), "ictc_gemm_tn launch: %s", hipGetErrorString(e));
    return fail(ICTC_ERR_RUNTIME, buf);
  }
  return ICTC_OK;
}

}  // namespace

extern "C" {

int64_t ictc_gemm_tn_workspace_bytes(int64_t k, int64_t m, int64_t n) {
  if (k < 0 || m <= 0 || n <= 0 || m > (1 << 20) || n > (1 << 20)) return -1;
  const Plan p = plan_for(k, (int)m, (int)n);
  return (int64_t)p.chunks * m * n * (int64_t)sizeof(float);
}

int ictc_gemm_tn(const float* a, int64_t k, int64_t m, int64_t lda, const float* b, int64_t n, int64_t ldb,
                 float* out, void* workspace, int64_t workspace_bytes, void* stream) {
  if (k < 0 || m <= 0 || n <= 0 || m > (1 << 20) || n > (1 << 20) || lda < m || ldb < n)
    return fail(ICTC_ERR_ARGUMENT, "gemm_tn: need k >= 0, 0 < m, n <= 2^20, lda >= m, ldb >= n");
  const Layout la{lda, 0, 0, 1, 1 << 30}, lb{ldb, 0, 0, 1, 1 << 30};
  return gemm_tn_launch(a, la, k, m, b, lb, n, false, out, workspace, workspace_bytes, stream);
}

int ictc_gemm_tn_grouped(const float* a, int64_t a_ldg, int64_t a_ldr, int a_cg, int64_t a_ldc, const float* b,
                         int64_t b_ldg, int64_t b_ldr, int b_cg, int64_t b_ldc, int64_t groups, int rows_per_group,
                         int64_t m, int64_t n, float* out, void* workspace, int64_t workspace_bytes, void* stream) {
  const int64_t k = groups * (int64_t)rows_per_group;
  if (groups < 0 || rows_per_group <= 0 || m <= 0 || n <= 0 || m > (1 << 20) || n > (1 << 20) || a_cg <= 0 ||
      b_cg <= 0 || k >= ((int64_t)1 << 31))
    return fail(ICTC_ERR_ARGUMENT, "gemm_tn_grouped: invalid sizes (rows below 2^31, 0 < m, n <= 2^20)");
  const Layout la{a_ldg, a_ldr, a_ldc, rows_per_group, a_cg}, lb{b_ldg, b_ldr, b_ldc, rows_per_group, b_cg};
  return gemm_tn_launch(a, la, k, m, b, lb, n, true, out, workspace, workspace_bytes, stream);
}

}  // extern "C"
