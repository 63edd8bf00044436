// Fused radial MLP on MFMA (gfx950): Bessel x polynomial-cutoff radial basis,
// then three bias-free 64-wide hidden layers with normalized SiLU
// (mace_ictc/models/mace/layers.py:826-835 `fc` without its last Linear,
// radial_basis.py:11-92), forward and the first adjoint down to d/dr.
//
// Tiling: a wave owns 16 edges; a block of 4 waves owns 64 edges.  Each
// 16 x 64 x K product is a chain of v_mfma_f32_16x16x4_f32 (A 16x4, B 4x16,
// C/D 16x16, FP32 in and out).  Operand layouts for lane l (l = 0..63):
//   A[i][k]: i = l % 16, k = l / 16          B[k][j]: k = l / 16, j = l % 16
//   D[i][j]: j = l % 16, i = 4 * (l / 16) + r for the lane's 4 registers r.
// D -> A re-layout between layers goes through a per-wave LDS tile.  The
// weights of the three hidden layers are staged in LDS once per block.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/ictc_mi355x.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int H = 64;        // hidden width (compiled for 64)
constexpr int KB = 8;        // radial basis size (compiled for 8)
constexpr int EW = 16;       // edges per wave
constexpr int WAVES = 4;
constexpr int EB = EW * WAVES;
constexpr int LD = H + 1;    // padded LDS row

__device__ __forceinline__ v4f mfma(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float sigm(float x) { return 1.f / (1.f + expf(-x)); }

struct Radial {
  float pre, rc, c1, c2, c3;
  int p;
};

__device__ __forceinline__ Radial radial_consts(float rc, int p) {
  Radial q;
  q.pre = sqrtf(2.f / rc);
  q.rc = rc;
  q.c1 = 0.5f * (p + 1) * (p + 2);
  q.c2 = (float)p * (p + 2);
  q.c3 = 0.5f * p * (p + 1);
  q.p = p;
  return q;
}

// b_k(r) (and optionally db_k/dr) for k = 1..KB.
__device__ __forceinline__ void radial_basis(const Radial& q, float x, float* b, float* db) {
  const bool inside = x < q.rc;
  const float u = x / q.rc;
  const float up = powf(u, (float)q.p);
  const float upm1 = powf(u, (float)(q.p - 1));
  const float env = inside ? 1.f - q.c1 * up + q.c2 * up * u - q.c3 * up * u * u : 0.f;
  const float denv = inside ? (-q.c1 * q.p * upm1 + q.c2 * (q.p + 1) * up - q.c3 * (q.p + 2) * up * u) / q.rc : 0.f;
  const float xr = fmaxf(x, 1e-12f), inv = 1.f / xr;
#pragma unroll
  for (int k = 1; k <= KB; ++k) {
    const float w = k * 3.14159265358979323846f / q.rc;
    float sn, cs;
    sincosf(w * x, &sn, &cs);
    const float f = q.pre * sn * inv;
    b[k - 1] = f * env;
    if (db) db[k - 1] = q.pre * (w * cs * inv - sn * inv * inv) * env + f * denv;
  }
}

// Stage W (row-major [H, K]) transposed into LDS: wt[k][j] = W[j][k].
__device__ __forceinline__ void stage_t(float (*wt)[LD], const float* __restrict__ W, int K) {
  for (int i = threadIdx.x; i < H * K; i += blockDim.x) {
    const int j = i / K, k = i % K;
    wt[k][j] = W[i];
  }
}

// Stage W row-major into LDS: w[j][k] = W[j][k].
__device__ __forceinline__ void stage(float (*w)[LD], const float* __restrict__ W) {
  for (int i = threadIdx.x; i < H * H; i += blockDim.x) w[i / H][i % H] = W[i];
}

// D (16 x 64, four v4f blocks) = A_tile (16 x 64, LDS rows) @ B (64 x 64, LDS [k][j]).
__device__ __forceinline__ void gemm16x64x64(const float (*a)[LD], const float (*b)[LD], v4f* acc) {
  const int l = threadIdx.x & 63, i = l & 15, kq = l >> 4;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int kk = 0; kk < H / 4; ++kk) {
    const float av = a[i][4 * kk + kq];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[nb] = mfma(av, b[4 * kk + kq][16 * nb + i], acc[nb]);
  }
}

// Store a D-layout tile into LDS rows.
__device__ __forceinline__ void d_to_lds(float (*t)[LD], const v4f* d) {
  const int l = threadIdx.x & 63, j = l & 15, i0 = 4 * (l >> 4);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int r = 0; r < 4; ++r) t[i0 + r][16 * nb + j] = d[nb][r];
}

__device__ __forceinline__ void d_store(float* __restrict__ out, int64_t e0, int64_t E, const v4f* d) {
  const int l = threadIdx.x & 63, j = l & 15, i0 = 4 * (l >> 4);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t e = e0 + i0 + r;
    if (e < E) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) out[e * H + 16 * nb + j] = d[nb][r];
    }
  }
}

__device__ __forceinline__ void d_load(const float* __restrict__ in, int64_t e0, int64_t E, v4f* d) {
  const int l = threadIdx.x & 63, j = l & 15, i0 = 4 * (l >> 4);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t e = e0 + i0 + r;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) d[nb][r] = e < E ? in[e * H + 16 * nb + j] : 0.f;
  }
}

// Forward: z1 = R W1^T, a1 = s silu(z1), z2 = a1 W2^T, a2, z3 = a2 W3^T, a3 = s silu(z3).
// Writes z1, z2, z3 (pre-activations, for the adjoint) and a3.
__global__ __launch_bounds__(256) void mlp_fwd_kernel(const float* __restrict__ r, int64_t E, float rc, int p,
                                                      const float* __restrict__ W1, const float* __restrict__ W2,
                                                      const float* __restrict__ W3, float s,
                                                      float* __restrict__ z1, float* __restrict__ z2,
                                                      float* __restrict__ z3, float* __restrict__ a3) {
  __shared__ float w1t[KB][LD];
  __shared__ float w2t[H][LD];
  __shared__ float w3t[H][LD];
  __shared__ float tile[WAVES][EW][LD];
  stage_t(w1t, W1, KB);
  stage_t(w2t, W2, H);
  stage_t(w3t, W3, H);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, i = l & 15, kq = l >> 4;
  const int64_t e0 = ((int64_t)blockIdx.x * WAVES + w) * EW;
  const Radial q = radial_consts(rc, p);
  if (l < EW) {
    float b[KB];
    const int64_t e = e0 + l;
    radial_basis(q, e < E ? r[e] : 2.f * rc, b, nullptr);
#pragma unroll
    for (int k = 0; k < KB; ++k) tile[w][l][k] = b[k];
  }
  __syncthreads();
  v4f acc[4];
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < KB / 4; ++kk) {
    const float av = tile[w][i][4 * kk + kq];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[nb] = mfma(av, w1t[4 * kk + kq][16 * nb + i], acc[nb]);
  }
  d_store(z1, e0, E, acc);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[nb][t] = s * acc[nb][t] * sigm(acc[nb][t]);
  __syncthreads();
  d_to_lds(tile[w], acc);
  __syncthreads();
  gemm16x64x64(tile[w], w2t, acc);
  d_store(z2, e0, E, acc);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[nb][t] = s * acc[nb][t] * sigm(acc[nb][t]);
  __syncthreads();
  d_to_lds(tile[w], acc);
  __syncthreads();
  gemm16x64x64(tile[w], w3t, acc);
  d_store(z3, e0, E, acc);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[nb][t] = s * acc[nb][t] * sigm(acc[nb][t]);
  d_store(a3, e0, E, acc);
}

// s silu'(z) = s sig(z) (1 + z (1 - sig(z)))
__device__ __forceinline__ float dact(float z, float s) {
  const float g = sigm(z);
  return s * g * (1.f + z * (1.f - g));
}

// Adjoint: given da3, returns dr (and dz1..dz3 when non-null, for weight gradients).
__global__ __launch_bounds__(256) void mlp_bwd_kernel(const float* __restrict__ r, int64_t E, float rc, int p,
                                                      const float* __restrict__ W1, const float* __restrict__ W2,
                                                      const float* __restrict__ W3, float s,
                                                      const float* __restrict__ z1, const float* __restrict__ z2,
                                                      const float* __restrict__ z3, const float* __restrict__ da3,
                                                      float* __restrict__ dr, float* __restrict__ dz1,
                                                      float* __restrict__ dz2, float* __restrict__ dz3) {
  __shared__ float w1[H][KB + 1];
  __shared__ float w2[H][LD];
  __shared__ float w3[H][LD];
  __shared__ float tile[WAVES][EW][LD];
  for (int t = threadIdx.x; t < H * KB; t += blockDim.x) w1[t / KB][t % KB] = W1[t];
  stage(w2, W2);
  stage(w3, W3);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int64_t e0 = ((int64_t)blockIdx.x * WAVES + w) * EW;
  v4f g[4], z[4];
  // dz3 = da3 * s silu'(z3)
  d_load(da3, e0, E, g);
  d_load(z3, e0, E, z);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) g[nb][t] *= dact(z[nb][t], s);
  if (dz3) d_store(dz3, e0, E, g);
  __syncthreads();
  d_to_lds(tile[w], g);
  __syncthreads();
  gemm16x64x64(tile[w], w3, g);      // da2 = dz3 W3  (B[k][j] = W3[k][j])
  d_load(z2, e0, E, z);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) g[nb][t] *= dact(z[nb][t], s);
  if (dz2) d_store(dz2, e0, E, g);
  __syncthreads();
  d_to_lds(tile[w], g);
  __syncthreads();
  gemm16x64x64(tile[w], w2, g);      // da1 = dz2 W2
  d_load(z1, e0, E, z);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) g[nb][t] *= dact(z[nb][t], s);
  if (dz1) d_store(dz1, e0, E, g);
  __syncthreads();
  d_to_lds(tile[w], g);
  __syncthreads();
  // dR = dz1 W1 (16 x 8) and dr = sum_k dR_k b_k'(r): lanes 0..15, one edge each
  if (l < EW) {
    const int64_t e = e0 + l;
    if (e < E) {
      float b[KB], db[KB];
      const Radial q = radial_consts(rc, p);
      radial_basis(q, r[e], b, db);
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < KB; ++k) {
        float dRk = 0.f;
        for (int j = 0; j < H; ++j) dRk = fmaf(tile[w][l][j], w1[j][k], dRk);
        acc = fmaf(dRk, db[k], acc);
      }
      dr[e] = acc;
    }
  }
}

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return ICTC_OK;
  char buf[256];
  snprintf(buf, sizeof(buf), "%s: %s", what, hipGetErrorString(e));
  return fail(ICTC_ERR_RUNTIME, buf);
}

}  // namespace

extern "C" {

int ictc_radial_mlp_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                        const float* W1, const float* W2, const float* W3, float silu_scale, float* z1, float* z2,
                        float* z3, float* a3, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 1) return fail(ICTC_ERR_ARGUMENT, "radial MLP: invalid arguments");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !z1 || !z2 || !z3 || !a3) return fail(ICTC_ERR_ARGUMENT, "radial MLP: null operand");
  const unsigned blocks = (unsigned)((edges + EB - 1) / EB);
  hipLaunchKernelGGL(mlp_fwd_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, r, edges, cutoff, poly_p, W1,
                     W2, W3, silu_scale, z1, z2, z3, a3);
  return launch_status("ictc_radial_mlp_fwd launch");
}

int ictc_radial_mlp_bwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                        const float* W1, const float* W2, const float* W3, float silu_scale, const float* z1,
                        const float* z2, const float* z3, const float* da3, float* dr, float* dz1, float* dz2,
                        float* dz3, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 1) return fail(ICTC_ERR_ARGUMENT, "radial MLP: invalid arguments");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !z1 || !z2 || !z3 || !da3 || !dr)
    return fail(ICTC_ERR_ARGUMENT, "radial MLP: null operand");
  const unsigned blocks = (unsigned)((edges + EB - 1) / EB);
  hipLaunchKernelGGL(mlp_bwd_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, r, edges, cutoff, poly_p, W1,
                     W2, W3, silu_scale, z1, z2, z3, da3, dr, dz1, dz2, dz3);
  return launch_status("ictc_radial_mlp_bwd launch");
}

}  // extern "C"
