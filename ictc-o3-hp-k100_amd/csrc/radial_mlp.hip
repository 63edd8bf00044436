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
constexpr int LA = H + 2;    // activation tile row: A-operand reads (row l%16, col l/16) conflict free
constexpr int LW = H + 17;   // weight tile row: row- and column-wise operand reads nearly conflict free

__device__ __forceinline__ v4f mfma(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Logistic function on the hardware exp2/reciprocal (1 ulp each); saturates cleanly
// (x -> -inf: exp2 -> inf, rcp -> 0; x -> +inf: exp2 -> 0, rcp -> 1).
__device__ __forceinline__ float sigm(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.44269504088896341f * x));
}

__device__ __forceinline__ float ipow(float u, int p) {
  float v = 1.f;
  for (int t = 0; t < p; ++t) v *= u;
  return v;
}

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

// b_k(r) and db_k/dr for one basis index k (1-based).
__device__ __forceinline__ void radial_one(const Radial& q, float x, int k, float& b, float& db) {
  const bool inside = x < q.rc;
  const float u = x / q.rc;
  const float upm1 = ipow(u, q.p - 1);
  const float up = upm1 * u;
  const float env = inside ? 1.f - q.c1 * up + q.c2 * up * u - q.c3 * up * u * u : 0.f;
  const float denv = inside ? (-q.c1 * q.p * upm1 + q.c2 * (q.p + 1) * up - q.c3 * (q.p + 2) * up * u) / q.rc : 0.f;
  const float xr = fmaxf(x, 1e-12f), inv = 1.f / xr;
  const float w = k * 3.14159265358979323846f / q.rc;
  float sn, cs;
  sincosf(w * x, &sn, &cs);
  const float f = q.pre * sn * inv;
  b = f * env;
  db = q.pre * (w * cs * inv - sn * inv * inv) * env + f * denv;
}

// Radial basis of the wave's 16 edges into tile rows (b) and optionally dbt (db/dr):
// lane l handles edge l % 16 and basis functions 2*(l/16), 2*(l/16)+1.
__device__ __forceinline__ void radial_tile(const Radial& q, const float* __restrict__ r, int64_t e0, int64_t E,
                                            float (*tile)[LA], float (*dbt)[KB]) {
  const int l = threadIdx.x & 63, i = l & 15, kq = l >> 4;
  const int64_t e = e0 + i;
  const float x = e < E ? r[e] : 2.f * q.rc;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int k = 2 * kq + t;
    float b, db;
    radial_one(q, x, k + 1, b, db);
    tile[i][k] = b;
    if (dbt) dbt[i][k] = db;
  }
}

// Stage W (row-major [H, K], nn.Linear layout) transposed: wt[k][j] = W[j][k].
__device__ __forceinline__ void stage_t(float (*wt)[LW], const float* __restrict__ W, int K) {
  for (int t = threadIdx.x; t < H * K; t += blockDim.x) wt[t % K][t / K] = W[t];
}

// acc (16 x 64) = A (LDS activation tile, 16 x 64) @ B with B[k][j] = wt[k][j] (transposed weight).
__device__ __forceinline__ void gemm_fwd(const float (*a)[LA], const float (*wt)[LW], v4f* acc) {
  const int l = threadIdx.x & 63, i = l & 15, kq = l >> 4;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int kk = 0; kk < H / 4; ++kk) {
    const float av = a[i][4 * kk + kq];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[nb] = mfma(av, wt[4 * kk + kq][16 * nb + i], acc[nb]);
  }
}

// acc (16 x 64) = A (16 x 64) @ W with W[k][j] = wt[j][k] (the adjoint of gemm_fwd's map).
__device__ __forceinline__ void gemm_adj(const float (*a)[LA], const float (*wt)[LW], v4f* acc) {
  const int l = threadIdx.x & 63, i = l & 15, kq = l >> 4;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int kk = 0; kk < H / 4; ++kk) {
    const float av = a[i][4 * kk + kq];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[nb] = mfma(av, wt[16 * nb + i][4 * kk + kq], acc[nb]);
  }
}

__device__ __forceinline__ void d_to_lds(float (*t)[LA], const v4f* d) {
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

// d <- s silu(d); with `keep`, z <- s silu'(z) = s sig(z) (1 + z (1 - sig(z))) for the adjoint.
__device__ __forceinline__ void act(v4f* d, v4f* z, float s, bool keep) {
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float x = d[nb][t], g = sigm(x);
      d[nb][t] = s * x * g;
      if (keep) z[nb][t] = s * g * (1.f + x * (1.f - g));
    }
}

struct Smem {
  float w1t[KB][LW];
  float w2t[H][LW];
  float w3t[H][LW];
  float tile[WAVES][EW][LA];
  float dbt[WAVES][EW][KB];
};

__device__ __forceinline__ void stage_weights(Smem& sm, const float* W1, const float* W2, const float* W3) {
  stage_t(sm.w1t, W1, KB);
  stage_t(sm.w2t, W2, H);
  stage_t(sm.w3t, W3, H);
}

// Forward pass of one wave's 16 edges; leaves a3 in `a` and, with want_db, the
// activation slopes s silu'(z_k) in z1, z2, z3 and db/dr in LDS.
// Optional global outputs (nullptr to skip): a1, a2 (training weight gradients).
__device__ __forceinline__ void forward_tile(Smem& sm, int w, const float* __restrict__ r, int64_t e0, int64_t E,
                                             const Radial& q, float s, bool want_db, v4f* z1, v4f* z2, v4f* z3,
                                             v4f* a, float* a1_out, float* a2_out) {
  const int l = threadIdx.x & 63, i = l & 15, kq = l >> 4;
  radial_tile(q, r, e0, E, sm.tile[w], want_db ? sm.dbt[w] : nullptr);
  __syncthreads();
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) z1[nb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < KB / 4; ++kk) {
    const float av = sm.tile[w][i][4 * kk + kq];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) z1[nb] = mfma(av, sm.w1t[4 * kk + kq][16 * nb + i], z1[nb]);
  }
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) a[nb] = z1[nb];
  act(a, z1, s, want_db);
  if (a1_out) d_store(a1_out, e0, E, a);
  __syncthreads();
  d_to_lds(sm.tile[w], a);
  __syncthreads();
  gemm_fwd(sm.tile[w], sm.w2t, z2);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) a[nb] = z2[nb];
  act(a, z2, s, want_db);
  if (a2_out) d_store(a2_out, e0, E, a);
  __syncthreads();
  d_to_lds(sm.tile[w], a);
  __syncthreads();
  gemm_fwd(sm.tile[w], sm.w3t, z3);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) a[nb] = z3[nb];
  act(a, z3, s, want_db);
}

// Forward: a3 = s silu(W3 s silu(W2 s silu(W1 R(r)))), written to a3 [E, 64].
__global__ __launch_bounds__(256) void mlp_fwd_kernel(const float* __restrict__ r, int64_t E, float rc, int p,
                                                      const float* __restrict__ W1, const float* __restrict__ W2,
                                                      const float* __restrict__ W3, float s,
                                                      float* __restrict__ a3) {
  __shared__ Smem sm;
  stage_weights(sm, W1, W2, W3);
  const int w = threadIdx.x >> 6;
  const int64_t e0 = ((int64_t)blockIdx.x * WAVES + w) * EW;
  const Radial q = radial_consts(rc, p);
  v4f z1[4], z2[4], z3[4], a[4];
  forward_tile(sm, w, r, e0, E, q, s, false, z1, z2, z3, a, nullptr, nullptr);
  d_store(a3, e0, E, a);
}

// Adjoint: recomputes the forward in registers, then given da3 returns dr [E];
// optional outputs dz1..dz3, a1, a2 (nullptr to skip) feed weight gradients.
__global__ __launch_bounds__(256) void mlp_bwd_kernel(const float* __restrict__ r, int64_t E, float rc, int p,
                                                      const float* __restrict__ W1, const float* __restrict__ W2,
                                                      const float* __restrict__ W3, float s,
                                                      const float* __restrict__ da3, float* __restrict__ dr,
                                                      float* __restrict__ dz1, float* __restrict__ dz2,
                                                      float* __restrict__ dz3, float* __restrict__ a1_out,
                                                      float* __restrict__ a2_out) {
  __shared__ Smem sm;
  stage_weights(sm, W1, W2, W3);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, i = l & 15, kq = l >> 4;
  const int64_t e0 = ((int64_t)blockIdx.x * WAVES + w) * EW;
  const Radial q = radial_consts(rc, p);
  v4f z1[4], z2[4], z3[4], g[4];
  forward_tile(sm, w, r, e0, E, q, s, true, z1, z2, z3, g, a1_out, a2_out);
  d_load(da3, e0, E, g);
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) g[nb][t] *= z3[nb][t];
  if (dz3) d_store(dz3, e0, E, g);
  __syncthreads();
  d_to_lds(sm.tile[w], g);
  __syncthreads();
  gemm_adj(sm.tile[w], sm.w3t, g);    // da2 = dz3 W3
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) g[nb][t] *= z2[nb][t];
  if (dz2) d_store(dz2, e0, E, g);
  __syncthreads();
  d_to_lds(sm.tile[w], g);
  __syncthreads();
  gemm_adj(sm.tile[w], sm.w2t, g);    // da1 = dz2 W2
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) g[nb][t] *= z1[nb][t];
  if (dz1) d_store(dz1, e0, E, g);
  __syncthreads();
  d_to_lds(sm.tile[w], g);
  __syncthreads();
  // dR = dz1 W1 (16 x 8): one MFMA column block, B[k][j] = W1[k][j] = w1t[j][k] for j < 8, else 0.
  v4f dR = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int kk = 0; kk < H / 4; ++kk) {
    const float av = sm.tile[w][i][4 * kk + kq];
    const float bv = i < KB ? sm.w1t[i][4 * kk + kq] : 0.f;
    dR = mfma(av, bv, dR);
  }
  // dr[e] = sum_k dR[e][k] db_k(r_e): lane holds k = l % 16, rows 4*(l/16) + t.
  const int j = l & 15, i0 = 4 * (l >> 4);
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float v = j < KB ? dR[t] * sm.dbt[w][i0 + t][j] : 0.f;
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false));   // quad xor 1
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false));   // quad xor 2
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false));  // half-row mirror
    const int64_t e = e0 + i0 + t;
    if (j == 0 && e < E) dr[e] = v;
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
                        const float* W1, const float* W2, const float* W3, float silu_scale, float* a3, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 2) return fail(ICTC_ERR_ARGUMENT, "radial MLP: invalid arguments");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !a3) return fail(ICTC_ERR_ARGUMENT, "radial MLP: null operand");
  const unsigned blocks = (unsigned)((edges + EB - 1) / EB);
  hipLaunchKernelGGL(mlp_fwd_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, r, edges, cutoff, poly_p, W1,
                     W2, W3, silu_scale, a3);
  return launch_status("ictc_radial_mlp_fwd launch");
}

int ictc_radial_mlp_bwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                        const float* W1, const float* W2, const float* W3, float silu_scale, const float* da3,
                        float* dr, float* dz1, float* dz2, float* dz3, float* a1, float* a2, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 2) return fail(ICTC_ERR_ARGUMENT, "radial MLP: invalid arguments");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !da3 || !dr) return fail(ICTC_ERR_ARGUMENT, "radial MLP: null operand");
  const unsigned blocks = (unsigned)((edges + EB - 1) / EB);
  hipLaunchKernelGGL(mlp_bwd_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, r, edges, cutoff, poly_p, W1,
                     W2, W3, silu_scale, da3, dr, dz1, dz2, dz3, a1, a2);
  return launch_status("ictc_radial_mlp_bwd launch");
}

}  // extern "C"
