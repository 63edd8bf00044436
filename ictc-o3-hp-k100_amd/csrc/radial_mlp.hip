// Fused radial MLP on MFMA (gfx950): Bessel x polynomial-cutoff radial basis,
// then three bias-free 64-wide hidden layers with normalized SiLU
// (mace_ictc/models/mace/layers.py:826-835 `fc` without its last Linear,
// radial_basis.py:11-92), forward and the first adjoint down to d/dr.
//
// Every product is computed transposed, D[unit][edge] = sum_k A[unit][k] B[k][edge],
// on 16-edge tiles (one wave per tile, grid-stride over tiles).  With the
// 16x16 MFMA register layouts (lane l: A row l%16, B column l%16, k-chunk
// l/16; D column l%16, rows 4*(l/16)+r) a lane ends every layer holding 16
// hidden units of ONE edge, units 16*nb + 4*(l/16) + r (nb, r = 0..3).  The
// reduction index of an MFMA may be permuted freely as long as A and B use
// the same permutation, so the next layer takes exactly those 16 registers as
// its B operand (k-chunk e of k-step ks <-> unit 16*(2ks + e/4) + 4*(l/16) + e%4)
// and the weights are staged in LDS already permuted: no LDS round-trip of
// activations between layers.
//
// Precision: the radial layer (8 -> 64) and the final d/dR product run on
// FP32 MFMA (v_mfma_f32_16x16x4f32).  The 64x64 layers run on bf16 MFMA with a
// three-way operand split: x = hi + mid + lo + r (bf16 parts, |r| <= 2^-27 |x|),
// keeping the six partial products of size >= 2^-24 (hi*hi, hi*mid, mid*hi,
// mid*mid, hi*lo, lo*hi), accumulated smallest first in FP32: FP32-level
// accuracy and FP32's exponent range.  Six v_mfma_f32_16x16x32_bf16 (16 cycles)
// replace eight v_mfma_f32_16x16x4f32 (32 cycles) per 16x16x32 block.
//
// Weights are split and permuted once per block into LDS (forward: 50 KB;
// adjoint: 102 KB); blocks are persistent (about one resident set per CU).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "../../include/ictc_mi355x.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int H = 64;          // hidden width (compiled for 64)
constexpr int KB = 8;          // radial basis size (compiled for 8)
constexpr int FWD_WAVES = 4;   // waves per forward block (three blocks per CU: 51 KB of LDS each)
constexpr int BWD_WAVES = 8;   // waves per adjoint block (one block per CU: 102 KB of LDS)
constexpr int BWD2_WAVES = 4;  // waves per second-derivative block (one block per CU: 102 KB of LDS)

// ---- split-bf16 helpers ------------------------------------------------------

struct Split {
  bf16x8 p[3];  // hi, mid, lo
};

// f32 -> bf16 by gfx950's convert (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ Split split8(const float* v) {
  bf16x8 h, m, l;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 hb = (__bf16)v[e];
    const float r1 = v[e] - (float)hb;
    const __bf16 mb = (__bf16)r1;
    const float r2 = r1 - (float)mb;
    h[e] = hb;
    m[e] = mb;
    l[e] = (__bf16)r2;
  }
  return {{h, m, l}};
}

__device__ __forceinline__ v4f mfma32(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Hidden unit carried by k-chunk element e of k-step ks in lane group g.
__device__ __forceinline__ int unit_of(int ks, int g, int e) { return 16 * (2 * ks + (e >> 2)) + 4 * g + (e & 3); }

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

// b_k(r), db_k/dr and d2b_k/dr2 for one basis index k (1-based).
__device__ __forceinline__ void radial_two(const Radial& q, float x, int k, float& b, float& db, float& d2b) {
  const bool inside = x < q.rc;
  const float u = x / q.rc;
  const float upm2 = ipow(u, q.p - 2);
  const float upm1 = upm2 * u;
  const float up = upm1 * u;
  const float env = inside ? 1.f - q.c1 * up + q.c2 * up * u - q.c3 * up * u * u : 0.f;
  const float denv = inside ? (-q.c1 * q.p * upm1 + q.c2 * (q.p + 1) * up - q.c3 * (q.p + 2) * up * u) / q.rc : 0.f;
  const float d2env = inside ? (-q.c1 * q.p * (q.p - 1) * upm2 + q.c2 * (q.p + 1) * q.p * upm1 -
                                q.c3 * (q.p + 2) * (q.p + 1) * up) / (q.rc * q.rc)
                             : 0.f;
  const float xr = fmaxf(x, 1e-12f), inv = 1.f / xr;
  const float w = k * 3.14159265358979323846f / q.rc;
  float sn, cs;
  sincosf(w * x, &sn, &cs);
  const float f = q.pre * sn * inv;
  const float df = q.pre * (w * cs * inv - sn * inv * inv);
  const float d2f = q.pre * (-w * w * sn * inv - 2.f * w * cs * inv * inv + 2.f * sn * inv * inv * inv);
  b = f * env;
  db = df * env + f * denv;
  d2b = d2f * env + 2.f * df * denv + f * d2env;
}

// ---- weights in LDS ----------------------------------------------------------
// Forward formats.  wf[L][part][jb][ks][lane] = split part of
// W[16*jb + l%16][unit_of(ks, l/16, e)], e = 0..7 (W = W2 for L = 0, W3 for L = 1);
// w1f[jb][ks][lane] = W1[16*jb + l%16][2*(l/16) + ks] (radial layer, FP32).
struct FwdWeights {
  bf16x8 wf[2][3][4][2][64];
  float w1f[4][2][64];
};

// Adjoint formats.  wa[L][part][kb][ks][lane] = split part of
// W[unit_of(ks, l/16, e)][16*kb + l%16] (the transposed map);
// w1a[ks][lane]: row q = l%16 of dR (basis 2*(q/4) + q%4 when q%4 < 2, else a
// zero row), k = unit 16*(ks/4) + 4*(l/16) + ks%4: W1[unit][basis].
struct AdjWeights {
  bf16x8 wa[2][3][4][2][64];
  float w1a[16][64];
};

__device__ __forceinline__ void stage_fwd(FwdWeights& w, const float* __restrict__ W1, const float* __restrict__ W2,
                                          const float* __restrict__ W3) {
  for (int t = threadIdx.x; t < 2 * 4 * 2 * 64; t += blockDim.x) {
    const int L = t >> 9, jb = (t >> 7) & 3, ks = (t >> 6) & 1, l = t & 63;
    const float* W = L ? W3 : W2;
    const int j = 16 * jb + (l & 15), g = l >> 4;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = W[j * H + unit_of(ks, g, e)];
    const Split s = split8(v);
#pragma unroll
    for (int p = 0; p < 3; ++p) w.wf[L][p][jb][ks][l] = s.p[p];
  }
  for (int t = threadIdx.x; t < 4 * 2 * 64; t += blockDim.x) {
    const int jb = t >> 7, ks = (t >> 6) & 1, l = t & 63;
    w.w1f[jb][ks][l] = W1[(16 * jb + (l & 15)) * KB + 2 * (l >> 4) + ks];
  }
}

__device__ __forceinline__ void stage_adj(AdjWeights& w, const float* __restrict__ W1, const float* __restrict__ W2,
                                          const float* __restrict__ W3) {
  for (int t = threadIdx.x; t < 2 * 4 * 2 * 64; t += blockDim.x) {
    const int L = t >> 9, kb = (t >> 7) & 3, ks = (t >> 6) & 1, l = t & 63;
    const float* W = L ? W3 : W2;
    const int k = 16 * kb + (l & 15), g = l >> 4;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = W[unit_of(ks, g, e) * H + k];
    const Split s = split8(v);
#pragma unroll
    for (int p = 0; p < 3; ++p) w.wa[L][p][kb][ks][l] = s.p[p];
  }
  for (int t = threadIdx.x; t < 16 * 64; t += blockDim.x) {
    const int ks = t >> 6, l = t & 63, q = l & 15, g = l >> 4;
    const int j = 16 * (ks >> 2) + 4 * g + (ks & 3);
    w.w1a[ks][l] = (q & 3) < 2 ? W1[j * KB + 2 * (q >> 2) + (q & 3)] : 0.f;
  }
}

// The weight formats are loop invariant: without this the compiler hoists every
// LDS operand read out of the tile loop and spills.  Passing the LDS pointer
// through an empty asm statement each tile keeps the reads next to their MFMAs.
// What crosses the asm is the 32-bit LDS address: a generic pointer would leave
// the compiler unable to tell the reads are LDS reads, and it would emit flat
// loads, which also wait on the vector-memory counter behind the wave's stores.
template <class T>
__device__ __forceinline__ const T* opaque(const T* p) {
  typedef const T __attribute__((address_space(3))) * LdsPtr;
  LdsPtr q = (LdsPtr)p;
  asm volatile("" : "+v"(q));
  return (const T*)q;
}

// acc[nb] (units 16*nb + 4*(l/16) + r of the lane's edge) = sum_k A[unit][k] B[k],
// A from an LDS format [3][4][2][64], B = the split activations (two k-steps).
// The 4 row blocks are independent accumulator chains, interleaved.
__device__ __forceinline__ void gemm6(const bf16x8 (*A)[4][2][64], const Split* B, v4f* acc) {
  const int l = threadIdx.x & 63;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = v4f{0.f, 0.f, 0.f, 0.f};
#define ICTC_STEP(PA, PB, KS) \
  _Pragma("unroll") for (int nb = 0; nb < 4; ++nb) acc[nb] = mfma16(A[PA][nb][KS][l], B[KS].p[PB], acc[nb]);
  // smallest terms first: lo*hi, hi*lo, mid*mid, then mid*hi, hi*mid, then hi*hi
  ICTC_STEP(2, 0, 0) ICTC_STEP(0, 2, 0) ICTC_STEP(1, 1, 0)
  ICTC_STEP(2, 0, 1) ICTC_STEP(0, 2, 1) ICTC_STEP(1, 1, 1)
  ICTC_STEP(1, 0, 0) ICTC_STEP(0, 1, 0) ICTC_STEP(1, 0, 1)
  ICTC_STEP(0, 1, 1) ICTC_STEP(0, 0, 0) ICTC_STEP(0, 0, 1)
#undef ICTC_STEP
}

// Split the lane's 16 values (units by register) into the two k-steps' B operands.
__device__ __forceinline__ void split_units(const v4f* a, Split* B) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = a[2 * ks + (e >> 2)][e & 3];
    B[ks] = split8(v);
  }
}

// a <- s silu(z); with `keep`, slope <- s silu'(z) = s sig(z) (1 + z (1 - sig(z))).
template <bool KEEP>
__device__ __forceinline__ void act(const v4f* z, float s, v4f* a, v4f* slope) {
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float x = z[nb][t], g = sigm(x);
      a[nb][t] = s * x * g;
      if (KEEP) slope[nb][t] = s * g * (1.f + x * (1.f - g));
    }
}

// Row-major [E, 64] arrays in the lane layout: edge e0 + l%16, units 16*nb + 4*(l/16) .. +3.
__device__ __forceinline__ void store_units(float* __restrict__ out, int64_t e, bool ok, const v4f* v) {
  if (!ok) return;
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) *reinterpret_cast<v4f*>(out + e * H + 16 * nb + 4 * g) = v[nb];
}

__device__ __forceinline__ void load_units(const float* __restrict__ in, int64_t e, bool ok, v4f* v) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
    v[nb] = ok ? *reinterpret_cast<const v4f*>(in + e * H + 16 * nb + 4 * g) : v4f{0.f, 0.f, 0.f, 0.f};
}

// Forward of one 16-edge tile for the lane's edge (e, in range `ok`).  Leaves
// the last activation in a3; with KEEP, the slopes and db/dr of the lane's two
// basis functions (2*(l/16), 2*(l/16)+1).
template <bool KEEP>
__device__ __forceinline__ void forward_tile(const FwdWeights& w, const Radial& q, float x, float s, v4f* a3,
                                             v4f* s1, v4f* s2, v4f* s3, float* db, float* a1_out, float* a2_out,
                                             int64_t e, bool ok) {
  const int l = threadIdx.x & 63, g = l >> 4;
  float b[2];
  radial_one(q, x, 2 * g + 1, b[0], db[0]);
  radial_one(q, x, 2 * g + 2, b[1], db[1]);
  v4f z[4], a[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    z[jb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) z[jb] = mfma32(w.w1f[jb][ks][l], b[ks], z[jb]);
  }
  act<KEEP>(z, s, a, s1);
  if (a1_out) store_units(a1_out, e, ok, a);
  Split B[2];
  split_units(a, B);
  gemm6(w.wf[0], B, z);
  act<KEEP>(z, s, a, s2);
  if (a2_out) store_units(a2_out, e, ok, a);
  split_units(a, B);
  gemm6(w.wf[1], B, z);
  act<KEEP>(z, s, a3, s3);
}

// gemm6 for two B operands that share the A operand reads (values and tangents).
__device__ __forceinline__ void gemm6_pair(const bf16x8 (*A)[4][2][64], const Split* B, const Split* Bt, v4f* acc,
                                           v4f* acct) {
  const int l = threadIdx.x & 63;
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) acc[nb] = acct[nb] = v4f{0.f, 0.f, 0.f, 0.f};
#define ICTC_STEP(PA, PB, KS)                                          \
  _Pragma("unroll") for (int nb = 0; nb < 4; ++nb) {                   \
    const bf16x8 a = A[PA][nb][KS][l];                                 \
    acc[nb] = mfma16(a, B[KS].p[PB], acc[nb]);                         \
    acct[nb] = mfma16(a, Bt[KS].p[PB], acct[nb]);                      \
  }
  ICTC_STEP(2, 0, 0) ICTC_STEP(0, 2, 0) ICTC_STEP(1, 1, 0)
  ICTC_STEP(2, 0, 1) ICTC_STEP(0, 2, 1) ICTC_STEP(1, 1, 1)
  ICTC_STEP(1, 0, 0) ICTC_STEP(0, 1, 0) ICTC_STEP(1, 0, 1)
  ICTC_STEP(0, 1, 1) ICTC_STEP(0, 0, 0) ICTC_STEP(0, 0, 1)
#undef ICTC_STEP
}

// a <- s silu(z), t <- s silu'(z) * tz (forward-mode derivative of the activation).
__device__ __forceinline__ void act_tangent(const v4f* z, const v4f* tz, float s, v4f* a, v4f* t) {
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float x = z[nb][k], g = sigm(x);
      a[nb][k] = s * x * g;
      t[nb][k] = s * g * (1.f + x * (1.f - g)) * tz[nb][k];
    }
}

// The MLP of one tile and its forward-mode derivative along r, layer by layer
// (each slope is used as soon as it is formed): a3 and t3 = d a3 / dr.
__device__ __forceinline__ void forward_tangent_tile(const FwdWeights& w, const Radial& q, float x, float s, v4f* a3,
                                                     v4f* t3) {
  const int l = threadIdx.x & 63, g = l >> 4;
  float b[2], db[2];
  radial_one(q, x, 2 * g + 1, b[0], db[0]);
  radial_one(q, x, 2 * g + 2, b[1], db[1]);
  v4f z[4], tz[4], a[4], t[4];
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) {
    z[jb] = tz[jb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      z[jb] = mfma32(w.w1f[jb][ks][l], b[ks], z[jb]);
      tz[jb] = mfma32(w.w1f[jb][ks][l], db[ks], tz[jb]);
    }
  }
  act_tangent(z, tz, s, a, t);
  Split B[2], Bt[2];
  split_units(a, B);
  split_units(t, Bt);
  gemm6_pair(w.wf[0], B, Bt, z, tz);
  act_tangent(z, tz, s, a, t);
  split_units(a, B);
  split_units(t, Bt);
  gemm6_pair(w.wf[1], B, Bt, z, tz);
  act_tangent(z, tz, s, a3, t3);
}

// Forward: a3 = s silu(W3 s silu(W2 s silu(W1 R(r)))), written to a3 [E, 64].
__global__ __launch_bounds__(FWD_WAVES * 64) void mlp_fwd_kernel(const float* __restrict__ r, int64_t E, float rc,
                                                                 int p, const float* __restrict__ W1,
                                                                 const float* __restrict__ W2,
                                                                 const float* __restrict__ W3, float s,
                                                                 float* __restrict__ a3) {
  __shared__ FwdWeights ws;
  stage_fwd(ws, W1, W2, W3);
  __syncthreads();
  const Radial q = radial_consts(rc, p);
  const int waves = blockDim.x >> 6;
  const int64_t tiles = (E + 15) / 16, stride = (int64_t)gridDim.x * waves;
  for (int64_t t = (int64_t)blockIdx.x * waves + (threadIdx.x >> 6); t < tiles; t += stride) {
    const int64_t e = 16 * t + (threadIdx.x & 15);
    const bool ok = e < E;
    const float x = ok ? r[e] : 2.f * rc;
    const FwdWeights& w = *opaque(&ws);
    v4f a[4];
    float db[2];
    forward_tile<false>(w, q, x, s, a, nullptr, nullptr, nullptr, db, nullptr, nullptr, e, ok);
    store_units(a3, e, ok, a);
  }
}

// Forward with the forward-mode derivative along r: a3 and t3 = d a3 / dr,
// both [E, 64] (the hidden state the fused radial-gate message projects).
// With rho: t3 = rho[e] * d a3 / dr and no a3 (the d da3 of the second
// derivative, ictc_radial_mlp_bwd2 without dr).
__global__ __launch_bounds__(FWD_WAVES * 64, 3) void mlp_tan_kernel(const float* __restrict__ r, int64_t E, float rc,
                                                                 int p, const float* __restrict__ W1,
                                                                 const float* __restrict__ W2,
                                                                 const float* __restrict__ W3, float s,
                                                                 const float* __restrict__ rho,
                                                                 float* __restrict__ a3, float* __restrict__ t3) {
  __shared__ FwdWeights ws;
  stage_fwd(ws, W1, W2, W3);
  __syncthreads();
  const Radial q = radial_consts(rc, p);
  const int waves = blockDim.x >> 6;
  const int64_t tiles = (E + 15) / 16, stride = (int64_t)gridDim.x * waves;
  for (int64_t t = (int64_t)blockIdx.x * waves + (threadIdx.x >> 6); t < tiles; t += stride) {
    const int64_t e = 16 * t + (threadIdx.x & 15);
    const bool ok = e < E;
    const float x = ok ? r[e] : 2.f * rc;
    const FwdWeights& w = *opaque(&ws);
    v4f a[4], tg[4];
    forward_tangent_tile(w, q, x, s, a, tg);
    if (rho) {
      const float rh = ok ? rho[e] : 0.f;
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) tg[nb] *= rh;
    } else {
      store_units(a3, e, ok, a);
    }
    store_units(t3, e, ok, tg);
  }
}

// ---- fused radial gates: MLP forward + gate projection ----------------------
// gates[E, M] = s silu(...) (the MLP's last activation a3) . W4^T, W4 [M, 64]
// (the last Linear of `fc`).  a3 never leaves the chip: each wave runs the MLP
// for one 16-edge tile and leaves a3 split into bf16 parts in exactly the B
// operand layout of the projection (units under the permuted reduction index),
// the block's four tiles meet in LDS, and the waves then take 16-output row
// blocks of W4 in turn (A operands pre-split once per call into a workspace,
// read from L2 and reused across the four tiles).  Same split-bf16 arithmetic
// as the hidden layers.  Workspace format: ws[rb][ks][part][lane] = part of
// W4[16 rb + l%16][unit_of(ks, l/16, e)], e = 0..7 (M * 384 bytes).
constexpr int GATE_TILES = 4;  // 16-edge tiles per block iteration (one per wave)

__global__ void gates_split_kernel(const float* __restrict__ W4, int M, bf16x8* __restrict__ ws) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)(M / 16) * 2 * 64) return;
  const int l = (int)(t & 63), ks = (int)((t >> 6) & 1), rb = (int)(t >> 7);
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = W4[(int64_t)(16 * rb + (l & 15)) * H + unit_of(ks, l >> 4, e)];
  const Split sp = split8(v);
#pragma unroll
  for (int p = 0; p < 3; ++p) ws[((int64_t)(rb * 2 + ks) * 3 + p) * 64 + l] = sp.p[p];
}

// With TAN each wave also runs the MLP's forward-mode derivative along r for
// its tile, and the block projects twice per group: the gates, then (the
// waves' tangent splits swapped into the same LDS tiles) d gates / dr.
template <bool TAN>
__global__ __launch_bounds__(GATE_TILES * 64, 2) void gates_fwd_kernel(
    const float* __restrict__ r, int64_t E, float rc, int p, const float* __restrict__ W1,
    const float* __restrict__ W2, const float* __restrict__ W3, float s, const bf16x8* __restrict__ w4s, int M,
    float* __restrict__ gates, float* __restrict__ gdot) {
  __shared__ FwdWeights ws;
  __shared__ bf16x8 bsh[GATE_TILES][2][3][64];
  stage_fwd(ws, W1, W2, W3);
  __syncthreads();
  const Radial q = radial_consts(rc, p);
  const int l = threadIdx.x & 63, w = threadIdx.x >> 6, g = l >> 4, i = l & 15;
  const int64_t groups = (E + 16 * GATE_TILES - 1) / (16 * GATE_TILES);
  const int nrb = M / 16;
  for (int64_t grp = blockIdx.x; grp < groups; grp += gridDim.x) {
    const int64_t e0 = 16 * GATE_TILES * grp;
    Split T[2];  // TAN: this wave's tangent split, projected in the second pass
    {
      const FwdWeights& wf = *opaque(&ws);
      const int64_t e = e0 + 16 * w + i;
      const bool ok = e < E;
      const float x = ok ? r[e] : 2.f * rc;
      v4f a[4];
      float db[2];
      if (TAN) {
        v4f t3[4];
        forward_tangent_tile(wf, q, x, s, a, t3);
        split_units(t3, T);
      } else {
        forward_tile<false>(wf, q, x, s, a, nullptr, nullptr, nullptr, db, nullptr, nullptr, e, ok);
      }
      Split B[2];
      split_units(a, B);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int pt = 0; pt < 3; ++pt) bsh[w][ks][pt][l] = B[ks].p[pt];
    }
    for (int pass = 0; pass < (TAN ? 2 : 1); ++pass) {
      if (TAN && pass == 1) {
        __syncthreads();  // every wave holds the first pass's tiles in registers
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int pt = 0; pt < 3; ++pt) bsh[w][ks][pt][l] = T[ks].p[pt];
      }
      __syncthreads();
      float* __restrict__ out = pass ? gdot : gates;
      Split Bt[GATE_TILES][2];
#pragma unroll
      for (int t = 0; t < GATE_TILES; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int pt = 0; pt < 3; ++pt) Bt[t][ks].p[pt] = bsh[t][ks][pt][l];
      // A operands of the wave's next row block are in flight while the current one multiplies
      bf16x8 An[2][3];
      if (w < nrb) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int pt = 0; pt < 3; ++pt) An[ks][pt] = w4s[((int64_t)w * 6 + ks * 3 + pt) * 64 + l];
      }
      for (int rb = w; rb < nrb; rb += GATE_TILES) {
        bf16x8 Aop[2][3];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int pt = 0; pt < 3; ++pt) Aop[ks][pt] = An[ks][pt];
        if (rb + GATE_TILES < nrb) {
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int pt = 0; pt < 3; ++pt)
              An[ks][pt] = w4s[((int64_t)(rb + GATE_TILES) * 6 + ks * 3 + pt) * 64 + l];
        }
        v4f acc[GATE_TILES];
#pragma unroll
        for (int t = 0; t < GATE_TILES; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
#define ICTC_STEP(PA, PB, KS) \
  _Pragma("unroll") for (int t = 0; t < GATE_TILES; ++t) acc[t] = mfma16(Aop[KS][PA], Bt[t][KS].p[PB], acc[t]);
        ICTC_STEP(2, 0, 0) ICTC_STEP(0, 2, 0) ICTC_STEP(1, 1, 0)
        ICTC_STEP(2, 0, 1) ICTC_STEP(0, 2, 1) ICTC_STEP(1, 1, 1)
        ICTC_STEP(1, 0, 0) ICTC_STEP(0, 1, 0) ICTC_STEP(1, 0, 1)
        ICTC_STEP(0, 1, 1) ICTC_STEP(0, 0, 0) ICTC_STEP(0, 0, 1)
#undef ICTC_STEP
        // D: lane holds edge i of tile t, outputs 16 rb + 4 g + r
#pragma unroll
        for (int t = 0; t < GATE_TILES; ++t) {
          const int64_t e = e0 + 16 * t + i;
          if (e < E) *reinterpret_cast<v4f*>(out + e * M + 16 * rb + 4 * g) = acc[t];
        }
      }
    }
    __syncthreads();  // bsh is rewritten by the next group
  }
}

// W4-resident projection (gates <= RES_MAX_GATES): the grouped kernel above
// streams its 6 KB of split W4 operands per row block from L2 inside the store
// loop, and every wait for them also waits for the stores issued before them
// (one vector-memory counter), which keeps its single wave per SIMD well below
// the write rate.  Here each of a block's 8 waves keeps its share of the split
// W4 in registers for the whole launch, and the 16-edge tiles reach every wave
// through a double-buffered LDS ring (4 tiles per group): while all waves
// project group k, waves 4..7 each run the MLP of one tile of group k + 1 into
// the other ring slot, radii read through the scalar cache.  Waves 0..3 hold 7
// row blocks (rb = w + 4j), waves 4..7, which also run the MLP, hold 4
// (rb = 28 + (w - 4) + 4j): 44 row blocks, 704 gates.  The store loop issues no
// vector loads at all; one barrier per 64-edge group.
constexpr int RES_WAVES = 8;
constexpr int RES_RB_PROJ = 7;                                          // row blocks of waves 0..3
constexpr int RES_RB_DUTY = 4;                                          // row blocks of waves 4..7
constexpr int RES_MAX_GATES = 4 * 16 * (RES_RB_PROJ + RES_RB_DUTY);    // 704
constexpr int RES_TILES = 4;                                            // 16-edge tiles per group

template <int KINDS>
struct ResRing {
  bf16x8 b[2][RES_TILES][KINDS][2][3][64];  // [slot][tile][value, tangent][ks][part][lane]
};

// The lane's radius (edge e0 + l%16) of a tile, through 16 scalar loads (indices
// clamped to the last edge; lanes past it take `dflt`): no vector load, whose
// wait would also wait for the wave's pending stores.
__device__ __forceinline__ float tile_radius(const float* __restrict__ r, int64_t e0, int64_t E, float dflt) {
  const int i = threadIdx.x & 15;
  float x = r[e0 < E - 1 ? e0 : E - 1];
#pragma unroll
  for (int j = 1; j < 16; ++j) {
    const float v = r[e0 + j < E - 1 ? e0 + j : E - 1];
    x = i == j ? v : x;
  }
  return e0 + i < E ? x : dflt;
}

// C row blocks (rb0 + 4j) of one tile: 12 split-bf16 MFMA steps on C independent chains, then the stores.
template <int C, int CMAX>
__device__ __forceinline__ void res_project(const bf16x8 (&A)[CMAX][2][3], const Split* B, float* __restrict__ out,
                                            int64_t e, int64_t E, int M, int rb0) {
  const int g = (threadIdx.x & 63) >> 4;
  v4f acc[C];
#pragma unroll
  for (int j = 0; j < C; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
#define ICTC_STEP(PA, PB, KS) \
  _Pragma("unroll") for (int j = 0; j < C; ++j) acc[j] = mfma16(A[j][KS][PA], B[KS].p[PB], acc[j]);
  ICTC_STEP(2, 0, 0) ICTC_STEP(0, 2, 0) ICTC_STEP(1, 1, 0)
  ICTC_STEP(2, 0, 1) ICTC_STEP(0, 2, 1) ICTC_STEP(1, 1, 1)
  ICTC_STEP(1, 0, 0) ICTC_STEP(0, 1, 0) ICTC_STEP(1, 0, 1)
  ICTC_STEP(0, 1, 1) ICTC_STEP(0, 0, 0) ICTC_STEP(0, 0, 1)
#undef ICTC_STEP
  if (e < E) {
#pragma unroll
    for (int j = 0; j < C; ++j) *reinterpret_cast<v4f*>(out + e * M + 16 * (rb0 + 4 * j) + 4 * g) = acc[j];
  }
}

// Runtime row-block count n <= C to a compile-time chain count.
template <int C, int CMAX>
__device__ __forceinline__ void res_project_n(int n, const bf16x8 (&A)[CMAX][2][3], const Split* B,
                                              float* __restrict__ out, int64_t e, int64_t E, int M, int rb0) {
  if (n == C) res_project<C>(A, B, out, e, E, M, rb0);
  else if constexpr (C > 1) res_project_n<C - 1>(n, A, B, out, e, E, M, rb0);
}

// One wave's whole launch: C row blocks held in registers; DUTY waves also run
// the MLP of one tile of the next group in every iteration.  The two roles are
// separate instantiations, so the MLP's registers only meet 4 row blocks.
template <bool TAN, int C, bool DUTY>
__device__ __forceinline__ void res_wave(const float* __restrict__ r, int64_t E, float rc, int p, float s,
                                         const bf16x8* __restrict__ w4s, int M, float* __restrict__ gates,
                                         float* __restrict__ gdot, const FwdWeights& ws,
                                         ResRing<TAN ? 2 : 1>& ring, int w) {
  constexpr int KINDS = TAN ? 2 : 1;
  const int l = threadIdx.x & 63, i = l & 15;
  const int nrb = M / 16;
  const int rb0 = DUTY ? 4 * RES_RB_PROJ + (w - 4) : w;
  int cnt = nrb > rb0 ? (nrb - rb0 + 3) / 4 : 0;
  cnt = cnt < C ? cnt : C;
  bf16x8 A[C][2][3];
#pragma unroll
  for (int j = 0; j < C; ++j)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int pt = 0; pt < 3; ++pt)
        A[j][ks][pt] = j < cnt ? w4s[((int64_t)(rb0 + 4 * j) * 6 + ks * 3 + pt) * 64 + l] : bf16x8{};
  // complete the row-block loads here, not at a first use inside the loop (whose wait would recur every iteration)
#pragma unroll
  for (int j = 0; j < C; ++j)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int pt = 0; pt < 3; ++pt) asm volatile("" : "+v"(A[j][ks][pt]));
  const Radial q = radial_consts(rc, p);
  const int64_t groups = (E + 16 * RES_TILES - 1) / (16 * RES_TILES);
  auto mlp = [&](int64_t grp, int buf) {
    const int t = w - 4;
    const int64_t e0 = 16 * (RES_TILES * grp + t);
    const float x = tile_radius(r, e0, E, 2.f * rc);
    const FwdWeights& wf = *opaque(&ws);
    v4f a[4];
    Split B[2];
    if (TAN) {
      v4f t3[4];
      forward_tangent_tile(wf, q, x, s, a, t3);
      split_units(t3, B);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int pt = 0; pt < 3; ++pt) ring.b[buf][t][KINDS - 1][ks][pt][l] = B[ks].p[pt];
    } else {
      float db[2];
      forward_tile<false>(wf, q, x, s, a, nullptr, nullptr, nullptr, db, nullptr, nullptr, e0 + i, false);
    }
    split_units(a, B);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int pt = 0; pt < 3; ++pt) ring.b[buf][t][0][ks][pt][l] = B[ks].p[pt];
  };
  // Iteration k runs the MLP of group k + 1 and projects group k; k = -1 only fills
  // the first slot (one MLP call site, so every tile's gates come from the same code).
  int k = -1;
  for (int64_t grp = (int64_t)blockIdx.x - gridDim.x; grp < groups; grp += gridDim.x, ++k) {
    const int64_t nxt = grp + gridDim.x;
    if (DUTY && nxt < groups) mlp(nxt, (k + 1) & 1);
    const ResRing<KINDS>& rg = *opaque(&ring);
#pragma unroll 1
    for (int tk = 0; tk < (grp >= 0 ? RES_TILES * KINDS : 0); ++tk) {
      const int t = tk / KINDS, kind = tk % KINDS;
      Split B[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int pt = 0; pt < 3; ++pt) B[ks].p[pt] = rg.b[k & 1][t][kind][ks][pt][l];
      res_project_n<C>(cnt, A, B, kind ? gdot : gates, 16 * (RES_TILES * grp + t) + i, E, M, rb0);
    }
    __syncthreads();  // the slot just read is rewritten in the next iteration
  }
}

// Block of 8 waves, one block per CU (M <= RES_MAX_GATES).
template <bool TAN>
__global__ __launch_bounds__(RES_WAVES * 64, 1) void gates_res_kernel(
    const float* __restrict__ r, int64_t E, float rc, int p, const float* __restrict__ W1,
    const float* __restrict__ W2, const float* __restrict__ W3, float s, const bf16x8* __restrict__ w4s, int M,
    float* __restrict__ gates, float* __restrict__ gdot) {
  __shared__ FwdWeights ws;
  __shared__ ResRing<TAN ? 2 : 1> ring;
  stage_fwd(ws, W1, W2, W3);
  __syncthreads();
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w < 4) res_wave<TAN, RES_RB_PROJ, false>(r, E, rc, p, s, w4s, M, gates, gdot, ws, ring, w);
  else res_wave<TAN, RES_RB_DUTY, true>(r, E, rc, p, s, w4s, M, gates, gdot, ws, ring, w);
}

// Narrow projections with r tangents (M <= 256 gates, e.g. an l = 0 input
// layer's 3 paths x 64): the split W4 (M * 384 bytes) fits in LDS beside the
// MLP weights, so every wave projects its own 16-edge tile (values and
// tangents) with A operands from LDS and no block-wide exchange: the waves run
// unsynchronised and one wave's MLP overlaps another's stores.  cfg4 layer 0
// (M = 192): 3.04 ms against 3.39 for the grouped kernel.  Without tangents
// the grouped kernel stays ahead (1.80 against 1.90 ms).
constexpr int SMALL_WAVES = 8;
constexpr int SMALL_MAX_GATES = 256;

template <bool TAN>
__global__ __launch_bounds__(SMALL_WAVES * 64) void gates_small_kernel(
    const float* __restrict__ r, int64_t E, float rc, int p, const float* __restrict__ W1,
    const float* __restrict__ W2, const float* __restrict__ W3, float s, const bf16x8* __restrict__ w4s, int M,
    float* __restrict__ gates, float* __restrict__ gdot) {
  __shared__ FwdWeights ws;
  extern __shared__ bf16x8 w4l[];  // [M / 16][2][3][64], the workspace format
  stage_fwd(ws, W1, W2, W3);
  const int nrb = M / 16;
  for (int t = threadIdx.x; t < nrb * 6 * 64; t += blockDim.x) w4l[t] = w4s[t];
  __syncthreads();
  const Radial q = radial_consts(rc, p);
  const int l = threadIdx.x & 63, g = l >> 4, i = l & 15;
  const int waves = blockDim.x >> 6;
  const int64_t tiles = (E + 15) / 16, stride = (int64_t)gridDim.x * waves;
  for (int64_t tile = (int64_t)blockIdx.x * waves + (threadIdx.x >> 6); tile < tiles; tile += stride) {
    const int64_t e = 16 * tile + i;
    const bool ok = e < E;
    const float x = ok ? r[e] : 2.f * rc;
    const FwdWeights& wf = *opaque(&ws);
    v4f a[4], t3[4];
    float db[2];
    if (TAN) forward_tangent_tile(wf, q, x, s, a, t3);
    else forward_tile<false>(wf, q, x, s, a, nullptr, nullptr, nullptr, db, nullptr, nullptr, e, ok);
    Split B[2], Bt[2];
    split_units(a, B);
    if (TAN) split_units(t3, Bt);
    const bf16x8* A = opaque(static_cast<const bf16x8*>(w4l));
    for (int rb = 0; rb < nrb; ++rb) {
      v4f acc = v4f{0.f, 0.f, 0.f, 0.f}, acct = v4f{0.f, 0.f, 0.f, 0.f};
#define ICTC_STEP(PA, PB, KS)                                   \
  {                                                             \
    const bf16x8 aop = A[((rb * 2 + KS) * 3 + PA) * 64 + l];    \
    acc = mfma16(aop, B[KS].p[PB], acc);                        \
    if (TAN) acct = mfma16(aop, Bt[KS].p[PB], acct);            \
  }
      ICTC_STEP(2, 0, 0) ICTC_STEP(0, 2, 0) ICTC_STEP(1, 1, 0)
      ICTC_STEP(2, 0, 1) ICTC_STEP(0, 2, 1) ICTC_STEP(1, 1, 1)
      ICTC_STEP(1, 0, 0) ICTC_STEP(0, 1, 0) ICTC_STEP(1, 0, 1)
      ICTC_STEP(0, 1, 1) ICTC_STEP(0, 0, 0) ICTC_STEP(0, 0, 1)
#undef ICTC_STEP
      if (ok) {
        *reinterpret_cast<v4f*>(gates + e * M + 16 * rb + 4 * g) = acc;
        if (TAN) *reinterpret_cast<v4f*>(gdot + e * M + 16 * rb + 4 * g) = acct;
      }
    }
  }
}

// Adjoint: recomputes the forward in registers, then given da3 returns dr [E];
// optional outputs dz1..dz3, a1, a2 (nullptr to skip) feed weight gradients.
__global__ __launch_bounds__(BWD_WAVES * 64) void mlp_bwd_kernel(
    const float* __restrict__ r, int64_t E, float rc, int p, const float* __restrict__ W1,
    const float* __restrict__ W2, const float* __restrict__ W3, float s, const float* __restrict__ da3,
    float* __restrict__ dr, float* __restrict__ dz1, float* __restrict__ dz2, float* __restrict__ dz3,
    float* __restrict__ a1_out, float* __restrict__ a2_out) {
  __shared__ FwdWeights wfs;
  __shared__ AdjWeights was;
  stage_fwd(wfs, W1, W2, W3);
  stage_adj(was, W1, W2, W3);
  __syncthreads();
  const Radial q = radial_consts(rc, p);
  const int l = threadIdx.x & 63;
  const int waves = blockDim.x >> 6;
  const int64_t tiles = (E + 15) / 16, stride = (int64_t)gridDim.x * waves;
  for (int64_t t = (int64_t)blockIdx.x * waves + (threadIdx.x >> 6); t < tiles; t += stride) {
    const int64_t e = 16 * t + (l & 15);
    const bool ok = e < E;
    const float x = ok ? r[e] : 2.f * rc;
    const FwdWeights& wf = *opaque(&wfs);
    const AdjWeights& wa = *opaque(&was);
    v4f s1[4], s2[4], s3[4], gv[4];
    float db[2];
    forward_tile<true>(wf, q, x, s, gv, s1, s2, s3, db, a1_out, a2_out, e, ok);
    load_units(da3, e, ok, gv);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) gv[nb] *= s3[nb];
    if (dz3) store_units(dz3, e, ok, gv);
    Split B[2];
    split_units(gv, B);
    gemm6(wa.wa[1], B, gv);  // da2 = dz3 W3
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) gv[nb] *= s2[nb];
    if (dz2) store_units(dz2, e, ok, gv);
    split_units(gv, B);
    gemm6(wa.wa[0], B, gv);  // da1 = dz2 W2
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) gv[nb] *= s1[nb];
    if (dz1) store_units(dz1, e, ok, gv);
    // dR = dz1 W1 on FP32 MFMA: k-step ks takes the lane's unit 16*(ks/4) + 4*(l/16) + ks%4.
    v4f dR = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) dR = mfma32(wa.w1a[ks][l], gv[ks >> 2][ks & 3], dR);
    // lane holds dR of basis 2*(l/16) + r in rows r = 0, 1; dr = sum_k dR_k db_k over the 4 lane groups
    float v = dR[0] * db[0] + dR[1] * db[1];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if (l < 16 && ok) dr[e] = v;
  }
}

// ---- second derivative of the hidden MLP ------------------------------------
// With u = da3 the cotangent of the last activation, the first adjoint's d/dr is
// dr = u . t3, t3 = d a3 / dr (the forward-mode tangent).  Its derivative for a
// cotangent rho on dr is the reverse pass through the tangent network, seeded
// with rho u on t3: per layer k (z_k = W_k a_{k-1}, a_k = s silu(z_k), primes
// = d/dr)
//   zb3' = rho u . sl3,   zb3 = rho u . cv3
//   zbk' = (W_{k+1}^T zb_{k+1}') . slk
//   zbk  = (W_{k+1}^T zb_{k+1}) . slk + (W_{k+1}^T zb_{k+1}') . cvk
// with slk = s silu'(z_k) and cvk = s silu''(z_k) z_k'; then
//   d W_k += zbk'^T a_{k-1}' + zbk^T a_{k-1}     (a_0 = R(r), a_0' = R'(r))
//   d r    = (W1^T zb1') . R''(r) + (W1^T zb1) . R'(r)
//   d u    = rho t3.
// s silu''(z) = s sig (1 - sig) (2 + z (1 - 2 sig)).
// With v (nullable), the cotangent of a3 itself, zb3 also takes v . sl3: the
// first adjoint's chain runs along the unprimed one, so one pass returns the sum
// of both derivatives.  Without dr only d u is written.
// The weight-gradient rows go to [2E, 64] arrays (primed rows 0..E-1, unprimed
// rows E..2E-1; the radial rows [2E, 8]), so that each d W_k is one product
// zrows^T arows over 2E rows.
__device__ __forceinline__ void act_dual(const v4f* z, const v4f* tz, float s, v4f* a, v4f* t, v4f* sl, v4f* cv) {
#pragma unroll
  for (int nb = 0; nb < 4; ++nb)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float x = z[nb][k], g = sigm(x), h = 1.f - g;
      a[nb][k] = s * x * g;
      sl[nb][k] = s * g * (1.f + x * h);
      t[nb][k] = sl[nb][k] * tz[nb][k];
      cv[nb][k] = s * g * h * (2.f + x * (h - g)) * tz[nb][k];
    }
}

__global__ __launch_bounds__(BWD2_WAVES * 64, 1) void mlp_bwd2_kernel(
    const float* __restrict__ r, int64_t E, float rc, int p, const float* __restrict__ W1,
    const float* __restrict__ W2, const float* __restrict__ W3, float s, const float* __restrict__ u,
    const float* __restrict__ rho, const float* __restrict__ v, float* __restrict__ dr, float* __restrict__ du,
    float* __restrict__ z3rows,
    float* __restrict__ a2rows, float* __restrict__ z2rows, float* __restrict__ a1rows, float* __restrict__ z1rows,
    float* __restrict__ brows) {
  __shared__ FwdWeights wfs;
  __shared__ AdjWeights was;
  stage_fwd(wfs, W1, W2, W3);
  stage_adj(was, W1, W2, W3);
  __syncthreads();
  const Radial q = radial_consts(rc, p);
  const int l = threadIdx.x & 63, g = l >> 4;
  const int waves = blockDim.x >> 6;
  const int64_t tiles = (E + 15) / 16, stride = (int64_t)gridDim.x * waves;
  const bool rows = z3rows != nullptr;
  for (int64_t t = (int64_t)blockIdx.x * waves + (threadIdx.x >> 6); t < tiles; t += stride) {
    const int64_t e = 16 * t + (l & 15);
    const bool ok = e < E;
    const float x = ok ? r[e] : 2.f * rc;
    const float rh = ok ? rho[e] : 0.f;
    const FwdWeights& wf = *opaque(&wfs);
    const AdjWeights& wa = *opaque(&was);
    float b[2], db[2], d2b[2];
    radial_two(q, x, 2 * g + 1, b[0], db[0], d2b[0]);
    radial_two(q, x, 2 * g + 2, b[1], db[1], d2b[1]);
    if (rows && ok) {
      *reinterpret_cast<float2*>(brows + e * KB + 2 * g) = make_float2(db[0], db[1]);
      *reinterpret_cast<float2*>(brows + (E + e) * KB + 2 * g) = make_float2(b[0], b[1]);
    }
    // forward with the tangent: slopes and curvatures kept per layer
    v4f sl1[4], cv1[4], sl2[4], cv2[4], sl3[4], cv3[4];
    v4f z[4], tz[4], a[4], ta[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      z[jb] = tz[jb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        z[jb] = mfma32(wf.w1f[jb][ks][l], b[ks], z[jb]);
        tz[jb] = mfma32(wf.w1f[jb][ks][l], db[ks], tz[jb]);
      }
    }
    act_dual(z, tz, s, a, ta, sl1, cv1);
    if (rows) {
      store_units(a1rows, e, ok, ta);
      store_units(a1rows + E * H, e, ok, a);
    }
    Split B[2], Bt[2];
    split_units(a, B);
    split_units(ta, Bt);
    gemm6_pair(wf.wf[0], B, Bt, z, tz);
    act_dual(z, tz, s, a, ta, sl2, cv2);
    if (rows) {
      store_units(a2rows, e, ok, ta);
      store_units(a2rows + E * H, e, ok, a);
    }
    split_units(a, B);
    split_units(ta, Bt);
    gemm6_pair(wf.wf[1], B, Bt, z, tz);
    act_dual(z, tz, s, a, ta, sl3, cv3);   // a = a3 (unused), ta = t3
    if (du) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) a[nb] = rh * ta[nb];
      store_units(du, e, ok, a);
    }
    if (!dr) continue;   // d u only
    // reverse through the tangent network (and, with v, the first adjoint for cotangent v on a3)
    load_units(u, e, ok, a);
    v4f zp[4], zu[4];
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const v4f seed = rh * a[nb];
      zp[nb] = seed * sl3[nb];
      zu[nb] = seed * cv3[nb];
    }
    if (v) {
      load_units(v, e, ok, a);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) zu[nb] += a[nb] * sl3[nb];
    }
    if (rows) {
      store_units(z3rows, e, ok, zp);
      store_units(z3rows + E * H, e, ok, zu);
    }
    split_units(zp, B);
    split_units(zu, Bt);
    gemm6_pair(wa.wa[1], B, Bt, zp, zu);   // W3^T zb3', W3^T zb3
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      zu[nb] = zu[nb] * sl2[nb] + zp[nb] * cv2[nb];
      zp[nb] = zp[nb] * sl2[nb];
    }
    if (rows) {
      store_units(z2rows, e, ok, zp);
      store_units(z2rows + E * H, e, ok, zu);
    }
    split_units(zp, B);
    split_units(zu, Bt);
    gemm6_pair(wa.wa[0], B, Bt, zp, zu);   // W2^T zb2', W2^T zb2
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      zu[nb] = zu[nb] * sl1[nb] + zp[nb] * cv1[nb];
      zp[nb] = zp[nb] * sl1[nb];
    }
    if (rows) {
      store_units(z1rows, e, ok, zp);
      store_units(z1rows + E * H, e, ok, zu);
    }
    // W1^T zb1' and W1^T zb1 on FP32 MFMA (rows of the lane's two basis functions)
    v4f dRp = v4f{0.f, 0.f, 0.f, 0.f}, dRu = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) {
      dRp = mfma32(wa.w1a[ks][l], zp[ks >> 2][ks & 3], dRp);
      dRu = mfma32(wa.w1a[ks][l], zu[ks >> 2][ks & 3], dRu);
    }
    float v = dRp[0] * d2b[0] + dRp[1] * d2b[1] + dRu[0] * db[0] + dRu[1] * db[1];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if (l < 16 && ok) dr[e] = v;
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

// Compute units of the current device (queried once per device).
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

// Blocks of `kernel` resident per CU (LDS, registers), at most `want`: the
// persistent kernels below size their grid to what runs at once, so that no
// block waits for a second round on a half-empty GPU.
template <class K>
int resident_per_cu(K kernel, int threads, int want) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n <= 0) n = 1;
  return n < want ? n : want;
}

unsigned grid_for(int64_t edges, int waves, int blocks_per_cu) {
  const int64_t tiles = (edges + 15) / 16, need = (tiles + waves - 1) / waves;
  const int64_t cap = (int64_t)cu_count() * blocks_per_cu;
  return (unsigned)(need < cap ? need : cap);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }


// Argument checks shared by the two gate-tangent entry points: a negative
// error code, 1 when there is nothing to do (no edges), 0 to launch.
int gates_tangent_check(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                        const float* W1, const float* W2, const float* W3, const float* W4, int gates,
                        const float* out, const float* tangent) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 2 || gates <= 0 || gates % 16)
    return fail(ICTC_ERR_ARGUMENT, "radial gates: invalid arguments (gates must be a positive multiple of 16)");
  if (edges == 0) return 1;
  if (!r || !W1 || !W2 || !W3 || !W4 || !out || !tangent) return fail(ICTC_ERR_ARGUMENT, "radial gates: null operand");
  if (!aligned16(out) || !aligned16(tangent)) return fail(ICTC_ERR_ARGUMENT, "radial gates: operands must be 16-byte aligned");
  return 0;
}

// W4 split into MFMA operand order in `ws`, then the gates and their r tangents.
int gates_tangent_launch(const float* r, int64_t edges, float cutoff, int poly_p, const float* W1, const float* W2,
                         const float* W3, const float* W4, int gates, float silu_scale, float* out, float* tangent,
                         bf16x8* ws, hipStream_t st) {
  const int split_threads = (gates / 16) * 2 * 64;
  hipLaunchKernelGGL(gates_split_kernel, dim3((split_threads + 255) / 256), dim3(256), 0, st, W4, gates, ws);
  if (int rc = launch_status("ictc_radial_gates_tangent_fwd split")) return rc;
  if (gates <= SMALL_MAX_GATES) {
    const size_t lds = (size_t)(gates / 16) * 6 * 64 * sizeof(bf16x8);
    const int64_t tiles = (edges + 15) / 16, cap = (int64_t)cu_count() * SMALL_WAVES;
    const int64_t blocks = (tiles + SMALL_WAVES - 1) / SMALL_WAVES;
    hipLaunchKernelGGL(gates_small_kernel<true>, dim3((unsigned)(blocks < cap / SMALL_WAVES ? blocks : cap / SMALL_WAVES)),
                       dim3(SMALL_WAVES * 64), lds, st, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale,
                       (const bf16x8*)ws, gates, out, tangent);
    return launch_status("ictc_radial_gates_tangent_fwd launch");
  }
  if (gates <= RES_MAX_GATES) {
    const int64_t groups = (edges + 16 * RES_TILES - 1) / (16 * RES_TILES), cap = cu_count();
    hipLaunchKernelGGL(gates_res_kernel<true>, dim3((unsigned)(groups < cap ? groups : cap)), dim3(RES_WAVES * 64),
                       0, st, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, (const bf16x8*)ws, gates, out,
                       tangent);
    return launch_status("ictc_radial_gates_tangent_fwd launch");
  }
  const int64_t groups = (edges + 16 * GATE_TILES - 1) / (16 * GATE_TILES);
  const int64_t cap = (int64_t)cu_count() * resident_per_cu(gates_fwd_kernel<true>, GATE_TILES * 64, 3);
  hipLaunchKernelGGL(gates_fwd_kernel<true>, dim3((unsigned)(groups < cap ? groups : cap)), dim3(GATE_TILES * 64), 0,
                     st, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, (const bf16x8*)ws, gates, out,
                     tangent);
  return launch_status("ictc_radial_gates_tangent_fwd launch");
}

// ---- static scratch of the no-alloc entry point ----------------------------
// The split W4 of ictc_radial_gates_tangent_fwd_noalloc lives in this
// file-scope device array (ICTC_NOALLOC_MAX_GATES * 384 bytes, held by every
// GPU the library runs on until the process ends).  Host code never passes
// the array's name to a kernel: its device address is looked up once per
// device with hipGetSymbolAddress and kept per device.
constexpr int kNoallocWords = ICTC_NOALLOC_MAX_GATES * 24;   // bf16x8 words (384 bytes per gate)
static __device__ __align__(256) bf16x8 scratch[kNoallocWords];

constexpr int kMaxDevices = 64;
bf16x8* g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mu;

int noalloc_scratch(bf16x8** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(ICTC_ERR_RUNTIME, "radial gates (no-alloc): no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      char buf[256];
      snprintf(buf, sizeof(buf), "radial gates (no-alloc): hipGetSymbolAddress: %s", hipGetErrorString(e));
      return fail(ICTC_ERR_RUNTIME, buf);
    }
    g_scratch[dev] = static_cast<bf16x8*>(ptr);
  }
  *out = g_scratch[dev];
  return ICTC_OK;
}

}  // namespace

extern "C" {

int ictc_radial_mlp_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                        const float* W1, const float* W2, const float* W3, float silu_scale, float* a3, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 2) return fail(ICTC_ERR_ARGUMENT, "radial MLP: invalid arguments");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !a3) return fail(ICTC_ERR_ARGUMENT, "radial MLP: null operand");
  if (!aligned16(a3)) return fail(ICTC_ERR_ARGUMENT, "radial MLP: a3 must be 16-byte aligned");
  const int fwd_per_cu = resident_per_cu(mlp_fwd_kernel, FWD_WAVES * 64, 3);
  hipLaunchKernelGGL(mlp_fwd_kernel, dim3(grid_for(edges, FWD_WAVES, fwd_per_cu)), dim3(FWD_WAVES * 64), 0,
                     (hipStream_t)stream, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, a3);
  return launch_status("ictc_radial_mlp_fwd launch");
}

int ictc_radial_mlp_tangent_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                                const float* W1, const float* W2, const float* W3, float silu_scale, float* a3,
                                float* t3, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 2) return fail(ICTC_ERR_ARGUMENT, "radial MLP: invalid arguments");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !a3 || !t3) return fail(ICTC_ERR_ARGUMENT, "radial MLP: null operand");
  if (!aligned16(a3) || !aligned16(t3)) return fail(ICTC_ERR_ARGUMENT, "radial MLP: a3 and t3 must be 16-byte aligned");
  const int per_cu = resident_per_cu(mlp_tan_kernel, FWD_WAVES * 64, 3);
  hipLaunchKernelGGL(mlp_tan_kernel, dim3(grid_for(edges, FWD_WAVES, per_cu)), dim3(FWD_WAVES * 64), 0,
                     (hipStream_t)stream, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, nullptr, a3, t3);
  return launch_status("ictc_radial_mlp_tangent_fwd launch");
}

int64_t ictc_radial_gates_workspace_bytes(int gates) {
  if (gates <= 0 || gates % 16) return -1;
  return (int64_t)gates * 384;
}

int ictc_radial_gates_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                          const float* W1, const float* W2, const float* W3, const float* W4, int gates,
                          float silu_scale, float* out, void* workspace, int64_t workspace_bytes, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 2 || gates <= 0 || gates % 16)
    return fail(ICTC_ERR_ARGUMENT, "radial gates: invalid arguments (gates must be a positive multiple of 16)");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !W4 || !out || !workspace) return fail(ICTC_ERR_ARGUMENT, "radial gates: null operand");
  if (workspace_bytes < ictc_radial_gates_workspace_bytes(gates))
    return fail(ICTC_ERR_ARGUMENT, "radial gates: workspace too small");
  if (!aligned16(out) || !aligned16(workspace)) return fail(ICTC_ERR_ARGUMENT, "radial gates: operands must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  const int split_threads = (gates / 16) * 2 * 64;
  hipLaunchKernelGGL(gates_split_kernel, dim3((split_threads + 255) / 256), dim3(256), 0, st, W4, gates,
                     (bf16x8*)workspace);
  if (int rc = launch_status("ictc_radial_gates_fwd split")) return rc;
  if (gates > SMALL_MAX_GATES && gates <= RES_MAX_GATES) {
    const int64_t groups = (edges + 16 * RES_TILES - 1) / (16 * RES_TILES), cap = cu_count();
    hipLaunchKernelGGL(gates_res_kernel<false>, dim3((unsigned)(groups < cap ? groups : cap)), dim3(RES_WAVES * 64),
                       0, st, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, (const bf16x8*)workspace, gates,
                       out, nullptr);
    return launch_status("ictc_radial_gates_fwd launch");
  }
  const int64_t groups = (edges + 16 * GATE_TILES - 1) / (16 * GATE_TILES);
  const int64_t cap = (int64_t)cu_count() * resident_per_cu(gates_fwd_kernel<false>, GATE_TILES * 64, 3);
  hipLaunchKernelGGL(gates_fwd_kernel<false>, dim3((unsigned)(groups < cap ? groups : cap)), dim3(GATE_TILES * 64), 0,
                     st, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, (const bf16x8*)workspace, gates, out,
                     nullptr);
  return launch_status("ictc_radial_gates_fwd launch");
}

int ictc_radial_gates_tangent_fwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                                  const float* W1, const float* W2, const float* W3, const float* W4, int gates,
                                  float silu_scale, float* out, float* tangent, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  if (int rc = gates_tangent_check(r, edges, num_basis, hidden, cutoff, poly_p, W1, W2, W3, W4, gates, out, tangent))
    return rc > 0 ? ICTC_OK : rc;
  if (!workspace) return fail(ICTC_ERR_ARGUMENT, "radial gates: null operand");
  if (workspace_bytes < ictc_radial_gates_workspace_bytes(gates))
    return fail(ICTC_ERR_ARGUMENT, "radial gates: workspace too small");
  if (!aligned16(workspace)) return fail(ICTC_ERR_ARGUMENT, "radial gates: operands must be 16-byte aligned");
  return gates_tangent_launch(r, edges, cutoff, poly_p, W1, W2, W3, W4, gates, silu_scale, out, tangent,
                              (bf16x8*)workspace, (hipStream_t)stream);
}

int ictc_radial_gates_tangent_fwd_noalloc(const float* r, int64_t edges, int num_basis, int hidden, float cutoff,
                                          int poly_p, const float* W1, const float* W2, const float* W3,
                                          const float* W4, int gates, float silu_scale, float* out, float* tangent,
                                          void* stream) {
  if (gates > ICTC_NOALLOC_MAX_GATES)
    return fail(ICTC_ERR_ARGUMENT, "radial gates (no-alloc): more gates than the static scratch holds");
  if (int rc = gates_tangent_check(r, edges, num_basis, hidden, cutoff, poly_p, W1, W2, W3, W4, gates, out, tangent))
    return rc > 0 ? ICTC_OK : rc;
  bf16x8* ws = nullptr;
  if (int rc = noalloc_scratch(&ws)) return rc;
  return gates_tangent_launch(r, edges, cutoff, poly_p, W1, W2, W3, W4, gates, silu_scale, out, tangent, ws,
                              (hipStream_t)stream);
}

int ictc_radial_mlp_bwd(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                        const float* W1, const float* W2, const float* W3, float silu_scale, const float* da3,
                        float* dr, float* dz1, float* dz2, float* dz3, float* a1, float* a2, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 2) return fail(ICTC_ERR_ARGUMENT, "radial MLP: invalid arguments");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !da3 || !dr) return fail(ICTC_ERR_ARGUMENT, "radial MLP: null operand");
  for (const float* p : {da3, (const float*)dz1, (const float*)dz2, (const float*)dz3, (const float*)a1,
                         (const float*)a2})
    if (p && !aligned16(p)) return fail(ICTC_ERR_ARGUMENT, "radial MLP: [E, 64] operands must be 16-byte aligned");
  const int bwd_per_cu = resident_per_cu(mlp_bwd_kernel, BWD_WAVES * 64, 1);
  hipLaunchKernelGGL(mlp_bwd_kernel, dim3(grid_for(edges, BWD_WAVES, bwd_per_cu)), dim3(BWD_WAVES * 64), 0,
                     (hipStream_t)stream, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, da3, dr, dz1, dz2, dz3,
                     a1, a2);
  return launch_status("ictc_radial_mlp_bwd launch");
}

int ictc_radial_mlp_bwd2(const float* r, int64_t edges, int num_basis, int hidden, float cutoff, int poly_p,
                         const float* W1, const float* W2, const float* W3, float silu_scale, const float* da3,
                         const float* rho, const float* v, float* dr, float* dda3, float* z3rows, float* a2rows,
                         float* z2rows, float* a1rows, float* z1rows, float* brows, void* stream) {
  if (num_basis != KB || hidden != H) return fail(ICTC_ERR_UNSUPPORTED, "fused radial MLP is compiled for 8 -> 64");
  if (edges < 0 || !(cutoff > 0.f) || poly_p < 2) return fail(ICTC_ERR_ARGUMENT, "radial MLP: invalid arguments");
  if (edges == 0) return ICTC_OK;
  if (!r || !W1 || !W2 || !W3 || !da3 || !rho) return fail(ICTC_ERR_ARGUMENT, "radial MLP: null operand");
  if (!dr && (!dda3 || v || z3rows || a2rows || z2rows || a1rows || z1rows || brows))
    return fail(ICTC_ERR_ARGUMENT, "radial MLP: without dr only dda3 is written");
  const float* rows[] = {z3rows, a2rows, z2rows, a1rows, z1rows, brows};
  const bool any = z3rows || a2rows || z2rows || a1rows || z1rows || brows;
  for (const float* q : rows)
    if (any && !q) return fail(ICTC_ERR_ARGUMENT, "radial MLP: weight-gradient rows are all given or all null");
  for (const float* q : {da3, v, (const float*)dda3, (const float*)z3rows, (const float*)a2rows, (const float*)z2rows,
                         (const float*)a1rows, (const float*)z1rows})
    if (q && !aligned16(q)) return fail(ICTC_ERR_ARGUMENT, "radial MLP: [E, 64] operands must be 16-byte aligned");
  if (brows && (reinterpret_cast<uintptr_t>(brows) & 7))
    return fail(ICTC_ERR_ARGUMENT, "radial MLP: radial rows must be 8-byte aligned");
  if (!dr) {   // d da3 = rho t3 alone: the forward-tangent kernel (3 blocks per CU)
    const int tan_per_cu = resident_per_cu(mlp_tan_kernel, FWD_WAVES * 64, 3);
    hipLaunchKernelGGL(mlp_tan_kernel, dim3(grid_for(edges, FWD_WAVES, tan_per_cu)), dim3(FWD_WAVES * 64), 0,
                       (hipStream_t)stream, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, rho, nullptr, dda3);
    return launch_status("ictc_radial_mlp_bwd2 launch");
  }
  const int per_cu = resident_per_cu(mlp_bwd2_kernel, BWD2_WAVES * 64, 1);
  hipLaunchKernelGGL(mlp_bwd2_kernel, dim3(grid_for(edges, BWD2_WAVES, per_cu)), dim3(BWD2_WAVES * 64), 0,
                     (hipStream_t)stream, r, edges, cutoff, poly_p, W1, W2, W3, silu_scale, da3, rho, v, dr, dda3,
                     z3rows, a2rows, z2rows, a1rows, z1rows, brows);
  return launch_status("ictc_radial_mlp_bwd2 launch");
}

}  // extern "C"
