// Elementwise kernels of the radial path: normalized SiLU (fused_activation.py /
// hip_activation.py:11-36) and the Bessel x polynomial-cutoff radial basis
// (mace_ictc/models/radial_basis.py:11-92), each with first and second derivatives.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/ictc_mi355x.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

// mode 0: y = s x sig(x); 1: y = g s silu'(x); 2: y = g h s silu''(x)
// silu'(x) = sig (1 + x (1 - sig)); silu''(x) = sig (1 - sig) (2 + x (1 - 2 sig))
__global__ __launch_bounds__(kBlock) void silu_kernel(int mode, const float* __restrict__ x,
                                                      const float* __restrict__ g, const float* __restrict__ h,
                                                      float s, int64_t n, float* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const float v = x[i], sg = sigmoid(v);
  float r;
  if (mode == 0) r = s * v * sg;
  else if (mode == 1) r = g[i] * s * sg * (1.f + v * (1.f - sg));
  else r = g[i] * h[i] * s * sg * (1.f - sg) * (2.f + v * (1.f - 2.f * sg));
  y[i] = r;
}

// Same, four consecutive elements per thread (16-byte loads and stores; n a
// multiple of 4 and every operand 16-byte aligned).
__global__ __launch_bounds__(kBlock) void silu4_kernel(int mode, const float4* __restrict__ x,
                                                       const float4* __restrict__ g, const float4* __restrict__ h,
                                                       float s, int64_t n4, float4* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n4) return;
  const float4 v4 = x[i];
  float4 g4 = make_float4(1.f, 1.f, 1.f, 1.f), h4 = g4;
  if (mode >= 1) g4 = g[i];
  if (mode == 2) h4 = h[i];
  const float v[4] = {v4.x, v4.y, v4.z, v4.w}, gv[4] = {g4.x, g4.y, g4.z, g4.w}, hv[4] = {h4.x, h4.y, h4.z, h4.w};
  float r[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float sg = sigmoid(v[k]);
    if (mode == 0) r[k] = s * v[k] * sg;
    else if (mode == 1) r[k] = gv[k] * s * sg * (1.f + v[k] * (1.f - sg));
    else r[k] = gv[k] * hv[k] * s * sg * (1.f - sg) * (2.f + v[k] * (1.f - 2.f * sg));
  }
  y[i] = make_float4(r[0], r[1], r[2], r[3]);
}

// Radial basis b_k(r) = sqrt(2/rc) sin(k pi r/rc) / r * env(r/rc) * [r < rc], k = 1..K,
// env(u) = 1 - (p+1)(p+2)/2 u^p + p(p+2) u^(p+1) - p(p+1)/2 u^(p+2).
// order 0: out[e,k] = b_k; order 1: out[e] = sum_k g[e,k] b_k'(r);
// order 2: out[e] = sum_k g[e,k] b_k''(r) * h[e]; order 3: out[e,k] = b_k'(r) * h[e]
__global__ __launch_bounds__(kBlock) void radial_kernel(int order, const float* __restrict__ r,
                                                        const float* __restrict__ g, const float* __restrict__ h,
                                                        int64_t E, int K, float rc, int p,
                                                        float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= E) return;
  const float x = r[e];
  const bool inside = x < rc;
  const float u = x / rc;
  const float c1 = 0.5f * (p + 1) * (p + 2), c2 = (float)p * (p + 2), c3 = 0.5f * p * (p + 1);
  const float up = powf(u, (float)p);
  const float env = inside ? 1.f - c1 * up + c2 * up * u - c3 * up * u * u : 0.f;
  // d env / dr and d2 env / dr2
  const float upm1 = p >= 1 ? powf(u, (float)(p - 1)) : 0.f;
  const float upm2 = p >= 2 ? powf(u, (float)(p - 2)) : 0.f;
  const float denv = inside ? (-c1 * p * upm1 + c2 * (p + 1) * up - c3 * (p + 2) * up * u) / rc : 0.f;
  const float d2env =
      inside ? (-c1 * p * (p - 1) * upm2 + c2 * (p + 1) * p * upm1 - c3 * (p + 2) * (p + 1) * up) / (rc * rc) : 0.f;
  const float pre = sqrtf(2.f / rc);
  const float xr = fmaxf(x, 1e-12f);
  const float inv = 1.f / xr;
  float acc = 0.f;
  for (int k = 1; k <= K; ++k) {
    const float w = k * 3.14159265358979323846f / rc;
    float sn, cs;
    sincosf(w * x, &sn, &cs);
    const float f = pre * sn * inv;                                   // sin(w r)/r
    const float df = pre * (w * cs * inv - sn * inv * inv);          // d/dr
    const float d2f = pre * (-w * w * sn * inv - 2.f * w * cs * inv * inv + 2.f * sn * inv * inv * inv);
    const float b = f * env;
    const float db = df * env + f * denv;
    const float d2b = d2f * env + 2.f * df * denv + f * d2env;
    if (order == 0) out[e * K + (k - 1)] = b;
    else if (order == 1) acc = fmaf(g[e * K + (k - 1)], db, acc);
    else if (order == 2) acc = fmaf(g[e * K + (k - 1)], d2b, acc);
    else out[e * K + (k - 1)] = db * h[e];
  }
  if (order == 1) out[e] = acc;
  else if (order == 2) out[e] = acc * h[e];
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

int ictc_silu(int mode, const float* x, const float* grad, const float* tangent, float scale, int64_t n, float* out,
              void* stream) {
  if (mode < 0 || mode > 2) return fail(ICTC_ERR_ARGUMENT, "silu mode must be 0, 1 or 2");
  if (n < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  if (n == 0) return ICTC_OK;
  if (!x || !out || (mode >= 1 && !grad) || (mode == 2 && !tangent))
    return fail(ICTC_ERR_ARGUMENT, "ictc_silu: null operand");
  const bool vec = n % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                                    reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(tangent)) & 15) == 0;
  if (vec) {
    const int64_t n4 = n / 4;
    hipLaunchKernelGGL(silu4_kernel, dim3((unsigned)((n4 + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                       (hipStream_t)stream, mode, (const float4*)x, (const float4*)grad, (const float4*)tangent, scale,
                       n4, (float4*)out);
    return launch_status("ictc_silu launch");
  }
  hipLaunchKernelGGL(silu_kernel, dim3((unsigned)((n + kBlock - 1) / kBlock)), dim3(kBlock), 0, (hipStream_t)stream,
                     mode, x, grad, tangent, scale, n, out);
  return launch_status("ictc_silu launch");
}

int ictc_radial(int order, const float* r, const float* grad, const float* tangent, int64_t edges, int num_basis,
                float cutoff, int poly_p, float* out, void* stream) {
  if (order < 0 || order > 3) return fail(ICTC_ERR_ARGUMENT, "radial order must be 0..3");
  if (edges < 0 || num_basis < 1 || !(cutoff > 0.f) || poly_p < 1)
    return fail(ICTC_ERR_ARGUMENT, "radial: invalid size / cutoff / polynomial order");
  if (edges == 0) return ICTC_OK;
  if (!r || !out || ((order == 1 || order == 2) && !grad) || (order >= 2 && !tangent))
    return fail(ICTC_ERR_ARGUMENT, "ictc_radial: null operand");
  hipLaunchKernelGGL(radial_kernel, dim3((unsigned)((edges + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                     (hipStream_t)stream, order, r, grad, tangent, edges, num_basis, cutoff, poly_p, out);
  return launch_status("ictc_radial launch");
}

}  // extern "C"
