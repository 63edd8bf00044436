// Edge geometry of the interaction input (mace_ictc/models/pure_cartesian_ictd_layers.py:
// 1288-1297): vec = pos[dst] - pos[src] + shift, r = |vec|, n = vec / max(r, 1e-8),
// mask = [r <= cutoff], and the first adjoint back to the positions.
//
// The adjoint is a deterministic gather, not a scatter: node i sums the edge
// adjoints of its incoming edges (receiver-sorted CSR) and subtracts those of
// its outgoing edges (source-sorted CSR) in a fixed order, so the result is
// bitwise reproducible and needs no float atomics.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ictc_mi355x.h"
#include "generated/ictc_tables.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

constexpr int kBlock = 256;
constexpr float kClamp = 1e-8f;

__global__ __launch_bounds__(kBlock) void geometry_fwd_kernel(const float* __restrict__ pos,
                                                              const float* __restrict__ shift,
                                                              const int64_t* __restrict__ src,
                                                              const int64_t* __restrict__ dst, int64_t E, float rc,
                                                              float* __restrict__ r, float* __restrict__ n,
                                                              float* __restrict__ mask) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= E) return;
  const int64_t s = src[e], d = dst[e];
  float v[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) v[c] = pos[3 * d + c] - pos[3 * s + c] + (shift ? shift[3 * e + c] : 0.f);
  const float len = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
  const float den = fmaxf(len, kClamp);
  r[e] = len;
#pragma unroll
  for (int c = 0; c < 3; ++c) n[3 * e + c] = v[c] / den;
  if (mask) mask[e] = len <= rc ? 1.f : 0.f;
}

// d vec of one edge from dr and dn:
//   dr * vec / r + dn / max(r, eps) - [r > eps] (dn . vec) vec / (max(r, eps)^2 r)
// which for r > eps is dr n + (dn - (dn . n) n) / r.
__device__ __forceinline__ void edge_adjoint_values(float len, float nx, float ny, float nz, float g,
                                                    const float* a, float* out) {
  if (len > kClamp) {
    const float inv = 1.f / len, dot = a[0] * nx + a[1] * ny + a[2] * nz;
    out[0] = g * nx + (a[0] - dot * nx) * inv;
    out[1] = g * ny + (a[1] - dot * ny) * inv;
    out[2] = g * nz + (a[2] - dot * nz) * inv;
  } else {
    // Here vec = n * eps: dr vec / r = dr (eps / r) n (0 at r = 0, torch's convention), and the clamp passes no gradient.
    const float inv = 1.f / kClamp, gr = len > 0.f ? g * kClamp / len : 0.f;
    out[0] = gr * nx + a[0] * inv;
    out[1] = gr * ny + a[1] * inv;
    out[2] = gr * nz + a[2] * inv;
  }
}

__device__ __forceinline__ void edge_adjoint(const float* __restrict__ r, const float* __restrict__ n,
                                             const float* __restrict__ dr, const float* __restrict__ dn, int64_t e,
                                             float* out) {
  float a[3] = {0.f, 0.f, 0.f};
  if (dn) {
    a[0] = dn[3 * e];
    a[1] = dn[3 * e + 1];
    a[2] = dn[3 * e + 2];
  }
  edge_adjoint_values(r[e], n[3 * e], n[3 * e + 1], n[3 * e + 2], dr ? dr[e] : 0.f, a, out);
}

template <bool VEC>
__device__ __forceinline__ void edge_cotangent(const float* __restrict__ r, const float* __restrict__ n,
                                               const float* __restrict__ dr, const float* __restrict__ dn,
                                               int64_t e, float* out) {
  if (VEC) {
#pragma unroll
    for (int c = 0; c < 3; ++c) out[c] = dn[3 * e + c];
  } else {
    edge_adjoint(r, n, dr, dn, e, out);
  }
}

// One wave per node: dpos[i] = sum_{dst(e)=i} dvec_e - sum_{src(e)=i} dvec_e.
// Lane j takes CSR positions j, j+64, ... of the node's incoming and outgoing
// segments (coalesced index reads, independent gathers in flight across the
// lanes); the lanes' partial sums are combined by a fixed butterfly, so the
// result is still bitwise reproducible.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

// VEC: the cotangent is given per edge vector (dn holds dvec [E, 3]; r, n, dr unused).
template <bool VEC>
__global__ __launch_bounds__(kBlock) void geometry_bwd_kernel(const float* __restrict__ r,
                                                              const float* __restrict__ n,
                                                              const float* __restrict__ dr,
                                                              const float* __restrict__ dn, int64_t N,
                                                              const int32_t* __restrict__ dptr,
                                                              const int32_t* __restrict__ dord,
                                                              const int32_t* __restrict__ sptr,
                                                              const int32_t* __restrict__ sord,
                                                              float* __restrict__ dshift,
                                                              float* __restrict__ dpos) {
  const int64_t i = (int64_t)blockIdx.x * (kBlock / 64) + (threadIdx.x >> 6);
  if (i >= N) return;
  const int lane = threadIdx.x & 63;
  float acc[3] = {0.f, 0.f, 0.f}, t[3];
  for (int32_t k = dptr[i] + lane; k < dptr[i + 1]; k += 64) {
    const int64_t e = dord ? dord[k] : k;   // dord == nullptr: edges already receiver-sorted
    edge_cotangent<VEC>(r, n, dr, dn, e, t);
#pragma unroll
    for (int c = 0; c < 3; ++c) acc[c] += t[c];
    if (dshift) {
#pragma unroll
      for (int c = 0; c < 3; ++c) dshift[3 * e + c] = t[c];
    }
  }
  for (int32_t k = sptr[i] + lane; k < sptr[i + 1]; k += 64) {
    edge_cotangent<VEC>(r, n, dr, dn, sord[k], t);
#pragma unroll
    for (int c = 0; c < 3; ++c) acc[c] -= t[c];
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) acc[c] = wave_sum(acc[c]);
  if (lane < 3) dpos[3 * i + lane] = lane == 0 ? acc[0] : (lane == 1 ? acc[1] : acc[2]);
}

// Edge geometry and direction harmonics in one pass (first-order E+F route): r, n (kept for the adjoint),
// mask and Y = Sh<L>(n), with n and Y computed exactly as geometry_fwd_kernel and sh_fwd_kernel do.
// Rows of NV floats per edge, for the kBlock edges of a block, move between global memory and LDS as one
// contiguous span (16-byte vectors over the block's rows, then the tail), so each thread's row of the
// harmonics (9 floats at lmax 2) costs no strided 4-byte accesses.
template <int NV>
__device__ __forceinline__ void rows_to_lds(const float* __restrict__ g, int64_t base, int cnt, float* sm) {
  const float* src = g + base * NV;   // base is a multiple of kBlock: 16-byte aligned
  const int total = cnt * NV, n4 = total / 4;
  for (int i = threadIdx.x; i < n4; i += kBlock) reinterpret_cast<float4*>(sm)[i] = reinterpret_cast<const float4*>(src)[i];
  for (int i = 4 * n4 + threadIdx.x; i < total; i += kBlock) sm[i] = src[i];
}

template <int NV>
__device__ __forceinline__ void rows_from_lds(float* __restrict__ g, int64_t base, int cnt, const float* sm) {
  float* dst = g + base * NV;
  const int total = cnt * NV, n4 = total / 4;
  for (int i = threadIdx.x; i < n4; i += kBlock) reinterpret_cast<float4*>(dst)[i] = reinterpret_cast<const float4*>(sm)[i];
  for (int i = 4 * n4 + threadIdx.x; i < total; i += kBlock) dst[i] = sm[i];
}

// Edge geometry and direction harmonics in one pass (first-order E+F route): r, n (kept for the adjoint),
// mask and Y = Sh<L>(n), with n and Y computed exactly as geometry_fwd_kernel and sh_fwd_kernel do.
template <int L>
__global__ __launch_bounds__(kBlock) void geometry_sh_fwd_kernel(const float* __restrict__ pos,
                                                                 const float* __restrict__ shift,
                                                                 const int64_t* __restrict__ src,
                                                                 const int64_t* __restrict__ dst, int64_t E,
                                                                 float rc, float* __restrict__ r,
                                                                 float* __restrict__ n, float* __restrict__ mask,
                                                                 float* __restrict__ Y) {
  constexpr int NY = ictc::Sh<L>::N;
  __shared__ __align__(16) float sy[kBlock * NY];
  const int64_t base = (int64_t)blockIdx.x * kBlock, e = base + threadIdx.x;
  const int cnt = (int)(E - base < kBlock ? E - base : kBlock);
  if (e < E) {
    const int64_t s = src[e], d = dst[e];
    float v[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) v[c] = pos[3 * d + c] - pos[3 * s + c] + (shift ? shift[3 * e + c] : 0.f);
    const float len = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    const float den = fmaxf(len, kClamp);
    r[e] = len;
    float u[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      u[c] = v[c] / den;
      n[3 * e + c] = u[c];
    }
    if (mask) mask[e] = len <= rc ? 1.f : 0.f;
    float y[NY];
    ictc::Sh<L>::fwd(u[0], u[1], u[2], y);
#pragma unroll
    for (int k = 0; k < NY; ++k) sy[threadIdx.x * NY + k] = y[k];
  }
  __syncthreads();
  rows_from_lds<NY>(Y, base, cnt, sy);
}

// Its adjoint per edge: dn = Sh<L> adjoint of dY (as sh_bwd_kernel), then d vec from dr and dn (as
// edge_adjoint), written per edge for the CSR gather geometry_bwd_kernel<true>.  dY2 / dr2 (optional): a
// second consumer's cotangents, added to dY / dr first (the sum autograd would form, in the same rounding).
template <int L>
__global__ __launch_bounds__(kBlock) void geometry_sh_bwd_kernel(const float* __restrict__ r,
                                                                 const float* __restrict__ n,
                                                                 const float* __restrict__ dr,
                                                                 const float* __restrict__ dY,
                                                                 const float* __restrict__ dr2,
                                                                 const float* __restrict__ dY2, int64_t E,
                                                                 float* __restrict__ dvec) {
  constexpr int NY = ictc::Sh<L>::N;
  __shared__ __align__(16) float sa[kBlock * NY];
  __shared__ __align__(16) float sb[kBlock * NY];
  const int64_t base = (int64_t)blockIdx.x * kBlock, e = base + threadIdx.x;
  const int cnt = (int)(E - base < kBlock ? E - base : kBlock);
  if (dY) rows_to_lds<NY>(dY, base, cnt, sa);
  if (dY2) rows_to_lds<NY>(dY2, base, cnt, sb);
  __syncthreads();
  if (e >= E) return;
  float dn[3] = {0.f, 0.f, 0.f};
  if (dY || dY2) {
    float g[NY];
#pragma unroll
    for (int k = 0; k < NY; ++k) {
      const int i = threadIdx.x * NY + k;
      g[k] = dY ? (dY2 ? sa[i] + sb[i] : sa[i]) : sb[i];
    }
    ictc::Sh<L>::bwd(n[3 * e], n[3 * e + 1], n[3 * e + 2], g, dn[0], dn[1], dn[2]);
  }
  const float gr = dr ? (dr2 ? dr[e] + dr2[e] : dr[e]) : (dr2 ? dr2[e] : 0.f);
  float t[3];
  edge_adjoint_values(r[e], n[3 * e], n[3 * e + 1], n[3 * e + 2], gr, dn, t);
#pragma unroll
  for (int c = 0; c < 3; ++c) dvec[3 * e + c] = t[c];
}

// Unit vectors of given edge vectors (the second-order route, where vec is an autograd input):
// r = |v|, n = v / max(r, eps); the first adjoint gv(v, gr, gn) as edge_adjoint_values; and that
// adjoint's derivative for a cotangent h on gv: with P x = (x - (x . n) n) / r (r > eps)
//   d gr = n . h,   d gn = P h,
//   d v  = gr P h - ((h . n) P gn + (gn . n) P h) / r - (gn . h - (gn . n)(h . n)) n / r^2.
// Below eps n = v / eps and gv = gr v / r + gn / eps: d gr = (v / r) . h, d gn = h / eps,
// d v = gr (h - (h . u) u) / r with u = v / r (zero at r = 0).
__global__ __launch_bounds__(kBlock) void unit_fwd_kernel(const float* __restrict__ v, int64_t E,
                                                          float* __restrict__ r, float* __restrict__ n) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= E) return;
  const float x = v[3 * e], y = v[3 * e + 1], z = v[3 * e + 2];
  const float len = sqrtf(x * x + y * y + z * z), den = fmaxf(len, kClamp);
  r[e] = len;
  n[3 * e] = x / den;
  n[3 * e + 1] = y / den;
  n[3 * e + 2] = z / den;
}

__global__ __launch_bounds__(kBlock) void unit_bwd_kernel(const float* __restrict__ r, const float* __restrict__ n,
                                                          const float* __restrict__ gr, const float* __restrict__ gn,
                                                          int64_t E, float* __restrict__ gv) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= E) return;
  const float a[3] = {gn ? gn[3 * e] : 0.f, gn ? gn[3 * e + 1] : 0.f, gn ? gn[3 * e + 2] : 0.f};
  float out[3];
  edge_adjoint_values(r[e], n[3 * e], n[3 * e + 1], n[3 * e + 2], gr ? gr[e] : 0.f, a, out);
#pragma unroll
  for (int c = 0; c < 3; ++c) gv[3 * e + c] = out[c];
}

__global__ __launch_bounds__(kBlock) void unit_bwd2_kernel(const float* __restrict__ r, const float* __restrict__ n,
                                                           const float* __restrict__ gr, const float* __restrict__ gn,
                                                           const float* __restrict__ h, int64_t E,
                                                           float* __restrict__ dv, float* __restrict__ dgr,
                                                           float* __restrict__ dgn) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= E) return;
  const float len = r[e], g = gr ? gr[e] : 0.f;
  const float nn[3] = {n[3 * e], n[3 * e + 1], n[3 * e + 2]};
  const float hv[3] = {h[3 * e], h[3 * e + 1], h[3 * e + 2]};
  const float a[3] = {gn ? gn[3 * e] : 0.f, gn ? gn[3 * e + 1] : 0.f, gn ? gn[3 * e + 2] : 0.f};
  float o[3], ogn[3], ogr;
  if (len > kClamp) {
    const float inv = 1.f / len;
    const float hn = hv[0] * nn[0] + hv[1] * nn[1] + hv[2] * nn[2];
    const float an = a[0] * nn[0] + a[1] * nn[1] + a[2] * nn[2];
    const float ah = a[0] * hv[0] + a[1] * hv[1] + a[2] * hv[2];
    ogr = hn;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float ph = (hv[c] - hn * nn[c]) * inv;   // P h
      const float pa = (a[c] - an * nn[c]) * inv;    // P gn
      ogn[c] = ph;
      o[c] = g * ph - (hn * pa + an * ph) * inv - (ah - an * hn) * nn[c] * inv * inv;
    }
  } else {
    const float inv = 1.f / kClamp;
    if (len > 0.f) {
      // u = v / r = n * eps / r
      const float s = kClamp / len, u[3] = {nn[0] * s, nn[1] * s, nn[2] * s};
      const float hu = hv[0] * u[0] + hv[1] * u[1] + hv[2] * u[2];
      ogr = hu;
#pragma unroll
      for (int c = 0; c < 3; ++c) o[c] = g * (hv[c] - hu * u[c]) / len;
    } else {
      ogr = 0.f;
#pragma unroll
      for (int c = 0; c < 3; ++c) o[c] = 0.f;
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) ogn[c] = hv[c] * inv;
  }
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    if (dv) dv[3 * e + c] = o[c];
    if (dgn) dgn[3 * e + c] = ogn[c];
  }
  if (dgr) dgr[e] = ogr;
}

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return ICTC_OK;
  char buf[256];
  snprintf(buf, sizeof(buf), "%s: %s", what, hipGetErrorString(e));
  return fail(ICTC_ERR_RUNTIME, buf);
}

// out[e, j] = (s0 c0j + s1 c1j) + s2 c2j with each product and sum rounded on its own (no contraction): the
// same operations for an edge and its reverse (shift -S), so their image shifts are exact negations.
__global__ __launch_bounds__(kBlock) void shift_vectors_kernel(const float* __restrict__ shifts, int64_t E,
                                                               const float* __restrict__ cell, int64_t cells,
                                                               const int64_t* __restrict__ batch,
                                                               const int64_t* __restrict__ src, int64_t N,
                                                               float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (e >= E) return;
  int64_t g = 0;
  if (batch) {
    const int64_t s = src[e];
    g = (s >= 0 && s < N) ? batch[s] : -1;
  }
  const float s0 = shifts[3 * e], s1 = shifts[3 * e + 1], s2 = shifts[3 * e + 2];
  if (g < 0 || g >= cells) {
    const float nan = __int_as_float(0x7fc00000);
    out[3 * e] = nan; out[3 * e + 1] = nan; out[3 * e + 2] = nan;
    return;
  }
  const float* c = cell + 9 * g;
#pragma unroll
  for (int j = 0; j < 3; ++j)
    out[3 * e + j] = __fadd_rn(__fadd_rn(__fmul_rn(s0, c[j]), __fmul_rn(s1, c[3 + j])), __fmul_rn(s2, c[6 + j]));
}

}  // namespace

extern "C" {

int ictc_edge_geometry_fwd(const float* pos, const float* shift, const int64_t* src, const int64_t* dst,
                           int64_t nodes, int64_t edges, float cutoff, float* r, float* n, float* mask,
                           void* stream) {
  if (nodes < 0 || edges < 0) return fail(ICTC_ERR_ARGUMENT, "edge geometry: negative size");
  if (edges == 0) return ICTC_OK;
  if (!pos || !src || !dst || !r || !n) return fail(ICTC_ERR_ARGUMENT, "edge geometry: null operand");
  hipLaunchKernelGGL(geometry_fwd_kernel, dim3((unsigned)((edges + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                     (hipStream_t)stream, pos, shift, src, dst, edges, cutoff, r, n, mask);
  return launch_status("ictc_edge_geometry_fwd launch");
}

int ictc_edge_harmonics_fwd(const float* pos, const float* shift, const int64_t* src, const int64_t* dst,
                            int64_t nodes, int64_t edges, float cutoff, int lmax, float* r, float* n, float* mask,
                            float* Y, void* stream) {
  if (nodes < 0 || edges < 0) return fail(ICTC_ERR_ARGUMENT, "edge harmonics: negative size");
  if (lmax < 0 || lmax > 3) return fail(ICTC_ERR_UNSUPPORTED, "edge harmonics: lmax outside 0..3");
  if (edges == 0) return ICTC_OK;
  if (!pos || !src || !dst || !r || !n || !Y) return fail(ICTC_ERR_ARGUMENT, "edge harmonics: null operand");
  if (reinterpret_cast<uintptr_t>(Y) % 16) return fail(ICTC_ERR_ARGUMENT, "edge harmonics: Y must be 16-byte aligned");
  const dim3 grid((unsigned)((edges + kBlock - 1) / kBlock));
  hipStream_t st = (hipStream_t)stream;
  switch (lmax) {
    case 0: hipLaunchKernelGGL(geometry_sh_fwd_kernel<0>, grid, dim3(kBlock), 0, st, pos, shift, src, dst, edges, cutoff, r, n, mask, Y); break;
    case 1: hipLaunchKernelGGL(geometry_sh_fwd_kernel<1>, grid, dim3(kBlock), 0, st, pos, shift, src, dst, edges, cutoff, r, n, mask, Y); break;
    case 2: hipLaunchKernelGGL(geometry_sh_fwd_kernel<2>, grid, dim3(kBlock), 0, st, pos, shift, src, dst, edges, cutoff, r, n, mask, Y); break;
    default: hipLaunchKernelGGL(geometry_sh_fwd_kernel<3>, grid, dim3(kBlock), 0, st, pos, shift, src, dst, edges, cutoff, r, n, mask, Y); break;
  }
  return launch_status("ictc_edge_harmonics_fwd launch");
}

int ictc_edge_harmonics_bwd(const float* r, const float* n, const float* dr, const float* dY, const float* dr2,
                            const float* dY2, int64_t edges, int lmax, float* dvec, void* stream) {
  if (edges < 0) return fail(ICTC_ERR_ARGUMENT, "edge harmonics adjoint: negative size");
  if (lmax < 0 || lmax > 3) return fail(ICTC_ERR_UNSUPPORTED, "edge harmonics adjoint: lmax outside 0..3");
  if (edges == 0) return ICTC_OK;
  if (!r || !n || !dvec) return fail(ICTC_ERR_ARGUMENT, "edge harmonics adjoint: null operand");
  if (reinterpret_cast<uintptr_t>(dY) % 16 || reinterpret_cast<uintptr_t>(dY2) % 16)
    return fail(ICTC_ERR_ARGUMENT, "edge harmonics adjoint: dY and dY2 must be 16-byte aligned");
  const dim3 grid((unsigned)((edges + kBlock - 1) / kBlock));
  hipStream_t st = (hipStream_t)stream;
  switch (lmax) {
    case 0: hipLaunchKernelGGL(geometry_sh_bwd_kernel<0>, grid, dim3(kBlock), 0, st, r, n, dr, dY, dr2, dY2, edges, dvec); break;
    case 1: hipLaunchKernelGGL(geometry_sh_bwd_kernel<1>, grid, dim3(kBlock), 0, st, r, n, dr, dY, dr2, dY2, edges, dvec); break;
    case 2: hipLaunchKernelGGL(geometry_sh_bwd_kernel<2>, grid, dim3(kBlock), 0, st, r, n, dr, dY, dr2, dY2, edges, dvec); break;
    default: hipLaunchKernelGGL(geometry_sh_bwd_kernel<3>, grid, dim3(kBlock), 0, st, r, n, dr, dY, dr2, dY2, edges, dvec); break;
  }
  return launch_status("ictc_edge_harmonics_bwd launch");
}

int ictc_shift_vectors(const float* shifts, int64_t edges, const float* cell, int64_t cells, const int64_t* batch,
                       const int64_t* src, int64_t nodes, float* out, void* stream) {
  if (edges < 0 || cells < 1 || nodes < 0) return fail(ICTC_ERR_ARGUMENT, "shift vectors: invalid size");
  if (edges == 0) return ICTC_OK;
  if (!shifts || !cell || !out || (cells > 1 && (!batch || !src)))
    return fail(ICTC_ERR_ARGUMENT, "shift vectors: null operand");
  hipLaunchKernelGGL(shift_vectors_kernel, dim3((unsigned)((edges + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                     (hipStream_t)stream, shifts, edges, cell, cells, cells > 1 ? batch : nullptr, src, nodes, out);
  return launch_status("ictc_shift_vectors launch");
}

int ictc_edge_geometry_bwd(const float* r, const float* n, const float* dr, const float* dn, int64_t nodes,
                           int64_t edges, const int32_t* dst_ptr, const int32_t* dst_order, const int32_t* src_ptr,
                           const int32_t* src_order, float* dshift, float* dpos, void* stream) {
  if (nodes < 0 || edges < 0) return fail(ICTC_ERR_ARGUMENT, "edge geometry: negative size");
  if (nodes == 0) return ICTC_OK;
  if (!dpos || !dst_ptr || !src_ptr || (edges > 0 && (!r || !n || !src_order)))
    return fail(ICTC_ERR_ARGUMENT, "edge geometry adjoint: null operand");
  hipLaunchKernelGGL(geometry_bwd_kernel<false>, dim3((unsigned)((nodes + kBlock / 64 - 1) / (kBlock / 64))), dim3(kBlock), 0,
                     (hipStream_t)stream, r, n, dr, dn, nodes, dst_ptr, dst_order, src_ptr, src_order, dshift, dpos);
  return launch_status("ictc_edge_geometry_bwd launch");
}

int ictc_edge_vector_bwd(const float* dvec, int64_t nodes, int64_t edges, const int32_t* dst_ptr,
                         const int32_t* dst_order, const int32_t* src_ptr, const int32_t* src_order, float* dpos,
                         void* stream) {
  if (nodes < 0 || edges < 0) return fail(ICTC_ERR_ARGUMENT, "edge vector adjoint: negative size");
  if (nodes == 0) return ICTC_OK;
  if (!dpos || !dst_ptr || !src_ptr || (edges > 0 && (!dvec || !src_order)))
    return fail(ICTC_ERR_ARGUMENT, "edge vector adjoint: null operand");
  hipLaunchKernelGGL(geometry_bwd_kernel<true>, dim3((unsigned)((nodes + kBlock / 64 - 1) / (kBlock / 64))),
                     dim3(kBlock), 0, (hipStream_t)stream, nullptr, nullptr, nullptr, dvec, nodes, dst_ptr, dst_order,
                     src_ptr, src_order, nullptr, dpos);
  return launch_status("ictc_edge_vector_bwd launch");
}

int ictc_edge_unit(int order, const float* v, const float* r, const float* n, const float* gr, const float* gn,
                   const float* h, int64_t edges, float* out0, float* out1, float* out2, void* stream) {
  if (edges < 0 || order < 0 || order > 2) return fail(ICTC_ERR_ARGUMENT, "edge_unit: order 0..2, edges >= 0");
  if (edges == 0) return ICTC_OK;
  const dim3 grid((unsigned)((edges + kBlock - 1) / kBlock));
  hipStream_t st = (hipStream_t)stream;
  if (order == 0) {
    if (!v || !out0 || !out1) return fail(ICTC_ERR_ARGUMENT, "edge_unit: null operand");
    hipLaunchKernelGGL(unit_fwd_kernel, grid, dim3(kBlock), 0, st, v, edges, out0, out1);
  } else if (order == 1) {
    if (!r || !n || !out0) return fail(ICTC_ERR_ARGUMENT, "edge_unit: null operand");
    hipLaunchKernelGGL(unit_bwd_kernel, grid, dim3(kBlock), 0, st, r, n, gr, gn, edges, out0);
  } else {
    if (!r || !n || !h) return fail(ICTC_ERR_ARGUMENT, "edge_unit: null operand");
    hipLaunchKernelGGL(unit_bwd2_kernel, grid, dim3(kBlock), 0, st, r, n, gr, gn, h, edges, out0, out1, out2);
  }
  return launch_status("ictc_edge_unit launch");
}

}  // extern "C"
