// Per-edge tensor product, CSR graph message and direction-harmonic kernels
// for gfx950 (CDNA4, wave64).
//
// Data layout in HBM (all FP32, row-major, "component-major, channel-minor"):
//   node / edge features  [rows, NX*C]   component k = l*l+m at k*C + c
//   harmonics             [E, NY]        NY = (LE+1)^2
//   gates                 [E, P*C]       path p at p*C + c
//   TP output             [rows, NO*C]   output slot k at k*C + c
// One wave owns one row (an edge for the edge TP, a node for the CSR message)
// and one lane owns channel c = lane + 64*j (j < CPL), so every feature,
// gate and output access is a fully coalesced 256-byte wave transaction and
// every per-edge scalar (indices, harmonics, mask) is wave-uniform.
//
// The graph message is deterministic and float-atomic free: the forward and
// the gate / harmonic adjoints run over the receiver-sorted CSR (one owner per
// output row); the feature adjoint runs over the source-sorted CSR.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "generated/ictc_tables.h"

namespace ictc {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

struct Operands {
  const float* x;       // features (edge rows for the edge TP, node rows for messages)
  const float* sh;      // [E, NY]
  const float* gates;   // [E, P*C]
  const float* weight;  // [P, C] or nullptr for unit coefficients
  const float* mask;    // [E] or nullptr
  int64_t rows;         // E (edge TP) or N (message)
  int64_t edges;
  int channels;
};

template <class T>
__device__ __forceinline__ void load_harmonics(const float* __restrict__ sh, int64_t e, float* y) {
  const float* p = sh + e * T::NY;
#pragma unroll
  for (int j = 0; j < T::NY; ++j) y[j] = p[j];
}

template <class T>
__device__ __forceinline__ void load_gw(const Operands& a, int64_t e, int c, float scale, float* gw) {
  const float* g = a.gates + e * (int64_t)(T::P * a.channels) + c;
#pragma unroll
  for (int p = 0; p < T::P; ++p) {
    float v = g[p * a.channels] * scale;
    if (a.weight) v *= a.weight[p * a.channels + c];
    gw[p] = v;
  }
}

template <int N>
__device__ __forceinline__ void load_row(const float* __restrict__ base, int C, int c, float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = base[i * C + c];
}

template <int N>
__device__ __forceinline__ void store_row(float* __restrict__ base, int C, int c, const float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) base[i * C + c] = v[i];
}

// ---------------------------------------------------------------------------
// Edge TP: one wave per edge.
// ---------------------------------------------------------------------------
template <class T, int CPL>
__global__ __launch_bounds__(kBlock) void edge_fwd_kernel(Operands a, float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * kWavesPerBlock + wave_id();
  if (e >= a.rows) return;
  const int C = a.channels;
  float y[T::NY];
  load_harmonics<T>(a.sh, e, y);
  const float* xr = a.x + e * (int64_t)(T::NX * C);
  float* orow = out + e * (int64_t)(T::NO * C);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane_id() + kWave * j;
    if (c < C) {
      float xv[T::NX], gw[T::P], o[T::NO];
      load_row<T::NX>(xr, C, c, xv);
      load_gw<T>(a, e, c, 1.f, gw);
#pragma unroll
      for (int k = 0; k < T::NO; ++k) o[k] = 0.f;
      T::fwd(xv, y, gw, o);
      store_row<T::NO>(orow, C, c, o);
    }
  }
}

template <class T, int CPL>
__global__ __launch_bounds__(kBlock) void edge_bwd_kernel(Operands a, const float* __restrict__ grad,
                                                          float* __restrict__ dx, float* __restrict__ dsh,
                                                          float* __restrict__ dgates) {
  const int64_t e = (int64_t)blockIdx.x * kWavesPerBlock + wave_id();
  if (e >= a.rows) return;
  const int C = a.channels;
  float y[T::NY], dyv[T::NY];
  load_harmonics<T>(a.sh, e, y);
#pragma unroll
  for (int j = 0; j < T::NY; ++j) dyv[j] = 0.f;
  const float* xr = a.x + e * (int64_t)(T::NX * C);
  const float* gr = grad + e * (int64_t)(T::NO * C);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane_id() + kWave * j;
    if (c < C) {
      float xv[T::NX], gw[T::P], go[T::NO];
      load_row<T::NX>(xr, C, c, xv);
      load_row<T::NO>(gr, C, c, go);
      load_gw<T>(a, e, c, 1.f, gw);
      if (dx) {
        float d[T::NX];
#pragma unroll
        for (int i = 0; i < T::NX; ++i) d[i] = 0.f;
        T::dx(y, gw, go, d);
        store_row<T::NX>(dx + e * (int64_t)(T::NX * C), C, c, d);
      }
      if (dsh) T::dy(xv, gw, go, dyv);
      if (dgates) {
        float d[T::P];
        T::dg(xv, y, go, d);
#pragma unroll
        for (int p = 0; p < T::P; ++p) {
          if (a.weight) d[p] *= a.weight[p * C + c];
        }
        store_row<T::P>(dgates + e * (int64_t)(T::P * C), C, c, d);
      }
    }
  }
  if (dsh) {
#pragma unroll
    for (int j = 0; j < T::NY; ++j) {
      const float s = wave_sum(dyv[j]);
      if (lane_id() == 0) dsh[e * T::NY + j] = s;
    }
  }
}

// ---------------------------------------------------------------------------
// CSR graph message.  ptr/order describe the receiver-sorted (dst) CSR: the
// edges into node n are order[ptr[n] .. ptr[n+1]) (order == nullptr: edges are
// already sorted and order is the identity).
// ---------------------------------------------------------------------------
struct Csr {
  const int32_t* ptr;    // [N+2]: ptr[N]..ptr[N+1] holds out-of-range edges
  const int32_t* order;  // [E] or nullptr
};

template <class T, int CPL>
__global__ __launch_bounds__(kBlock) void msg_fwd_kernel(Operands a, const int64_t* __restrict__ src, Csr csr,
                                                         float* __restrict__ out) {
  const int64_t n = (int64_t)blockIdx.x * kWavesPerBlock + wave_id();
  if (n >= a.rows) return;
  const int C = a.channels;
  float o[CPL][T::NO];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int k = 0; k < T::NO; ++k) o[j][k] = 0.f;
  const int32_t beg = csr.ptr[n], end = csr.ptr[n + 1];
  for (int32_t k = beg; k < end; ++k) {
    const int64_t e = csr.order ? (int64_t)csr.order[k] : (int64_t)k;
    const int64_t s = src[e];
    if (s < 0 || s >= a.rows) continue;
    const float m = a.mask ? a.mask[e] : 1.f;
    float y[T::NY];
    load_harmonics<T>(a.sh, e, y);
    const float* xr = a.x + s * (int64_t)(T::NX * C);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane_id() + kWave * j;
      if (c < C) {
        float xv[T::NX], gw[T::P];
        load_row<T::NX>(xr, C, c, xv);
        load_gw<T>(a, e, c, m, gw);
        T::fwd(xv, y, gw, o[j]);
      }
    }
  }
  float* orow = out + n * (int64_t)(T::NO * C);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane_id() + kWave * j;
    if (c < C) store_row<T::NO>(orow, C, c, o[j]);
  }
}

// Receiver-owned adjoint: per-edge gate and harmonic gradients.
template <class T, int CPL>
__global__ __launch_bounds__(kBlock) void msg_bwd_edge_kernel(Operands a, const int64_t* __restrict__ src, Csr csr,
                                                              const float* __restrict__ grad,
                                                              float* __restrict__ dsh, float* __restrict__ dgates) {
  // Waves 0..rows-1 own receivers; wave `rows` owns the out-of-range tail
  // segment ptr[rows]..ptr[rows+1] and writes zero gradients for it.
  const int64_t n = (int64_t)blockIdx.x * kWavesPerBlock + wave_id();
  if (n > a.rows) return;
  const bool tail = n == a.rows;
  const int C = a.channels;
  float go[CPL][T::NO];
  const float* gr = grad + (tail ? 0 : n) * (int64_t)(T::NO * C);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane_id() + kWave * j;
    if (c < C && !tail) load_row<T::NO>(gr, C, c, go[j]);
    else {
#pragma unroll
      for (int k = 0; k < T::NO; ++k) go[j][k] = 0.f;
    }
  }
  const int32_t beg = csr.ptr[n], end = csr.ptr[n + 1];
  for (int32_t k = beg; k < end; ++k) {
    const int64_t e = csr.order ? (int64_t)csr.order[k] : (int64_t)k;
    const int64_t s = src[e];
    const bool valid = s >= 0 && s < a.rows;
    const float m = a.mask ? a.mask[e] : 1.f;
    float y[T::NY], dyv[T::NY];
    load_harmonics<T>(a.sh, e, y);
#pragma unroll
    for (int j = 0; j < T::NY; ++j) dyv[j] = 0.f;
    const float* xr = a.x + (valid ? s : 0) * (int64_t)(T::NX * C);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane_id() + kWave * j;
      if (c < C) {
        float xv[T::NX];
        if (valid) load_row<T::NX>(xr, C, c, xv);
        else {
#pragma unroll
          for (int i = 0; i < T::NX; ++i) xv[i] = 0.f;
        }
        if (dsh) {
          float gw[T::P];
          load_gw<T>(a, e, c, m, gw);
          T::dy(xv, gw, go[j], dyv);
        }
        if (dgates) {
          float d[T::P];
          T::dg(xv, y, go[j], d);
#pragma unroll
          for (int p = 0; p < T::P; ++p) {
            float v = d[p] * m;
            if (a.weight) v *= a.weight[p * C + c];
            d[p] = v;
          }
          store_row<T::P>(dgates + e * (int64_t)(T::P * C), C, c, d);
        }
      }
    }
    if (dsh) {
#pragma unroll
      for (int j = 0; j < T::NY; ++j) {
        const float s2 = wave_sum(dyv[j]);
        if (lane_id() == 0) dsh[e * T::NY + j] = s2;
      }
    }
  }
}

// Source-owned adjoint: node feature gradient over the source-sorted CSR.
template <class T, int CPL>
__global__ __launch_bounds__(kBlock) void msg_bwd_x_kernel(Operands a, const int64_t* __restrict__ dst, Csr scsr,
                                                           const float* __restrict__ grad, float* __restrict__ dx) {
  const int64_t n = (int64_t)blockIdx.x * kWavesPerBlock + wave_id();
  if (n >= a.rows) return;
  const int C = a.channels;
  float d[CPL][T::NX];
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int i = 0; i < T::NX; ++i) d[j][i] = 0.f;
  const int32_t beg = scsr.ptr[n], end = scsr.ptr[n + 1];
  for (int32_t k = beg; k < end; ++k) {
    const int64_t e = scsr.order ? (int64_t)scsr.order[k] : (int64_t)k;
    const int64_t r = dst[e];
    if (r < 0 || r >= a.rows) continue;
    const float m = a.mask ? a.mask[e] : 1.f;
    float y[T::NY];
    load_harmonics<T>(a.sh, e, y);
    const float* gr = grad + r * (int64_t)(T::NO * C);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane_id() + kWave * j;
      if (c < C) {
        float go[T::NO], gw[T::P];
        load_row<T::NO>(gr, C, c, go);
        load_gw<T>(a, e, c, m, gw);
        T::dx(y, gw, go, d[j]);
      }
    }
  }
  float* xr = dx + n * (int64_t)(T::NX * C);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane_id() + kWave * j;
    if (c < C) store_row<T::NX>(xr, C, c, d[j]);
  }
}

// ---------------------------------------------------------------------------
// Direction harmonics: one thread per edge.
// ---------------------------------------------------------------------------
template <int L>
__global__ __launch_bounds__(256) void sh_fwd_kernel(const float* __restrict__ n, int64_t E, float* __restrict__ Y) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float v[Sh<L>::N];
  Sh<L>::fwd(n[3 * e], n[3 * e + 1], n[3 * e + 2], v);
#pragma unroll
  for (int k = 0; k < Sh<L>::N; ++k) Y[e * Sh<L>::N + k] = v[k];
}

template <int L>
__global__ __launch_bounds__(256) void sh_bwd_kernel(const float* __restrict__ n, const float* __restrict__ gY,
                                                     int64_t E, float* __restrict__ gn) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float g[Sh<L>::N];
#pragma unroll
  for (int k = 0; k < Sh<L>::N; ++k) g[k] = gY[e * Sh<L>::N + k];
  float gx, gy, gz;
  Sh<L>::bwd(n[3 * e], n[3 * e + 1], n[3 * e + 2], g, gx, gy, gz);
  gn[3 * e] = gx;
  gn[3 * e + 1] = gy;
  gn[3 * e + 2] = gz;
}

template <int L>
__global__ __launch_bounds__(256) void sh_jvp_kernel(const float* __restrict__ n, const float* __restrict__ hn,
                                                     int64_t E, float* __restrict__ dY) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float v[Sh<L>::N];
  Sh<L>::jvp(n[3 * e], n[3 * e + 1], n[3 * e + 2], hn[3 * e], hn[3 * e + 1], hn[3 * e + 2], v);
#pragma unroll
  for (int k = 0; k < Sh<L>::N; ++k) dY[e * Sh<L>::N + k] = v[k];
}

template <int L>
__global__ __launch_bounds__(256) void sh_hvp_kernel(const float* __restrict__ n, const float* __restrict__ gY,
                                                     const float* __restrict__ hn, int64_t E, float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float g[Sh<L>::N];
#pragma unroll
  for (int k = 0; k < Sh<L>::N; ++k) g[k] = gY[e * Sh<L>::N + k];
  float ox, oy, oz;
  Sh<L>::hvp(n[3 * e], n[3 * e + 1], n[3 * e + 2], g, hn[3 * e], hn[3 * e + 1], hn[3 * e + 2], ox, oy, oz);
  out[3 * e] = ox;
  out[3 * e + 1] = oy;
  out[3 * e + 2] = oz;
}

}  // namespace ictc
