// Symmetric-contraction kernels (one wave per node, lane = channel, runtime
// loop over 64-channel tiles).  The polynomial bodies are generated in
// generated/ictc_sc.h.  Layouts (FP32, component-major, channel-minor):
//   x   [N, NX*C]  (ICTC basis, packed by degree)
//   out [N, NO*C]  NO = sum_{L<=LT} (2L+1)
//   W(L, nu) [S, P, C]  per-species weights (reference layout, _mace_symmetric_contraction.py:152-155)
// Weight gradients are reduced over a species-sorted node CSR in fixed-size
// chunks (partials [S, chunks, NW, C]) and then summed over chunks in order:
// deterministic, no atomics.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "generated/ictc_sc.h"

namespace ictc {
namespace sc {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kChunk = 256;  // nodes per weight-gradient partial

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

template <int N>
__device__ __forceinline__ void load(const float* __restrict__ b, int C, int c, float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = b[i * C + c];
}
template <int N>
__device__ __forceinline__ void store(float* __restrict__ b, int C, int c, const float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) b[i * C + c] = v[i];
}

struct Args {
  const float* x;
  const int64_t* species;
  ScWeights w;
  int64_t nodes;
  int num_species;
  int channels;
};

__device__ __forceinline__ int species_of(const Args& a, int64_t n) {
  const int64_t s = a.species[n];
  return (s >= 0 && s < a.num_species) ? (int)s : -1;
}

// out = SC(x)  (mode 0) or out = J(x) h (mode 1, h given)
template <class T, int MODE>
__global__ __launch_bounds__(256) void fwd_kernel(Args a, const float* __restrict__ h, float* __restrict__ out) {
  const int64_t n = (int64_t)blockIdx.x * kWaves + wave_id();
  if (n >= a.nodes) return;
  const int s = species_of(a, n);
  const int C = a.channels;
  const float* xr = a.x + n * (int64_t)(T::NX * C);
  float* orow = out + n * (int64_t)(T::NO * C);
  for (int c = lane_id(); c < C; c += kWave) {
    float o[T::NO];
    if (s < 0) {
#pragma unroll
      for (int k = 0; k < T::NO; ++k) o[k] = 0.f;
    } else {
      float xv[T::NX];
      load<T::NX>(xr, C, c, xv);
      if (MODE == 0) {
        T::fwd(xv, a.w, s, C, c, o);
      } else {
        float hv[T::NX];
        load<T::NX>(h + n * (int64_t)(T::NX * C), C, c, hv);
        T::jvp(xv, a.w, s, C, c, hv, o);
      }
    }
    store<T::NO>(orow, C, c, o);
  }
}

// dx = grad_x (go . SC(x))  (mode 0)  or  dx = Hess (go . SC) h  (mode 1)
template <class T, int MODE>
__global__ __launch_bounds__(256) void dx_kernel(Args a, const float* __restrict__ go, const float* __restrict__ h,
                                                 float* __restrict__ dx) {
  const int64_t n = (int64_t)blockIdx.x * kWaves + wave_id();
  if (n >= a.nodes) return;
  const int s = species_of(a, n);
  const int C = a.channels;
  const float* xr = a.x + n * (int64_t)(T::NX * C);
  float* drow = dx + n * (int64_t)(T::NX * C);
  for (int c = lane_id(); c < C; c += kWave) {
    float d[T::NX];
    if (s < 0) {
#pragma unroll
      for (int i = 0; i < T::NX; ++i) d[i] = 0.f;
    } else {
      float xv[T::NX], gv[T::NO];
      load<T::NX>(xr, C, c, xv);
      load<T::NO>(go + n * (int64_t)(T::NO * C), C, c, gv);
      if (MODE == 0) {
        T::dx(xv, a.w, s, C, c, gv, d);
      } else {
        float hv[T::NX];
        load<T::NX>(h + n * (int64_t)(T::NX * C), C, c, hv);
        T::hvp(xv, a.w, s, C, c, gv, hv, d);
      }
    }
    store<T::NX>(drow, C, c, d);
  }
}

// Partial weight gradients: wave (s, chunk) sums the nodes
// order[ptr[s] + chunk*kChunk ...] of species s.  mode 0: dw, mode 1: dwjvp.
template <class T, int MODE>
__global__ __launch_bounds__(256) void dw_partial_kernel(Args a, const float* __restrict__ go,
                                                         const float* __restrict__ h, const int32_t* __restrict__ ptr,
                                                         const int32_t* __restrict__ order, int chunks,
                                                         float* __restrict__ partial) {
  const int64_t w = (int64_t)blockIdx.x * kWaves + wave_id();
  if (w >= (int64_t)a.num_species * chunks) return;
  const int s = (int)(w / chunks), chunk = (int)(w % chunks);
  const int C = a.channels;
  const int32_t beg = ptr[s] + chunk * kChunk;
  const int32_t end = min(ptr[s + 1], beg + kChunk);
  float* prow = partial + w * (int64_t)(T::NW * C);
  for (int c = lane_id(); c < C; c += kWave) {
    float acc[T::NW];
#pragma unroll
    for (int q = 0; q < T::NW; ++q) acc[q] = 0.f;
    for (int32_t k = beg; k < end; ++k) {
      const int64_t n = order[k];
      float xv[T::NX], gv[T::NO], v[T::NW];
      load<T::NX>(a.x + n * (int64_t)(T::NX * C), C, c, xv);
      load<T::NO>(go + n * (int64_t)(T::NO * C), C, c, gv);
      if (MODE == 0) {
        T::dw(xv, gv, v);
      } else {
        float hv[T::NX];
        load<T::NX>(h + n * (int64_t)(T::NX * C), C, c, hv);
        T::dwjvp(xv, gv, hv, v);
      }
#pragma unroll
      for (int q = 0; q < T::NW; ++q) acc[q] += v[q];
    }
    store<T::NW>(prow, C, c, acc);
  }
}

struct WeightGrads {
  float* w[4][3];
};

// dW(L, nu)[s, p, c] = sum over chunks (in order) of partial[s, chunk, q, c].
template <class T>
__global__ __launch_bounds__(256) void dw_reduce_kernel(const float* __restrict__ partial, int num_species,
                                                        int chunks, int C, WeightGrads g) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)num_species * T::NW * C;
  if (i >= total) return;
  const int c = (int)(i % C);
  const int q = (int)((i / C) % T::NW);
  const int s = (int)(i / ((int64_t)C * T::NW));
  float acc = 0.f;
  for (int k = 0; k < chunks; ++k) acc += partial[(((int64_t)s * chunks + k) * T::NW + q) * C + c];
  const int L = T::WQ[q][0], nu = T::WQ[q][1], p = T::WQ[q][2];
  float* dst = g.w[L][nu];
  if (dst) dst[((int64_t)s * T::P[L][nu] + p) * C + c] = acc;
}

}  // namespace sc
}  // namespace ictc
