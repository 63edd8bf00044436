// Symmetric-contraction kernels (one wave per node, lane = channel, runtime
// loop over 64-channel tiles).  The polynomial bodies are generated in
// generated/ictc_sc.h.  Layouts (FP32, component-major, channel-minor):
//   x   [N, NX*C]  (ICTC basis, packed by degree)
//   out [N, NO*C]  NO = sum_{L<=LT} (2L+1)
//   W(L, nu) [S, P, C]  per-species weights (reference layout, _mace_symmetric_contraction.py:152-155)
// Weight gradients are reduced over a species-sorted node CSR in chunks of
// kChunk nodes that never straddle a species (chunk table cbeg: species s owns
// chunks cbeg[s] .. cbeg[s+1]); each wave sums one chunk for one channel group
// and one block of kDwBlock weights into partials [chunks, NW, C], which are
// then summed over the species' chunks in order: deterministic, no atomics.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "generated/ictc_sc.h"

namespace ictc {
namespace sc {

constexpr int kWave = 64;
constexpr int kWaves = 4;
constexpr int kChunk = 16;    // nodes per weight-gradient partial
constexpr int kDwBlock = 32;  // weights per weight-gradient wave (DW_BLOCK in gen_sc.py)

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

template <int N>
__device__ __forceinline__ void load(const float* __restrict__ b, int C, int c, float* v) {
  const uint32_t off = sc_lane_offset(c);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = sc_load(b + (int64_t)i * C, off);
}
template <int N>
__device__ __forceinline__ void store(float* __restrict__ b, int C, int c, const float* v) {
  const uint32_t off = sc_lane_offset(c);
#pragma unroll
  for (int i = 0; i < N; ++i) *reinterpret_cast<float*>(reinterpret_cast<char*>(b + (int64_t)i * C) + off) = v[i];
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

// Chunk table of the species-sorted CSR ptr [S+2]: cbeg[s] = first chunk of
// species s, cbeg[S] = number of chunks.  One thread (S is small).  A template
// only so that every translation unit that includes this header may define it.
template <int = 0>
__global__ void chunk_table_kernel(const int32_t* __restrict__ ptr, int S, int32_t* __restrict__ cbeg) {
  if (blockIdx.x != 0 || threadIdx.x != 0) return;
  int32_t k = 0;
  for (int s = 0; s < S; ++s) {
    cbeg[s] = k;
    k += (ptr[s + 1] - ptr[s] + kChunk - 1) / kChunk;
  }
  cbeg[S] = k;
}

template <class T, int MODE, int B>
__device__ __forceinline__ void dw_block(const Args& a, const float* __restrict__ go, const float* __restrict__ h,
                                         const int32_t* __restrict__ order, int32_t beg, int32_t end, int c,
                                         float* __restrict__ prow) {
  constexpr int Q0 = B * kDwBlock;
  constexpr int NQ = T::NW - Q0 < kDwBlock ? T::NW - Q0 : kDwBlock;
  const int C = a.channels;
  float acc[kDwBlock];
#pragma unroll
  for (int q = 0; q < kDwBlock; ++q) acc[q] = 0.f;
  for (int32_t k = beg; k < end; ++k) {
    const int64_t n = order[k];
    float xv[T::NX], gv[T::NO];
    load<T::NX>(a.x + n * (int64_t)(T::NX * C), C, c, xv);
    load<T::NO>(go + n * (int64_t)(T::NO * C), C, c, gv);
    if (MODE == 0) {
      T::template dwb<B>(xv, gv, acc);
    } else {
      float hv[T::NX];
      load<T::NX>(h + n * (int64_t)(T::NX * C), C, c, hv);
      T::template dwjvpb<B>(xv, gv, hv, acc);
    }
  }
  store<NQ>(prow + Q0 * (int64_t)C, C, c, acc);
}

template <class T, int MODE, int B = 0>
__device__ __forceinline__ void dw_blocks(int b, const Args& a, const float* __restrict__ go,
                                          const float* __restrict__ h, const int32_t* __restrict__ order,
                                          int32_t beg, int32_t end, int c, float* __restrict__ prow) {
  if constexpr (B < T::NB) {
    if (b == B) dw_block<T, MODE, B>(a, go, h, order, beg, end, c, prow);
    else dw_blocks<T, MODE, B + 1>(b, a, go, h, order, beg, end, c, prow);
  }
}

// Partial weight gradients: wave (chunk k, channel group blockIdx.y, weight
// block blockIdx.z) sums the nodes order[beg .. end) of chunk k.
// mode 0: dw, mode 1: dwjvp.
template <class T, int MODE>
__global__ __launch_bounds__(256) void dw_partial_kernel(Args a, const float* __restrict__ go,
                                                         const float* __restrict__ h, const int32_t* __restrict__ ptr,
                                                         const int32_t* __restrict__ order,
                                                         const int32_t* __restrict__ cbeg, int64_t max_chunks,
                                                         float* __restrict__ partial) {
  const int64_t k = (int64_t)blockIdx.x * kWaves + wave_id();
  const int S = a.num_species;
  if (k >= max_chunks || k >= cbeg[S]) return;
  int lo = 0, hi = S - 1;  // species s with cbeg[s] <= k < cbeg[s + 1]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cbeg[mid] <= k) lo = mid;
    else hi = mid - 1;
  }
  const int s = lo;
  const int32_t beg = ptr[s] + (int32_t)(k - cbeg[s]) * kChunk;
  const int32_t end = min(ptr[s + 1], beg + kChunk);
  const int c = 64 * (int)blockIdx.y + lane_id();
  if (c >= a.channels) return;
  dw_blocks<T, MODE>((int)blockIdx.z, a, go, h, order, beg, end, c, partial + k * (int64_t)(T::NW * a.channels));
}

struct WeightGrads {
  float* w[4][3];
};

// dW(L, nu)[s, p, c] = sum over the chunks of species s (in order) of partial[chunk, q, c].
template <class T>
__global__ __launch_bounds__(256) void dw_reduce_kernel(const float* __restrict__ partial, int num_species,
                                                        const int32_t* __restrict__ cbeg, int C, WeightGrads g) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)num_species * T::NW * C;
  if (i >= total) return;
  const int c = (int)(i % C);
  const int q = (int)((i / C) % T::NW);
  const int s = (int)(i / ((int64_t)C * T::NW));
  float acc = 0.f;
  for (int32_t k = cbeg[s]; k < cbeg[s + 1]; ++k) acc += partial[((int64_t)k * T::NW + q) * C + c];
  const int L = T::WQ[q][0], nu = T::WQ[q][1], p = T::WQ[q][2];
  float* dst = g.w[L][nu];
  if (dst) dst[((int64_t)s * T::P[L][nu] + p) * C + c] = acc;
}

}  // namespace sc
}  // namespace ictc
