// Per-configuration symmetric-contraction launchers.  Declared here, defined
// (explicitly instantiated) in the sc_part*.hip translation units so the large
// generated polynomial bodies compile in parallel.
#pragma once
#include "sc_kernels.h"

namespace ictc {
namespace sc {

// Upper bound on the weight-gradient chunks of N nodes over S species.
inline int64_t max_chunks(int64_t nodes, int species) { return (nodes + kChunk - 1) / kChunk + species; }
// Partial buffer bytes (256-aligned); the chunk table [S+1] int32 follows it.
inline int64_t partial_bytes(int64_t nodes, int species, int nw, int channels) {
  return (max_chunks(nodes, species) * nw * channels * (int64_t)sizeof(float) + 255) / 256 * 256;
}
inline unsigned node_blocks(int64_t n) { return (unsigned)((n + kWaves - 1) / kWaves); }

template <class T>
struct Launch {
  static hipError_t fwd(const Args& a, const float* h, float* out, int mode, hipStream_t st);
  static hipError_t dx(const Args& a, const float* go, const float* h, float* dx, int mode, hipStream_t st);
  static hipError_t dw(const Args& a, const float* go, const float* h, const int32_t* ptr, const int32_t* order,
                       float* const* dw, float* partial, int mode, hipStream_t st);
};

#define ICTC_SC_DEFINE(A, B, C)                                                                                      \
  template <>                                                                                                        \
  hipError_t Launch<Sc<A, B, C>>::fwd(const Args& a, const float* h, float* out, int mode, hipStream_t st) {        \
    using T = Sc<A, B, C>;                                                                                           \
    if (mode == 0)                                                                                                   \
      hipLaunchKernelGGL((fwd_kernel<T, 0>), dim3(node_blocks(a.nodes)), dim3(256), 0, st, a, h, out);               \
    else                                                                                                             \
      hipLaunchKernelGGL((fwd_kernel<T, 1>), dim3(node_blocks(a.nodes)), dim3(256), 0, st, a, h, out);               \
    return hipGetLastError();                                                                                        \
  }                                                                                                                  \
  template <>                                                                                                        \
  hipError_t Launch<Sc<A, B, C>>::dx(const Args& a, const float* go, const float* h, float* d, int mode,            \
                                     hipStream_t st) {                                                               \
    using T = Sc<A, B, C>;                                                                                           \
    if (mode == 0)                                                                                                   \
      hipLaunchKernelGGL((dx_kernel<T, 0>), dim3(node_blocks(a.nodes)), dim3(256), 0, st, a, go, h, d);              \
    else                                                                                                             \
      hipLaunchKernelGGL((dx_kernel<T, 1>), dim3(node_blocks(a.nodes)), dim3(256), 0, st, a, go, h, d);              \
    return hipGetLastError();                                                                                        \
  }                                                                                                                  \
  template <>                                                                                                        \
  hipError_t Launch<Sc<A, B, C>>::dw(const Args& a, const float* go, const float* h, const int32_t* ptr,            \
                                     const int32_t* order, float* const* dwp, float* partial, int mode,              \
                                     hipStream_t st) {                                                               \
    using T = Sc<A, B, C>;                                                                                           \
    const int64_t chunks = max_chunks(a.nodes, a.num_species);                                                       \
    int32_t* cbeg = (int32_t*)((char*)partial + partial_bytes(a.nodes, a.num_species, T::NW, a.channels));           \
    hipLaunchKernelGGL(chunk_table_kernel<0>, dim3(1), dim3(64), 0, st, ptr, a.num_species, cbeg);                      \
    const dim3 grid(node_blocks(chunks), (a.channels + 63) / 64, T::NB);                                             \
    if (mode == 0)                                                                                                   \
      hipLaunchKernelGGL((dw_partial_kernel<T, 0>), grid, dim3(256), 0, st, a, go, h, ptr, order, cbeg, chunks,      \
                         partial);                                                                                   \
    else                                                                                                             \
      hipLaunchKernelGGL((dw_partial_kernel<T, 1>), grid, dim3(256), 0, st, a, go, h, ptr, order, cbeg, chunks,      \
                         partial);                                                                                   \
    hipError_t e = hipGetLastError();                                                                                \
    if (e != hipSuccess) return e;                                                                                   \
    WeightGrads g;                                                                                                   \
    for (int L = 0; L < 4; ++L)                                                                                      \
      for (int n = 0; n < 3; ++n) g.w[L][n] = T::P[L][n] > 0 ? dwp[L * 3 + n] : nullptr;                             \
    const int64_t total = (int64_t)a.num_species * T::NW * a.channels;                                               \
    hipLaunchKernelGGL((dw_reduce_kernel<T>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, partial,      \
                       a.num_species, cbeg, a.channels, g);                                                          \
    return hipGetLastError();                                                                                        \
  }

// Explicit specialisations live in exactly one sc_part*.hip each.
#define ICTC_SC_DECLARE(A, B, C)                                                                                     \
  template <>                                                                                                        \
  hipError_t Launch<Sc<A, B, C>>::fwd(const Args&, const float*, float*, int, hipStream_t);                          \
  template <>                                                                                                        \
  hipError_t Launch<Sc<A, B, C>>::dx(const Args&, const float*, const float*, float*, int, hipStream_t);             \
  template <>                                                                                                        \
  hipError_t Launch<Sc<A, B, C>>::dw(const Args&, const float*, const float*, const int32_t*, const int32_t*,        \
                                     float* const*, float*, int, hipStream_t);
ICTC_FOR_EACH_SC(ICTC_SC_DECLARE)

}  // namespace sc
}  // namespace ictc
