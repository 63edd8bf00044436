// Per-configuration symmetric-contraction launchers.  Declared here, defined
// (explicitly instantiated) in the sc_part*.hip translation units so the large
// generated polynomial bodies compile in parallel.
#pragma once
#include "sc_kernels.h"

namespace ictc {
namespace sc {

inline int chunks_for(int64_t nodes) { return (int)((nodes + kChunk - 1) / kChunk); }
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
    const int chunks = chunks_for(a.nodes);                                                                          \
    const int64_t waves = (int64_t)a.num_species * chunks;                                                           \
    if (mode == 0)                                                                                                   \
      hipLaunchKernelGGL((dw_partial_kernel<T, 0>), dim3(node_blocks(waves)), dim3(256), 0, st, a, go, h, ptr,       \
                         order, chunks, partial);                                                                    \
    else                                                                                                             \
      hipLaunchKernelGGL((dw_partial_kernel<T, 1>), dim3(node_blocks(waves)), dim3(256), 0, st, a, go, h, ptr,       \
                         order, chunks, partial);                                                                    \
    hipError_t e = hipGetLastError();                                                                                \
    if (e != hipSuccess) return e;                                                                                   \
    WeightGrads g;                                                                                                   \
    for (int L = 0; L < 4; ++L)                                                                                      \
      for (int n = 0; n < 3; ++n) g.w[L][n] = T::P[L][n] > 0 ? dwp[L * 3 + n] : nullptr;                             \
    const int64_t total = (int64_t)a.num_species * T::NW * a.channels;                                               \
    hipLaunchKernelGGL((dw_reduce_kernel<T>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, partial,      \
                       a.num_species, chunks, a.channels, g);                                                        \
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
