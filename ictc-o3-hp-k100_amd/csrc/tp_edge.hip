// Per-edge TP forward / first adjoint launchers.
#include "ictc_launch.h"

namespace ictc {

namespace {
struct EdgeFwd {
  const Operands& a;
  float* out;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    hipLaunchKernelGGL((edge_fwd_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock), 0, st, a, out);
    return hipGetLastError();
  }
};
struct EdgeBwd {
  const Operands& a;
  const float* grad;
  float *dx, *dsh, *dg;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    if (G == 1)
      hipLaunchKernelGGL((edge_bwd_kernel<T>), dim3(blocks_for(a.rows)), dim3(kBlock), 0, st, a, grad, dx, dsh, dg,
                         G);
    else
      hipLaunchKernelGGL((edge_bwd_kernel<T>), dim3((unsigned)a.rows), dim3(kWave * G), G * T::NY * sizeof(float),
                         st, a, grad, dx, dsh, dg, G);
    return hipGetLastError();
  }
};
}  // namespace

hipError_t launch_edge_fwd(const TpShape& s, const Operands& a, float* out, hipStream_t st) {
  return dispatch_tp(s, EdgeFwd{a, out, st});
}

hipError_t launch_edge_bwd(const TpShape& s, const Operands& a, const float* grad, float* dx, float* dsh, float* dg,
                           hipStream_t st) {
  return dispatch_tp(s, EdgeBwd{a, grad, dx, dsh, dg, st});
}

}  // namespace ictc
