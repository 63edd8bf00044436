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
  float *dx, *dsh, *dg, *ws;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    hipLaunchKernelGGL((edge_bwd_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock), 0, st, a, grad, dx, dsh, ws,
                       dg);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !dsh) return err;
    return launch_group_sum(dsh, ws, a.rows * T::NY, G - 1, st);
  }
};
}  // namespace

hipError_t launch_edge_fwd(const TpShape& s, const Operands& a, float* out, hipStream_t st) {
  return dispatch_tp(s, EdgeFwd{a, out, st});
}

hipError_t launch_edge_bwd(const TpShape& s, const Operands& a, const float* grad, float* dx, float* dsh, float* dg,
                           float* ws, hipStream_t st) {
  return dispatch_tp(s, EdgeBwd{a, grad, dx, dsh, dg, ws, st});
}

}  // namespace ictc
