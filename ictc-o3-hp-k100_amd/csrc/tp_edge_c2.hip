// Per-edge TP forward / first adjoint launchers, CPL = 2 channels per lane.
#include "ictc_launch.h"

namespace ictc {

namespace {
struct EdgeFwd {
  const Operands& a;
  float* out;
  hipStream_t st;
  template <class T, int CPL>
  hipError_t run() {
    hipLaunchKernelGGL((edge_fwd_kernel<T, CPL>), dim3(blocks_for(a.rows)), dim3(kBlock), 0, st, a, out);
    return hipGetLastError();
  }
};
struct EdgeBwd {
  const Operands& a;
  const float* grad;
  float *dx, *dsh, *dg;
  hipStream_t st;
  template <class T, int CPL>
  hipError_t run() {
    hipLaunchKernelGGL((edge_bwd_kernel<T, CPL>), dim3(blocks_for(a.rows)), dim3(kBlock), 0, st, a, grad, dx, dsh,
                       dg);
    return hipGetLastError();
  }
};
}  // namespace

hipError_t launch_edge_fwd_c2(const TpShape& s, const Operands& a, float* out, hipStream_t st) {
  return dispatch_cpl<2>(s, EdgeFwd{a, out, st});
}

hipError_t launch_edge_bwd_c2(const TpShape& s, const Operands& a, const float* grad, float* dx, float* dsh,
                               float* dg, hipStream_t st) {
  return dispatch_cpl<2>(s, EdgeBwd{a, grad, dx, dsh, dg, st});
}

}  // namespace ictc
