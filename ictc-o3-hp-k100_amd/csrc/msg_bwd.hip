// CSR graph message first-adjoint launchers: receiver-owned gate / harmonic
// gradients, then the source-owned feature gradient.
#include "ictc_launch.h"

namespace ictc {

namespace {
struct MsgBwd {
  const Operands& a;
  const int64_t *src, *dst;
  Csr dcsr, scsr;
  const float* grad;
  float *dx, *dsh, *dg;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    if (dsh || dg) {
      // rows + 1 row slots: the last one zero-fills the out-of-range tail segment.
      if (G == 1)
        hipLaunchKernelGGL((msg_bwd_edge_kernel<T>), dim3(blocks_for(a.rows + 1)), dim3(kBlock), 0, st, a, src,
                           dcsr, grad, dsh, dg, G);
      else
        hipLaunchKernelGGL((msg_bwd_edge_kernel<T>), dim3((unsigned)(a.rows + 1)), dim3(kWave * G),
                           dsh ? G * kWave * T::NY * sizeof(float) : 0, st, a, src, dcsr, grad, dsh, dg, G);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    if (dx) {
      hipLaunchKernelGGL((msg_bwd_x_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock), 0, st, a, dst, scsr, grad,
                         dx);
      return hipGetLastError();
    }
    return hipSuccess;
  }
};
}  // namespace

hipError_t launch_msg_bwd(const TpShape& s, const Operands& a, const int64_t* src, const int64_t* dst, Csr dcsr,
                          Csr scsr, const float* grad, float* dx, float* dsh, float* dg, hipStream_t st) {
  return dispatch_tp(s, MsgBwd{a, src, dst, dcsr, scsr, grad, dx, dsh, dg, st});
}

}  // namespace ictc
