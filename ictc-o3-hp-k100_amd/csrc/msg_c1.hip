// CSR graph message forward / first adjoint launchers, CPL = 1 channels per lane.
#include "ictc_launch.h"

namespace ictc {

namespace {
struct MsgFwd {
  const Operands& a;
  const int64_t* src;
  Csr csr;
  float* out;
  hipStream_t st;
  template <class T, int CPL>
  hipError_t run() {
    hipLaunchKernelGGL((msg_fwd_kernel<T, CPL>), dim3(blocks_for(a.rows)), dim3(kBlock), 0, st, a, src, csr, out);
    return hipGetLastError();
  }
};
struct MsgBwd {
  const Operands& a;
  const int64_t *src, *dst;
  Csr dcsr, scsr;
  const float* grad;
  float *dx, *dsh, *dg;
  hipStream_t st;
  template <class T, int CPL>
  hipError_t run() {
    if (dsh || dg) {
      // rows + 1 waves: the last one zero-fills the out-of-range tail segment.
      hipLaunchKernelGGL((msg_bwd_edge_kernel<T, CPL>), dim3(blocks_for(a.rows + 1)), dim3(kBlock), 0, st, a, src,
                         dcsr, grad, dsh, dg);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    if (dx) {
      hipLaunchKernelGGL((msg_bwd_x_kernel<T, CPL>), dim3(blocks_for(a.rows)), dim3(kBlock), 0, st, a, dst, scsr,
                         grad, dx);
      return hipGetLastError();
    }
    return hipSuccess;
  }
};
}  // namespace

hipError_t launch_msg_fwd_c1(const TpShape& s, const Operands& a, const int64_t* src, Csr dcsr, float* out,
                              hipStream_t st) {
  return dispatch_cpl<1>(s, MsgFwd{a, src, dcsr, out, st});
}

hipError_t launch_msg_bwd_c1(const TpShape& s, const Operands& a, const int64_t* src, const int64_t* dst,
                              Csr dcsr, Csr scsr, const float* grad, float* dx, float* dsh, float* dg,
                              hipStream_t st) {
  return dispatch_cpl<1>(s, MsgBwd{a, src, dst, dcsr, scsr, grad, dx, dsh, dg, st});
}

}  // namespace ictc
