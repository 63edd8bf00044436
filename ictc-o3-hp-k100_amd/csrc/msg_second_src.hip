// CSR graph message mixed-second-derivative launcher, source-owned pass: the feature output.
#include "ictc_launch.h"

namespace ictc {

namespace {
struct MsgSecondSrc {
  const Operands& a;
  const Tangents& t;
  const int64_t* dst;
  Csr csr;
  const float* grad;
  float* dx;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    hipLaunchKernelGGL((msg_bwd_x2_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock), 0, st, a, t, dst, csr, grad,
                       dx);
    return hipGetLastError();
  }
};
}  // namespace

hipError_t launch_msg_second_src(const TpShape& s, const Operands& a, const Tangents& t, const int64_t* dst, Csr scsr,
                                 const float* grad, float* dx, hipStream_t st) {
  return dispatch_tp(s, MsgSecondSrc{a, t, dst, scsr, grad, dx, st});
}

}  // namespace ictc
