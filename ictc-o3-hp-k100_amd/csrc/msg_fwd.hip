// CSR graph message forward launcher.
#include "ictc_launch.h"

namespace ictc {

namespace {
struct MsgFwd {
  const Operands& a;
  const int64_t* src;
  Csr csr;
  float* out;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    hipLaunchKernelGGL((msg_fwd_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock), 0, st, a, src, csr, out);
    return hipGetLastError();
  }
};
}  // namespace

hipError_t launch_msg_fwd(const TpShape& s, const Operands& a, const int64_t* src, Csr dcsr, float* out,
                          hipStream_t st) {
  return dispatch_tp(s, MsgFwd{a, src, dcsr, out, st});
}

}  // namespace ictc
