// CSR graph message mixed-second-derivative launchers, receiver-owned passes:
// the cotangent tangent (sum into receivers) and the per-edge harmonic / gate outputs.
#include "ictc_launch.h"

namespace ictc {

namespace {
struct MsgSecondRcv {
  const Operands& a;
  const Tangents& t;
  const int64_t* src;
  Csr csr;
  const float* grad;
  float *dgrad, *dsh, *dg, *ws;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    if (dgrad) {
      hipLaunchKernelGGL((msg_fwd2_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock), 0, st, a, t, src, csr,
                         dgrad);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    if (dsh || dg) {
      const int parts = row_parts(a.rows + 1, G);
      hipLaunchKernelGGL((msg_bwd_edge2_kernel<T>), dim3(blocks_for((a.rows + 1) * parts), G), dim3(kBlock), 0, st,
                         a, t, src, csr, grad, dsh, ws, dg, parts);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess || !dsh) return err;
      return launch_group_sum(dsh, ws, a.edges * T::NY, G - 1, st);
    }
    return hipSuccess;
  }
};
}  // namespace

hipError_t launch_msg_second_rcv(const TpShape& s, const Operands& a, const Tangents& t, const int64_t* src, Csr dcsr,
                                 const float* grad, float* dgrad, float* dsh, float* dg, float* ws, hipStream_t st) {
  return dispatch_tp(s, MsgSecondRcv{a, t, src, dcsr, grad, dgrad, dsh, dg, ws, st});
}

}  // namespace ictc
