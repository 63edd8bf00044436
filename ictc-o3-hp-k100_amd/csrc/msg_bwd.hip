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
  float *dx, *dsh, *dg, *ws;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    // One source-owned pass for all three (rows + 1 slots: the last covers the out-of-range tail) where it
    // keeps 2 waves per SIMD; the P17 shapes need the register room of two separate passes.
    if (Occupancy<kMsgBwdSrc, T::LI, T::LE, T::LO>::value >= 2 && dx && (dsh || dg)) {
      hipLaunchKernelGGL((msg_bwd_src_kernel<T, false>), dim3(blocks_for(a.rows + 1), G), dim3(kBlock),
                         0, st, a, dst, scsr, grad, dx, dsh, ws, dg, nullptr, nullptr, nullptr);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
      if (dsh) return launch_group_sum(dsh, ws, a.edges * T::NY, G - 1, st);
      return hipSuccess;
    }
    if (dsh || dg) {
      // rows + 1 row slots: the last one zero-fills the out-of-range tail segment.
      const int parts = row_parts(a.rows + 1, G);
      hipLaunchKernelGGL((msg_bwd_edge_kernel<T, false>), dim3(blocks_for((a.rows + 1) * parts), G), dim3(kBlock),
                         0, st, a, src, dcsr, grad, dsh, ws, dg, parts, nullptr, nullptr, nullptr);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
      if (dsh && (err = launch_group_sum(dsh, ws, a.edges * T::NY, G - 1, st)) != hipSuccess) return err;
    }
    if (dx) {
      hipLaunchKernelGGL((msg_bwd_x_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock), bwd_x_lds_cap<T>(a.rows),
                         st, a, dst, scsr, grad, dx);
      return hipGetLastError();
    }
    return hipSuccess;
  }
};
}  // namespace

hipError_t launch_msg_bwd(const TpShape& s, const Operands& a, const int64_t* src, const int64_t* dst, Csr dcsr,
                          Csr scsr, const float* grad, float* dx, float* dsh, float* dg, float* ws, hipStream_t st) {
  return dispatch_tp(s, MsgBwd{a, src, dst, dcsr, scsr, grad, dx, dsh, dg, ws, st});
}

}  // namespace ictc
