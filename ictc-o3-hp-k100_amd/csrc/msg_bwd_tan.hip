// CSR graph message first adjoint in gate-tangent mode: the edge-length
// gradient sum(dgates * d gates / dr) in place of the gate gradient.
#include "ictc_launch.h"

namespace ictc {

namespace {
// Gate-tangent adjoint: dx, dsh as MsgBwd, and dr[e] = sum dgates * gdot in place of dgates.
// Workspace: [G-1][E][NY] harmonic partials, then [G-1][E] dr partials.
struct MsgBwdTan {
  const Operands& a;
  const int64_t *src, *dst;
  Csr dcsr, scsr;
  const float *grad, *gdot;
  float *dx, *dsh, *dr, *ws;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    float* ws_dr = ws ? ws + (int64_t)(G - 1) * a.edges * T::NY : nullptr;
    hipError_t err;
    if (Occupancy<kMsgBwdSrc, T::LI, T::LE, T::LO>::value >= 2 && dx) {
      if (a.weight)
        hipLaunchKernelGGL((msg_bwd_src_kernel<T, true, true>), dim3(blocks_for(a.rows + 1), G), dim3(kBlock), 0, st,
                           a, dst, scsr, grad, dx, dsh, ws, nullptr, gdot, dr, ws_dr);
      else
        hipLaunchKernelGGL((msg_bwd_src_kernel<T, true, false>), dim3(blocks_for(a.rows + 1), G), dim3(kBlock), 0, st,
                           a, dst, scsr, grad, dx, dsh, ws, nullptr, gdot, dr, ws_dr);
      if ((err = hipGetLastError()) != hipSuccess) return err;
    } else {
      const int parts = row_parts(a.rows + 1, G);
      hipLaunchKernelGGL((msg_bwd_edge_kernel<T, true>), dim3(blocks_for((a.rows + 1) * parts), G), dim3(kBlock), 0,
                         st, a, src, dcsr, grad, dsh, ws, nullptr, parts, gdot, dr, ws_dr);
      if ((err = hipGetLastError()) != hipSuccess) return err;
      if (dx) {
        hipLaunchKernelGGL((msg_bwd_x_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock),
                           bwd_x_lds_cap<T>(a.rows), st, a, dst, scsr, grad, dx);
        if ((err = hipGetLastError()) != hipSuccess) return err;
      }
    }
    if (dsh && (err = launch_group_sum(dsh, ws, a.edges * T::NY, G - 1, st)) != hipSuccess) return err;
    return launch_group_sum(dr, ws_dr, a.edges, G - 1, st);
  }
};
}  // namespace

hipError_t launch_msg_bwd_tangent(const TpShape& s, const Operands& a, const int64_t* src, const int64_t* dst,
                                  Csr dcsr, Csr scsr, const float* grad, const float* gdot, float* dx, float* dsh,
                                  float* dr, float* ws, hipStream_t st) {
  return dispatch_tp(s, MsgBwdTan{a, src, dst, dcsr, scsr, grad, gdot, dx, dsh, dr, ws, st});
}

}  // namespace ictc
