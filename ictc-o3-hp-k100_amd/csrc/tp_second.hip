// Per-edge TP mixed-second-derivative launcher.
#include "ictc_launch.h"

namespace ictc {

namespace {
struct EdgeSecond {
  const Operands& a;
  const Tangents& t;
  const float* grad;
  float *dgrad, *dx, *dsh, *dg, *ws;
  hipStream_t st;
  template <class T>
  hipError_t run() {
    const int G = channel_groups(a.channels);
    hipLaunchKernelGGL((edge_second_kernel<T>), dim3(blocks_for(a.rows), G), dim3(kBlock), 0, st, a, t, grad, dgrad,
                       dx, dsh, ws, dg);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !dsh) return err;
    return launch_group_sum(dsh, ws, a.rows * T::NY, G - 1, st);
  }
};
}  // namespace

hipError_t launch_edge_second(const TpShape& s, const Operands& a, const Tangents& t, const float* grad, float* dgrad,
                              float* dx, float* dsh, float* dg, float* ws, hipStream_t st) {
  return dispatch_tp(s, EdgeSecond{a, t, grad, dgrad, dx, dsh, dg, ws, st});
}

}  // namespace ictc
