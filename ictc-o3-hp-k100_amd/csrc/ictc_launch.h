// Internal launch interface between the C ABI (capi.hip) and the kernel
// translation units (tp_edge.hip, msg.hip).  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ictc_kernels.h"

namespace ictc {

struct TpShape {
  int li, le, lo, channels;
};

// Channels per lane for a channel count (0: unsupported).
inline int channels_per_lane(int C) { return C <= 64 ? 1 : C <= 128 ? 2 : C <= 256 ? 4 : 0; }

// Per-CPL launchers (defined in tp_edge_c{1,2,4}.hip and msg_c{1,2,4}.hip).
#define ICTC_DECLARE_LAUNCHERS(CPL)                                                                            \
  hipError_t launch_edge_fwd_c##CPL(const TpShape& s, const Operands& a, float* out, hipStream_t st);          \
  hipError_t launch_edge_bwd_c##CPL(const TpShape& s, const Operands& a, const float* grad, float* dx,         \
                                    float* dsh, float* dg, hipStream_t st);                                  \
  hipError_t launch_msg_fwd_c##CPL(const TpShape& s, const Operands& a, const int64_t* src, Csr dcsr,          \
                                   float* out, hipStream_t st);                                              \
  hipError_t launch_msg_bwd_c##CPL(const TpShape& s, const Operands& a, const int64_t* src, const int64_t* dst, \
                                   Csr dcsr, Csr scsr, const float* grad, float* dx, float* dsh, float* dg,  \
                                   hipStream_t st);
ICTC_DECLARE_LAUNCHERS(1)
ICTC_DECLARE_LAUNCHERS(2)
ICTC_DECLARE_LAUNCHERS(4)

// Dispatch a runtime (LI, LE, LO) onto a functor templated on Tp<...> for a fixed CPL.
template <int CPL, class F>
hipError_t dispatch_cpl(const TpShape& s, F&& f) {
#define ICTC_CASE(A, B, C) \
  if (s.li == A && s.le == B && s.lo == C) return f.template run<Tp<A, B, C>, CPL>();
  ICTC_FOR_EACH_TP(ICTC_CASE)
#undef ICTC_CASE
  return hipErrorInvalidValue;
}

inline unsigned blocks_for(int64_t waves) { return (unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock); }

}  // namespace ictc
