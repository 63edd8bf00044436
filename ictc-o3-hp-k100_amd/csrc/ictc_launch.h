// Internal launch interface between the C ABI (capi.hip) and the kernel
// translation units (tp_edge.hip, msg_fwd.hip, msg_bwd.hip).  Not part of the
// public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ictc_kernels.h"
#include "ictc_second.h"

namespace ictc {

struct TpShape {
  int li, le, lo, channels;
};

// Channel groups of 64 for a channel count (0: unsupported).
inline int channel_groups(int C) { return C < 1 || C > 64 * kMaxGroups ? 0 : (C + 63) / 64; }

hipError_t launch_edge_fwd(const TpShape& s, const Operands& a, float* out, hipStream_t st);
hipError_t launch_edge_bwd(const TpShape& s, const Operands& a, const float* grad, float* dx, float* dsh, float* dg,
                           float* ws, hipStream_t st);
hipError_t launch_msg_fwd(const TpShape& s, const Operands& a, const int64_t* src, Csr dcsr, float* out,
                          hipStream_t st);
// The source-owned feature adjoint gathers a 9 KB receiver cotangent row per
// edge; with more rows in flight than the L2 holds, the re-reads grow faster
// than the latency hiding gains.  Unused dynamic LDS caps the resident blocks
// per CU (160 KB / cap bytes).  Measured on the cfg4 layer-1 shape: 2 blocks
// (8 waves) per CU 4.85 ms and 31.7 GB fetched, 3 blocks 4.94 ms / 36.4 GB,
// uncapped (16 waves) 5.19 ms / 39.5 GB.  The receiver-owned kernels lose
// more latency hiding than they save (msg_fwd 3.50 -> 3.95 ms when capped).
// Small graphs (cfg2's 4,096 rows) fit the L2 and keep every wave.
template <class T>
inline size_t bwd_x_lds_cap(int64_t rows) {
  return (T::LI == 2 && T::LE == 2 && T::LO == 2 && rows >= 65536) ? 72 * 1024 : 0;
}

hipError_t launch_msg_bwd(const TpShape& s, const Operands& a, const int64_t* src, const int64_t* dst, Csr dcsr,
                          Csr scsr, const float* grad, float* dx, float* dsh, float* dg, float* ws, hipStream_t st);

hipError_t launch_msg_bwd_tangent(const TpShape& s, const Operands& a, const int64_t* src, const int64_t* dst,
                                  Csr dcsr, Csr scsr, const float* grad, const float* gdot, float* dx, float* dsh,
                                  float* dr, float* ws, hipStream_t st);

hipError_t launch_edge_second(const TpShape& s, const Operands& a, const Tangents& t, const float* grad, float* dgrad,
                              float* dx, float* dsh, float* dg, float* ws, hipStream_t st);
hipError_t launch_msg_second_rcv(const TpShape& s, const Operands& a, const Tangents& t, const int64_t* src, Csr dcsr,
                                 const float* grad, float* dgrad, float* dsh, float* dg, float* ws, hipStream_t st);
hipError_t launch_msg_second_src(const TpShape& s, const Operands& a, const Tangents& t, const int64_t* dst, Csr scsr,
                                 const float* grad, float* dx, hipStream_t st);

// out[i] += sum_{s < slabs} part[s * n + i], slabs added in order (deterministic
// combination of the channel groups' harmonic gradients).  No-op for slabs == 0.
hipError_t launch_group_sum(float* out, const float* part, int64_t n, int slabs, hipStream_t st);

// Dispatch a runtime (LI, LE, LO) onto a functor templated on Tp<...>.
template <class F>
hipError_t dispatch_tp(const TpShape& s, F&& f) {
#define ICTC_CASE(A, B, C) \
  if (s.li == A && s.le == B && s.lo == C) return f.template run<Tp<A, B, C>>();
  ICTC_FOR_EACH_TP(ICTC_CASE)
#undef ICTC_CASE
  return hipErrorInvalidValue;
}

inline unsigned blocks_for(int64_t waves) { return (unsigned)((waves + kWavesPerBlock - 1) / kWavesPerBlock); }

// Waves per row for the receiver-owned per-edge kernels: enough shares of
// each row's edges to give about 32k waves when the graph has few rows (up to
// 8 per row; 1 for large graphs).
inline int row_parts(int64_t row_slots, int groups) {
  const int64_t waves = row_slots * groups;
  if (waves <= 0) return 1;
  const int64_t p = (32768 + waves - 1) / waves;
  return (int)(p < 1 ? 1 : (p > 8 ? 8 : p));
}

}  // namespace ictc
