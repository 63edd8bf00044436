// Mixed second derivatives of the per-edge TP and of the CSR graph message,
// fused (gfx950).
//
// The first adjoint (x, y, g; go) -> (dx, dy, dg) is multilinear, so its
// derivative along tangents (tx, ty, tg) of its cotangent outputs is a sum of
// first-order maps with one operand replaced by a tangent:
//   dgo = fwd(tx, y, g) + fwd(x, ty, g) + fwd(x, y, tg)
//   dx  = dx(ty, g, go) + dx(y, tg, go)
//   dy  = dy(tx, g, go) + dy(x, tg, go)
//   dg  = dg(tx, y, go) + dg(x, ty, go)
// (the reference's generated_second, backends/k100/generated_message_second.py:78-204,
// and its formula in ops/fused_message.py:677-729).  Each kernel here reads
// every operand and tangent once and writes each output once; absent
// tangents (nullptr) drop their terms through wave-uniform branches.
// Layouts, launch geometry and determinism are those of ictc_kernels.h.
#pragma once
#include "ictc_kernels.h"

namespace ictc {

struct Tangents {
  const float* x;      // tangent of the features (rows like Operands::x) or nullptr
  const float* sh;     // [E, NY] or nullptr
  const float* gates;  // [E, P*C] or nullptr
};

// Gates from an arbitrary [E, P*C] base (operand or tangent), times weight and scale.
template <class T>
__device__ __forceinline__ void load_gates(const float* __restrict__ base, const Operands& a, int64_t e, int c,
                                           float scale, float* gw) {
  load_row<T::P>(base + e * (int64_t)(T::P * a.channels), a.channels, c, gw);
  if (a.weight) {
    float w[T::P];
#pragma unroll
    for (int p = 0; p < T::P; ++p) w[p] = a.weight[p * a.channels + c];
#pragma unroll
    for (int p = 0; p < T::P; ++p) gw[p] *= w[p];
  }
#pragma unroll
  for (int p = 0; p < T::P; ++p) gw[p] *= scale;
}

template <int N>
__device__ __forceinline__ void zero(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = 0.f;
}

// This channel group's sum of a [NY] harmonic gradient into out[e] (group 0:
// the output; group g > 0: its workspace slab, summed by launch_group_sum).
template <class T>
__device__ __forceinline__ void store_dsh(float* __restrict__ out, int64_t e, const float* dyv) {
  const float mine = wave_sums<T::NY>(dyv);
  const int j = wave_sums_slot();
  if (j >= 0 && j < T::NY) out[e * T::NY + j] = mine;
}

// dyv += dy(x, w, go) when want_dy; dacc += dg(x, y, go) when want_dg; one
// pass over the CG entries when both are wanted.
template <class T>
__device__ __forceinline__ void dy_dg_add(bool want_dy, bool want_dg, const float* x, const float* y,
                                          const float* w, const float* go, float* dyv, float* dacc) {
  float d2[T::P];
  if (want_dy && want_dg) T::dydg(x, y, w, go, dyv, d2);
  else if (want_dy) T::dy(x, w, go, dyv);
  else if (want_dg) T::dg(x, y, go, d2);
  if (want_dg) {
#pragma unroll
    for (int p = 0; p < T::P; ++p) dacc[p] += d2[p];
  }
}

// ---------------------------------------------------------------------------
// Per-edge TP: one wave per (edge, channel group); every output optional.
// ---------------------------------------------------------------------------
template <class T>
__global__ __launch_bounds__(kBlock, (Occupancy<kEdgeSecond, T::LI, T::LE, T::LO>::value)) void edge_second_kernel(
    Operands a, Tangents t, const float* __restrict__ grad, float* __restrict__ dgrad, float* __restrict__ dx,
    float* __restrict__ dsh, float* __restrict__ dsh_part, float* __restrict__ dgates) {
  const RowGroup rg = row_group_y();
  const int64_t e = rg.row;
  if (e >= a.rows) return;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  const bool active = c < C;
  float y[T::NY], ty[T::NY], dyv[T::NY];
  load_harmonics<T>(a.sh, e, y);
  if (t.sh) load_harmonics<T>(t.sh, e, ty);
  else zero<T::NY>(ty);
  zero<T::NY>(dyv);
  if (active) {
    const int64_t xo = e * (int64_t)(T::NX * C);
    float xv[T::NX], tx[T::NX], gw[T::P], tg[T::P];
    if (t.sh || t.gates) load_row<T::NX>(a.x + xo, C, c, xv);
    else zero<T::NX>(xv);
    if (t.x) load_row<T::NX>(t.x + xo, C, c, tx);
    else zero<T::NX>(tx);
    load_gates<T>(a.gates, a, e, c, 1.f, gw);
    if (t.gates) load_gates<T>(t.gates, a, e, c, 1.f, tg);
    else zero<T::P>(tg);
    if (dgrad) {
      float o[T::NO];
      zero<T::NO>(o);
      if (t.x) T::fwd(tx, y, gw, o);
      if (t.sh) T::fwd(xv, ty, gw, o);
      if (t.gates) T::fwd(xv, y, tg, o);
      store_row<T::NO>(dgrad + e * (int64_t)(T::NO * C), C, c, o);
    }
    if (dx || dsh || dgates) {
      float go[T::NO];
      load_row<T::NO>(grad + e * (int64_t)(T::NO * C), C, c, go);
      if (dx) {
        float d[T::NX];
        zero<T::NX>(d);
        if (t.sh) T::dx_v(ty, gw, go, d);
        if (t.gates) T::dx_v(y, tg, go, d);
        store_row<T::NX>(dx + xo, C, c, d);
      }
      float d[T::P];
      zero<T::P>(d);
      if (t.x) dy_dg_add<T>(dsh != nullptr, dgates != nullptr, tx, y, gw, go, dyv, d);
      dy_dg_add<T>(dsh && t.gates, dgates && t.sh, xv, ty, tg, go, dyv, d);
      if (dgates) {
        if (a.weight) {
#pragma unroll
          for (int p = 0; p < T::P; ++p) d[p] *= a.weight[p * C + c];
        }
        store_row<T::P>(dgates + e * (int64_t)(T::P * C), C, c, d);
      }
    }
  }
  if (dsh) store_dsh<T>(group_target(dsh, dsh_part, rg.group, a.rows, T::NY), e, dyv);
}

// Tangent harmonics of a staged chunk (lane i holds edge ch.e's row).
template <class T>
__device__ __forceinline__ void stage_tangent(const float* __restrict__ tsh, const Chunk<T>& ch, int count,
                                              float* ty) {
  const bool mine = lane_id() < count && tsh;
#pragma unroll
  for (int j = 0; j < T::NY; ++j) ty[j] = mine ? tsh[(int64_t)ch.e * T::NY + j] : 0.f;
}

// ---------------------------------------------------------------------------
// Graph message, receiver-owned: dgrad[n] = sum over edges into n of the three
// forward terms.
// ---------------------------------------------------------------------------
template <class T>
__global__ __launch_bounds__(kBlock, (Occupancy<kMsgFwd2, T::LI, T::LE, T::LO>::value)) void msg_fwd2_kernel(
    Operands a, Tangents t, const int64_t* __restrict__ src, Csr csr, float* __restrict__ out) {
  const RowGroup rg = row_group_y_xcd();
  if (rg.row >= a.rows) return;
  const int64_t n = visit_row(csr, rg.row, a.rows);
  if (n < 0) return;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  const bool active = c < C;
  float o[T::NO];
  zero<T::NO>(o);
  const int32_t beg = csr.ptr[n], end = csr.ptr[n + 1];
  for (int32_t pos = beg; pos < end; pos += kWave) {
    const int32_t count = min(end - pos, kWave);
    Chunk<T> ch;
    stage_chunk<T>(a, src, csr.order, pos, count, ch);
    float tys[T::NY];
    stage_tangent<T>(t.sh, ch, count, tys);
    for (int i = 0; i < count; ++i) {
      const int64_t e = lane_i(ch.e, i);
      const int64_t s = lane_i(ch.peer, i);
      const float m = lane_f(ch.m, i);
      float y[T::NY], ty[T::NY];
#pragma unroll
      for (int j = 0; j < T::NY; ++j) {
        y[j] = lane_f(ch.y[j], i);
        ty[j] = lane_f(tys[j], i);
      }
      if (active) {
        const int64_t xo = s * (int64_t)(T::NX * C);
        float gw[T::P];
        load_gates<T>(a.gates, a, e, c, m, gw);
        if (t.x) {
          float tx[T::NX];
          load_row<T::NX>(t.x + xo, C, c, tx);
          T::fwd(tx, y, gw, o);
        }
        if (t.sh || t.gates) {
          float xv[T::NX];
          load_row<T::NX>(a.x + xo, C, c, xv);
          if (t.sh) T::fwd(xv, ty, gw, o);
          if (t.gates) {
            float tg[T::P];
            load_gates<T>(t.gates, a, e, c, m, tg);
            T::fwd(xv, y, tg, o);
          }
        }
      }
    }
  }
  if (active) store_row<T::NO>(out + n * (int64_t)(T::NO * C), C, c, o);
}

// Receiver-owned: per-edge harmonic and gate outputs (row `rows` zero-fills the
// out-of-range tail segment).
template <class T>
__global__ __launch_bounds__(kBlock, (Occupancy<kMsgBwdEdge2, T::LI, T::LE, T::LO>::value)) void msg_bwd_edge2_kernel(
    Operands a, Tangents t, const int64_t* __restrict__ src, Csr csr, const float* __restrict__ grad,
    float* __restrict__ dsh, float* __restrict__ dsh_part, float* __restrict__ dgates, int parts) {
  const RowGroup rg = row_group_y_xcd();
  const int64_t slot = rg.row / parts;
  if (slot > a.rows) return;
  const int64_t n = visit_row(csr, slot, a.rows);
  if (n < 0) return;
  int32_t beg, end;
  if (!row_part(csr, n, (int)(rg.row % parts), parts, beg, end)) return;
  const bool tail = n == a.rows;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  const bool active = c < C;
  float* dsh_g = group_target(dsh, dsh_part, rg.group, a.edges, T::NY);
  float go[T::NO];
  if (active && !tail) load_row<T::NO>(grad + n * (int64_t)(T::NO * C), C, c, go);
  else zero<T::NO>(go);
  const bool need_x = (dsh && t.gates) || (dgates && t.sh);
  const bool need_tx = t.x != nullptr;
  for (int32_t pos = beg; pos < end; pos += kWave) {
    const int32_t count = min(end - pos, kWave);
    Chunk<T> ch;
    stage_chunk<T>(a, src, csr.order, pos, count, ch);
    float tys[T::NY];
    stage_tangent<T>(t.sh, ch, count, tys);
    for (int i = 0; i < count; ++i) {
      const int64_t e = lane_i(ch.e, i);
      const int64_t s = lane_i(ch.peer, i);
      const float m = lane_f(ch.m, i);
      float y[T::NY], ty[T::NY], dyv[T::NY];
#pragma unroll
      for (int j = 0; j < T::NY; ++j) {
        y[j] = lane_f(ch.y[j], i);
        ty[j] = lane_f(tys[j], i);
        dyv[j] = 0.f;
      }
      if (active) {
        const int64_t xo = s * (int64_t)(T::NX * C);
        float xv[T::NX], tx[T::NX];
        if (need_x) load_row<T::NX>(a.x + xo, C, c, xv);
        else zero<T::NX>(xv);
        if (need_tx) load_row<T::NX>(t.x + xo, C, c, tx);
        else zero<T::NX>(tx);
        float d[T::P];
        zero<T::P>(d);
        if (t.x) {
          float gw[T::P];
          if (dsh) load_gates<T>(a.gates, a, e, c, m, gw);
          else zero<T::P>(gw);
          dy_dg_add<T>(dsh != nullptr, dgates != nullptr, tx, y, gw, go, dyv, d);
        }
        {
          float tg[T::P];
          if (dsh && t.gates) load_gates<T>(t.gates, a, e, c, m, tg);
          else zero<T::P>(tg);
          dy_dg_add<T>(dsh && t.gates, dgates && t.sh, xv, ty, tg, go, dyv, d);
        }
        if (dgates) {
#pragma unroll
          for (int p = 0; p < T::P; ++p) d[p] *= m;
          if (a.weight) {
#pragma unroll
            for (int p = 0; p < T::P; ++p) d[p] *= a.weight[p * C + c];
          }
          store_row<T::P>(dgates + e * (int64_t)(T::P * C), C, c, d);
        }
      }
      if (dsh) {
        // this group's harmonic gradient of edge e, one component per slot lane
        const float v = wave_sums<T::NY>(dyv);
        const int j = wave_sums_slot();
        if (j >= 0 && j < T::NY) dsh_g[e * T::NY + j] = v;
      }
    }
  }
}

// Source-owned: dx[s] = sum over edges out of s of dx(ty, g, go) + dx(y, tg, go).
template <class T>
__global__ __launch_bounds__(kBlock, (Occupancy<kMsgBwdX2, T::LI, T::LE, T::LO>::value)) void msg_bwd_x2_kernel(
    Operands a, Tangents t, const int64_t* __restrict__ dst, Csr scsr, const float* __restrict__ grad,
    float* __restrict__ dx) {
  const RowGroup rg = row_group_y_xcd();
  if (rg.row >= a.rows) return;
  const int64_t n = visit_row(scsr, rg.row, a.rows);
  if (n < 0) return;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  const bool active = c < C;
  float d[T::NX];
  zero<T::NX>(d);
  const int32_t beg = scsr.ptr[n], end = scsr.ptr[n + 1];
  for (int32_t pos = beg; pos < end; pos += kWave) {
    const int32_t count = min(end - pos, kWave);
    Chunk<T> ch;
    stage_chunk<T>(a, dst, scsr.order, pos, count, ch);
    float tys[T::NY];
    stage_tangent<T>(t.sh, ch, count, tys);
    for (int i = 0; i < count; ++i) {
      const int64_t e = lane_i(ch.e, i);
      const int64_t r = lane_i(ch.peer, i);
      const float m = lane_f(ch.m, i);
      float y[T::NY], ty[T::NY];
#pragma unroll
      for (int j = 0; j < T::NY; ++j) {
        y[j] = lane_f(ch.y[j], i);
        ty[j] = lane_f(tys[j], i);
      }
      if (active) {
        float go[T::NO];
        load_row<T::NO>(grad + r * (int64_t)(T::NO * C), C, c, go);
        if (t.sh) {
          float gw[T::P];
          load_gates<T>(a.gates, a, e, c, m, gw);
          T::dx_v(ty, gw, go, d);
        }
        if (t.gates) {
          float tg[T::P];
          load_gates<T>(t.gates, a, e, c, m, tg);
          T::dx_v(y, tg, go, d);
        }
      }
    }
  }
  if (active) store_row<T::NX>(dx + n * (int64_t)(T::NX * C), C, c, d);
}

}  // namespace ictc
