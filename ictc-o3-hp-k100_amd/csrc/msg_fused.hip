// Fused radial-gate graph message for energy + forces: the gates
// g[e, p, c] = sum_k h3[e, k] W4[p C + c, k] (the last Linear of the radial MLP
// `fc`, layers.py:826-835) are formed tile by tile inside the message kernels
// from the MLP's last hidden activation h3 [E, 64] and never written to HBM
// (the reference's streamed gate message, ictc_o3/ops/streamed_gate_message.py:
// 51-57 and _StreamedGate :87-223, which tiles the projection with the TP the
// same way for frozen-weight force inference).  The adjoint rebuilds the
// gates and their r tangents gdot = sum_k t3[e, k] W4[p C + c, k] (t3 =
// d h3 / dr) per tile and forms dE/dr = sum dgates * gdot in registers.
//
// Path groups.  The projection matrix of 11 paths x 64 channels (64 x 704,
// 270 KB as the three bf16 parts below) does not fit the 160 KB LDS, so a
// launch covers the paths of one input degree l1 (a contiguous range of path
// indices: paths are enumerated l1 outer), whose W4 rows (PG x 64 x 64, split:
// PG x 24 KB) stay in LDS for a persistent block.  Such a group reads only
// the degree-l1 block of the gathered features and writes only its own
// output slots, so the groups' launches together gather each feature row
// once; the per-edge harmonic gradient and dr are sums over all paths and
// accumulate over the group launches in launch order (deterministic, no
// atomics).  Each launch also covers one channel group of 64.
//
// Projection on bf16 MFMA with the three-way operand split (split_bf16.h):
// A = h3 rows of a 16-edge tile (edge = MFMA row), B = W4^T columns of 16
// channels, v_mfma_f32_16x16x32_bf16, six products per 16x16x32 block,
// FP32-level accuracy.  The result D[edge][channel] (lane (q, j) holds edges
// 4q .. 4q+3 of channel 16 cb + j) is transposed to one channel per lane
// (lane 16 b + j holds edges 0 .. 15 of channel 16 b + j) by a 4 x 4 block
// transpose across the lane rows: one v_permlane32_swap and one
// v_permlane16_swap stage.  The edge loop then runs the generated group
// contraction TpG on wave-uniform harmonics exactly like the materialised-gate
// kernels.  The adjoint's tiles are 8 edges: rows 0..7 carry h3 and rows
// 8..15 t3 of the same edges, so one MFMA pass yields gates and tangents.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ictc_mi355x.h"
#include "ictc_launch.h"
#include "split_bf16.h"

namespace ictc {
int set_error(int code, const char* msg);
int gemm_nt_grouped(const float* a, int64_t m, int64_t k, int64_t lda, int64_t a_group, int64_t a_gstride,
                    const float* b, int64_t n, int64_t ldb, float* c, int64_t ldc, int64_t c_group,
                    int64_t c_gstride, int accumulate, void* stream, int split);
}

namespace ictc {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

// Waves per block (one block per CU: the W4 slice fills the LDS): 16 where the
// kernel fits 128 VGPRs (input degree 0 groups), else 8.
template <class TG>
constexpr int fused_waves() { return TG::L1 == 0 ? 16 : 8; }
constexpr int kSlice = 4 * 2 * 3 * 64;       // bf16x8 words of one path's split W4 for one channel group (24 KB)

__device__ __forceinline__ v4f mfma_bf16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Split projection: ws[((p G + cg) 4 + cb) 2 + ks][part][lane] = part of
// W4[p C + 64 cg + 16 cb + l%16][32 ks + 8 (l/16) + e] * w[p, 64 cg + 16 cb + l%16]
// (e = 0..7; w the TP path weight, nullptr = 1): the B operand of the 16x16x32 MFMA.
__global__ void fused_split_kernel(const float* __restrict__ W4, const float* __restrict__ tpw, int P, int C,
                                   bf16x8* __restrict__ ws) {
  const int G = C / 64;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)P * G * 4 * 2 * 64) return;
  const int l = (int)(t & 63), ks = (int)((t >> 6) & 1), cb = (int)((t >> 7) & 3);
  const int64_t pg = t >> 9;
  const int p = (int)(pg / G), cg = (int)(pg % G);
  const int c = 64 * cg + 16 * cb + (l & 15);
  const float scale = tpw ? tpw[(int64_t)p * C + c] : 1.f;
  float v[8];
  const float* row = W4 + ((int64_t)p * C + c) * 64 + 32 * ks + 8 * (l >> 4);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = row[e] * scale;
  const Split s = split8(v);
  bf16x8* o = ws + (t >> 6) * 3 * 64 + l;
  o[0] = s.hi;
  o[64] = s.mid;
  o[128] = s.lo;
}

__global__ void fused_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// Block-wide copy of the group's W4 slices (paths P0 .. P0+PG-1, channel group cg) into LDS.
template <int PG, int P0>
__device__ __forceinline__ void stage_slice(const bf16x8* __restrict__ ws, int G, int cg, bf16x8* lds) {
  for (int t = threadIdx.x; t < PG * kSlice; t += blockDim.x) {
    const int p = t / kSlice, rest = t - p * kSlice;
    lds[t] = ws[((int64_t)(P0 + p) * G + cg) * kSlice + rest];
  }
}

// 4 x 4 block transpose across the lane rows (16 lanes each) of four 4-vectors:
// lane (q, j) register [b][r]  ->  lane (b, j) register [q][r].
__device__ __forceinline__ void transpose_rows(v4f* D) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(D[b][r]), __float_as_uint(D[b + 2][r]), false,
                                                      false);
      D[b][r] = __uint_as_float(s[0]);
      D[b + 2][r] = __uint_as_float(s[1]);
    }
#pragma unroll
    for (int b = 0; b < 4; b += 2) {
      const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(D[b][r]), __float_as_uint(D[b + 1][r]), false,
                                                      false);
      D[b][r] = __uint_as_float(s[0]);
      D[b + 1][r] = __uint_as_float(s[1]);
    }
  }
}

// Gates of one 16-row tile for every path of the group: A[ks] is the split
// row block (row l%16, k = 32 ks + 8 (l/16) + e); on return Gt[p][i] holds row
// i's gate of path p for this lane's channel.
template <int PG>
__device__ __forceinline__ void project_tile(const bf16x8* __restrict__ w4l, const Split* A, float (*Gt)[16]) {
  const int l = lane_id();
#pragma unroll
  for (int p = 0; p < PG; ++p) {
    v4f D[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const bf16x8* b = w4l + (p * 4 + cb) * 2 * 3 * 64 + l;
      const bf16x8 b0h = b[0], b0m = b[64], b0l = b[128], b1h = b[192], b1m = b[256], b1l = b[320];
      v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
      // the six products of each k-step, smallest first: lo*hi, hi*lo, mid*mid, mid*hi, hi*mid, hi*hi
      acc = mfma_bf16(A[0].lo, b0h, acc);
      acc = mfma_bf16(A[0].hi, b0l, acc);
      acc = mfma_bf16(A[0].mid, b0m, acc);
      acc = mfma_bf16(A[1].lo, b1h, acc);
      acc = mfma_bf16(A[1].hi, b1l, acc);
      acc = mfma_bf16(A[1].mid, b1m, acc);
      acc = mfma_bf16(A[0].mid, b0h, acc);
      acc = mfma_bf16(A[0].hi, b0m, acc);
      acc = mfma_bf16(A[1].mid, b1h, acc);
      acc = mfma_bf16(A[1].hi, b1m, acc);
      acc = mfma_bf16(A[0].hi, b0h, acc);
      acc = mfma_bf16(A[1].hi, b1h, acc);
      D[cb] = acc;
    }
    transpose_rows(D);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) Gt[p][4 * q + r] = D[q][r];
  }
}

// Split A operand of one row: 16 floats of row `row` (k = 32 ks + 8 (l/16) .. +7), zero when !ok.
__device__ __forceinline__ void load_a(const float* __restrict__ h, int64_t row, bool ok, Split* A) {
  const int g = lane_id() >> 4;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    float v[8];
    if (ok) {
      const v4f* p = reinterpret_cast<const v4f*>(h + row * 64 + 32 * ks + 8 * g);
      const v4f a = p[0], b = p[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = b[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
    A[ks] = split8(v);
  }
}

// Edge metadata of up to 64 consecutive CSR positions, one edge per lane.
template <int NY>
struct FChunk {
  int32_t e, peer;
  float m;
  float y[NY];
};

template <int NY>
__device__ __forceinline__ void stage(const float* __restrict__ sh, const float* __restrict__ mask,
                                      const int64_t* __restrict__ peer_ids, const int32_t* __restrict__ order,
                                      int64_t rows, int32_t pos, int32_t count, FChunk<NY>& ch) {
  const int l = lane_id();
  ch.e = 0;
  ch.peer = 0;
  ch.m = 0.f;
#pragma unroll
  for (int j = 0; j < NY; ++j) ch.y[j] = 0.f;
  if (l < count) {
    const int32_t e = order ? order[pos + l] : pos + l;
    const int64_t p = peer_ids[e];
    const bool ok = p >= 0 && p < rows;
    ch.e = e;
    ch.peer = ok ? (int32_t)p : 0;
    ch.m = ok ? (mask ? mask[e] : 1.f) : 0.f;
#pragma unroll
    for (int j = 0; j < NY; ++j) ch.y[j] = sh[(int64_t)e * NY + j];
  }
}

// Rows of a persistent block.  Block b runs on XCD b % 8; XCD x owns a
// contiguous share of the row slots, and its blocks stride through that share
// together (block i of the XCD, wave w: slots begin + i W + w, then + nbx W),
// so at any time the XCD's waves work on one window of nbx * W consecutive
// rows and the neighbour rows they gather stay in that XCD's L2.
struct RowRange {
  int64_t first, end, stride;
};
template <int W>
__device__ __forceinline__ RowRange block_rows(int64_t slots) {
  const int64_t nb = gridDim.x, x = blockIdx.x % kXcds, i = blockIdx.x / kXcds;
  const int64_t q = nb / kXcds, rem = nb % kXcds;
  const int64_t nbx = q + (x < rem ? 1 : 0);                  // blocks on this XCD
  const int64_t before = x * q + (x < rem ? x : rem);         // blocks on lower XCDs
  const int64_t b0 = slots * before / nb, b1 = slots * (before + nbx) / nb;
  return {b0 + i * W + wave_id(), b1, nbx * W};
}

// dsh[e, 0..NY) and dr[e] from this lane's shares (dyv, dgt), reduced over the
// wave's channels; `acc` adds to what the earlier group launches wrote.
template <int NY>
__device__ __forceinline__ void put_dsh_dr(float* __restrict__ dsh, float* __restrict__ dr, int64_t e, const float* dyv,
                                           float dgt, bool acc) {
  const int j = wave_sums_slot();
  if constexpr (NY + 1 <= 16) {
    if (dsh) {
      float v[NY + 1];
#pragma unroll
      for (int k = 0; k < NY; ++k) v[k] = dyv[k];
      v[NY] = dgt;
      const float t = wave_sums<NY + 1>(v);
      if (j >= 0 && j < NY) {
        float* q = dsh + e * NY + j;
        *q = acc ? *q + t : t;
      } else if (j == NY) {
        dr[e] = acc ? dr[e] + t : t;
      }
      return;
    }
  } else {
    if (dsh) {
      const float t = wave_sums<NY>(dyv);
      if (j >= 0 && j < NY) {
        float* q = dsh + e * NY + j;
        *q = acc ? *q + t : t;
      }
    }
  }
  const float t = wave_sums<1>(&dgt);
  if (j == 0) dr[e] = acc ? dr[e] + t : t;
}

struct FusedArgs {
  const float* x;       // node features [N, NX*C]
  const float* sh;      // [E, NY]
  const float* h;       // h3 [E, 64]
  const float* t;       // t3 = d h3 / dr [E, 64] (adjoint only)
  const bf16x8* w4s;    // split projection (fused_split_kernel)
  const float* mask;    // [E] or nullptr
  const int64_t* peer;  // src (receiver-owned kernels) or dst (source-owned)
  int64_t rows, edges;
  int C, cg;            // channels, channel group of this launch
  Csr csr;
  const int32_t* grow;  // row of h / t for each edge ([E], nullptr = the edge itself)
};

__device__ __forceinline__ int64_t hrow(const FusedArgs& a, int32_t e) { return a.grow ? (int64_t)a.grow[e] : e; }

// Forward: out[n, SLOT[k], c] for the group's slots (receiver-owned).
template <class TG>
__global__ __launch_bounds__(fused_waves<TG>() * 64, 1) void msg_fused_fwd_kernel(FusedArgs a, float* __restrict__ out) {
  extern __shared__ bf16x8 w4l[];
  constexpr int NX = (TG::LI + 1) * (TG::LI + 1);
  stage_slice<TG::PG, TG::P0>(a.w4s, a.C / 64, a.cg, w4l);
  __syncthreads();
  const int C = a.C, l = lane_id(), c = 64 * a.cg + l;
  const RowRange rr = block_rows<fused_waves<TG>()>(a.rows);
  for (int64_t slot = rr.first; slot < rr.end; slot += rr.stride) {
    const int64_t n = visit_row(a.csr, slot, a.rows);
    if (n < 0) continue;
    float o[TG::NOG];
#pragma unroll
    for (int k = 0; k < TG::NOG; ++k) o[k] = 0.f;
    const int32_t beg = a.csr.ptr[n], end = a.csr.ptr[n + 1];
    for (int32_t pos = beg; pos < end; pos += 64) {
      const int32_t count = min(end - pos, 64);
      FChunk<TG::NY> ch;
      stage<TG::NY>(a.sh, a.mask, a.peer, a.csr.order, a.rows, pos, count, ch);
      for (int t0 = 0; t0 < count; t0 += 16) {
        const int ci = t0 + (l & 15);
        const int32_t ea = __shfl(ch.e, ci);
        Split A[2];
        load_a(a.h, ci < count ? hrow(a, ea) : 0, ci < count, A);
        float Gt[TG::PG][16];
        project_tile<TG::PG>(w4l, A, Gt);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (t0 + i < count) {
            const int64_t s = lane_i(ch.peer, t0 + i);
            const float m = lane_f(ch.m, t0 + i);
            float y[TG::NY], xv[TG::NXG], gw[TG::PG];
#pragma unroll
            for (int j = 0; j < TG::NY; ++j) y[j] = lane_f(ch.y[j], t0 + i);
            load_row<TG::NXG>(a.x + s * (int64_t)(NX * C) + TG::X0 * C, C, c, xv);
#pragma unroll
            for (int p = 0; p < TG::PG; ++p) gw[p] = Gt[p][i] * m;
            TG::fwd_b(xv, y, gw, o);
          }
        }
      }
    }
    float* row = out + n * (int64_t)(TG::NO * C) + c;
#pragma unroll
    for (int k = 0; k < TG::NOG; ++k) row[(int64_t)TG::SLOT[k] * C] = o[k];
  }
}

// Gate-tangent adjoint, source-owned (sender rows of the source-sorted CSR, the
// tail slot `rows` holding edges whose sender is out of range): dx of the
// group's input block, and the group's shares of dsh and dr per edge.
template <class TG>
__global__ __launch_bounds__(fused_waves<TG>() * 64, 1) void msg_fused_bwd_src_kernel(FusedArgs a,
                                                                                const float* __restrict__ grad,
                                                                                float* __restrict__ dx,
                                                                                float* __restrict__ dsh,
                                                                                float* __restrict__ dr, int acc) {
  extern __shared__ bf16x8 w4l[];
  constexpr int NX = (TG::LI + 1) * (TG::LI + 1);
  stage_slice<TG::PG, TG::P0>(a.w4s, a.C / 64, a.cg, w4l);
  __syncthreads();
  const int C = a.C, l = lane_id(), c = 64 * a.cg + l;
  const RowRange rr = block_rows<fused_waves<TG>()>(a.rows + 1);
  for (int64_t slot = rr.first; slot < rr.end; slot += rr.stride) {
    const int64_t n = visit_row(a.csr, slot, a.rows);
    if (n < 0) continue;
    const bool tail = n == a.rows;
    float xv[TG::NXG], d[TG::NXG];
    if (!tail) load_row<TG::NXG>(a.x + n * (int64_t)(NX * C) + TG::X0 * C, C, c, xv);
    else zero_row<TG::NXG>(xv);
    zero_row<TG::NXG>(d);
    const int32_t beg = a.csr.ptr[n], end = a.csr.ptr[n + 1];
    for (int32_t pos = beg; pos < end; pos += 64) {
      const int32_t count = min(end - pos, 64);
      FChunk<TG::NY> ch;
      stage<TG::NY>(a.sh, a.mask, a.peer, a.csr.order, a.rows, pos, count, ch);
      for (int t0 = 0; t0 < count; t0 += 8) {
        // rows 0..7: h3 of the tile's edges, rows 8..15: their r tangents
        const int ci = t0 + (l & 7);
        const int32_t ea = __shfl(ch.e, ci);
        Split A[2];
        load_a((l & 8) ? a.t : a.h, ci < count ? hrow(a, ea) : 0, ci < count, A);
        float Gt[TG::PG][16];
        project_tile<TG::PG>(w4l, A, Gt);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (t0 + i < count) {
            const int64_t e = lane_i(ch.e, t0 + i);
            const int64_t r = lane_i(ch.peer, t0 + i);
            const float m = lane_f(ch.m, t0 + i);
            float y[TG::NY], dyv[TG::NY], go[TG::NOG], gw[TG::PG], dg[TG::PG];
#pragma unroll
            for (int j = 0; j < TG::NY; ++j) {
              y[j] = lane_f(ch.y[j], t0 + i);
              dyv[j] = 0.f;
            }
            const float* grow = grad + r * (int64_t)(TG::NO * C) + c;
#pragma unroll
            for (int k = 0; k < TG::NOG; ++k) go[k] = grow[(int64_t)TG::SLOT[k] * C];
#pragma unroll
            for (int p = 0; p < TG::PG; ++p) gw[p] = Gt[p][i] * m;
            if (!tail) TG::dx(y, gw, go, d);
            if (dsh) TG::dydg(xv, y, gw, go, dyv, dg);
            else TG::dg(xv, y, go, dg);
            float dgt = 0.f;
#pragma unroll
            for (int p = 0; p < TG::PG; ++p) dgt = fmaf(dg[p], Gt[p][8 + i], dgt);
            put_dsh_dr<TG::NY>(dsh, dr, e, dyv, m * dgt, acc != 0);
          }
          // two edges' loads in flight at most: hoisting all eight edges' cotangent rows spills
          if (i & 1) __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    if (!tail && dx) {
      float* row = dx + n * (int64_t)(NX * C) + TG::X0 * C + c;
#pragma unroll
      for (int i = 0; i < TG::NXG; ++i) row[(int64_t)i * C] = d[i];
    }
  }
}

// Gate-tangent adjoint without the feature gradient, receiver-owned: the
// receiver's cotangent row is read once per row; the tail slot `rows` holds
// edges whose receiver is out of range (zero gradients).
template <class TG>
__global__ __launch_bounds__(fused_waves<TG>() * 64, 1) void msg_fused_bwd_rcv_kernel(FusedArgs a,
                                                                                const float* __restrict__ grad,
                                                                                float* __restrict__ dsh,
                                                                                float* __restrict__ dr, int acc) {
  extern __shared__ bf16x8 w4l[];
  constexpr int NX = (TG::LI + 1) * (TG::LI + 1);
  stage_slice<TG::PG, TG::P0>(a.w4s, a.C / 64, a.cg, w4l);
  __syncthreads();
  const int C = a.C, l = lane_id(), c = 64 * a.cg + l;
  const RowRange rr = block_rows<fused_waves<TG>()>(a.rows + 1);
  for (int64_t slot = rr.first; slot < rr.end; slot += rr.stride) {
    const int64_t n = visit_row(a.csr, slot, a.rows);
    if (n < 0) continue;
    const bool tail = n == a.rows;
    float go[TG::NOG];
    if (!tail) {
      const float* grow = grad + n * (int64_t)(TG::NO * C) + c;
#pragma unroll
      for (int k = 0; k < TG::NOG; ++k) go[k] = grow[(int64_t)TG::SLOT[k] * C];
    } else {
#pragma unroll
      for (int k = 0; k < TG::NOG; ++k) go[k] = 0.f;
    }
    const int32_t beg = a.csr.ptr[n], end = a.csr.ptr[n + 1];
    for (int32_t pos = beg; pos < end; pos += 64) {
      const int32_t count = min(end - pos, 64);
      FChunk<TG::NY> ch;
      stage<TG::NY>(a.sh, a.mask, a.peer, a.csr.order, a.rows, pos, count, ch);
      for (int t0 = 0; t0 < count; t0 += 8) {
        const int ci = t0 + (l & 7);
        const int32_t ea = __shfl(ch.e, ci);
        Split A[2];
        load_a((l & 8) ? a.t : a.h, ci < count ? hrow(a, ea) : 0, ci < count, A);
        float Gt[TG::PG][16];
        project_tile<TG::PG>(w4l, A, Gt);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (t0 + i < count) {
            const int64_t e = lane_i(ch.e, t0 + i);
            const int64_t s = lane_i(ch.peer, t0 + i);
            const float m = tail ? 0.f : lane_f(ch.m, t0 + i);
            float y[TG::NY], dyv[TG::NY], xv[TG::NXG], gw[TG::PG], dg[TG::PG];
#pragma unroll
            for (int j = 0; j < TG::NY; ++j) {
              y[j] = lane_f(ch.y[j], t0 + i);
              dyv[j] = 0.f;
            }
            load_row<TG::NXG>(a.x + s * (int64_t)(NX * C) + TG::X0 * C, C, c, xv);
#pragma unroll
            for (int p = 0; p < TG::PG; ++p) gw[p] = Gt[p][i] * m;
            if (dsh) TG::dydg(xv, y, gw, go, dyv, dg);
            else TG::dg(xv, y, go, dg);
            float dgt = 0.f;
#pragma unroll
            for (int p = 0; p < TG::PG; ++p) dgt = fmaf(dg[p], Gt[p][8 + i], dgt);
            put_dsh_dr<TG::NY>(dsh, dr, e, dyv, m * dgt, acc != 0);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Input degree 0 (paths (0, l, l), the model's first layer): the tensor product
// is an outer product per edge, y[d, (l, m), c] = sum_e Y_lm(e) m_e x_s[c] g_e[l, c]
// (times the path's CG constant), so both passes are GEMMs over an edge tile
// on FP32 MFMA (v_mfma_f32_16x16x4f32) after the split-bf16 gate projection:
//   forward   Out[lm][c]  += sum_e  A[lm][e] P_l[e][c],  A = Y m coef, P_l = x g_l
//   adjoint   Q_l[e][lm]   = sum_c  P_l[e][c] go[lm][c]     (dsh = Q_l(lm), mask in P)
//             R_l[e][lm]   = sum_c  x gdot_l[e][c] go[lm][c] (dr = sum_lm Y_lm R_l(lm))
// The forward's projection result D[edge][channel] (lane (q, j): edges 4q + r,
// channel j) is directly the B operand of four 16x16x4 steps (k = q, edge
// 4q + r in step r); the adjoint projects transposed (W4 slice as the A
// operand, h3 as B), so D[channel][edge] (lane (q, i): channels 4q + r, edge
// i) is directly its A operand.  No lane transposes and no per-edge
// reductions over the 64 channels: the channel sum is the MFMA's reduction.
// ---------------------------------------------------------------------------
// 16-edge projection tiles per LDS read of a W4 slice.  Two (12 waves per CU, 168 VGPRs) measured
// 1.47 ms against 1.07 ms for one (16 waves) at the cfg4 layer-0 shape: ~40 edges per receiver fill
// 63 % of two 32-edge tiles against 83 % of three 16-edge tiles, and fewer waves hide less latency.
constexpr int kS0FwdTiles = 1;
constexpr int kS0FwdWaves = kS0FwdTiles == 1 ? 16 : 12;
constexpr int kS0BwdWaves = 16;  // 122 VGPRs: 4 waves per SIMD, one block per CU

__device__ __forceinline__ v4f mfma_f32(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int degree_of(int k) { return k < 1 ? 0 : k < 4 ? 1 : k < 9 ? 2 : 3; }

// CG constant of output component i of a degree-0-input group (one-hot harmonic, unit gate, x = 1).
template <class TG>
__device__ __forceinline__ float s0_coef(int i) {
  float x[1] = {1.f}, y[TG::NY], gw[TG::PG], o[TG::NOG];
#pragma unroll
  for (int k = 0; k < TG::NY; ++k) y[k] = k == i ? 1.f : 0.f;
#pragma unroll
  for (int p = 0; p < TG::PG; ++p) gw[p] = 1.f;
#pragma unroll
  for (int k = 0; k < TG::NOG; ++k) o[k] = 0.f;
  TG::fwd_b(x, y, gw, o);
  float c = 0.f;
#pragma unroll
  for (int k = 0; k < TG::NOG; ++k) c = k == i ? o[k] : c;
  return c;
}

// The six split-bf16 W4 operands of one (path, 16-channel block), from LDS.
struct SliceOps {
  bf16x8 h0, m0, l0, h1, m1, l1;
};
__device__ __forceinline__ SliceOps slice_ops(const bf16x8* __restrict__ w4l, int p, int cb) {
  const bf16x8* b = w4l + (p * 4 + cb) * 2 * 3 * 64 + lane_id();
  return {b[0], b[64], b[128], b[192], b[256], b[320]};
}

// Split-bf16 projection of one (path, 16-channel block) for a 16-row tile.
// TRANS = false: D[row][channel] (A = rows, B = W4 slice); true: D[channel][row].
template <bool TRANS>
__device__ __forceinline__ v4f project_block(const SliceOps& w, const Split* A) {
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  auto mm = [&](bf16x8 a, bf16x8 b) { acc = TRANS ? mfma_bf16(b, a, acc) : mfma_bf16(a, b, acc); };
  mm(A[0].lo, w.h0);
  mm(A[0].hi, w.l0);
  mm(A[0].mid, w.m0);
  mm(A[1].lo, w.h1);
  mm(A[1].hi, w.l1);
  mm(A[1].mid, w.m1);
  mm(A[0].mid, w.h0);
  mm(A[0].hi, w.m0);
  mm(A[1].mid, w.h1);
  mm(A[1].hi, w.m1);
  mm(A[0].hi, w.h0);
  mm(A[1].hi, w.h1);
  return acc;
}

// Edge id, sender and mask of up to 64 consecutive CSR positions, one edge per lane.
struct S0Chunk {
  int32_t e, s, row;  // edge, sender, its h / t row
  float m;
};
__device__ __forceinline__ S0Chunk s0_stage(const FusedArgs& a, int32_t pos, int32_t count) {
  const int l = lane_id();
  S0Chunk ch{0, 0, 0, 0.f};
  if (l < count) {
    const int32_t e = a.csr.order ? a.csr.order[pos + l] : pos + l;
    const int64_t p = a.peer[e];
    const bool ok = p >= 0 && p < a.rows;
    ch.e = e;
    ch.s = ok ? (int32_t)p : 0;
    ch.row = (int32_t)hrow(a, e);
    ch.m = ok ? (a.mask ? a.mask[e] : 1.f) : 0.f;
  }
  // complete the chunk's loads here, once per chunk: a per-tile index load or a first use inside the
  // tile loop would wait, with the same counter, for the previous tile's stores
  asm volatile("" : "+v"(ch.e), "+v"(ch.s), "+v"(ch.row), "+v"(ch.m));
  return ch;
}

template <class TG>
__global__ __launch_bounds__(kS0FwdWaves * 64, 1) void msg_s0_fwd_kernel(FusedArgs a, float* __restrict__ out) {
  static_assert(TG::LI == 0 && TG::P0 == 0 && TG::NOG == TG::NY && TG::NO == TG::NY && TG::NY <= 16,
                "degree-0 input group with one output slot per harmonic component");
  extern __shared__ bf16x8 w4l[];
  constexpr int NY = TG::NY, PG = TG::PG;
  stage_slice<PG, 0>(a.w4s, a.C / 64, a.cg, w4l);
  __syncthreads();
  const int C = a.C, l = lane_id(), q = l >> 4, j = l & 15, c0 = 64 * a.cg;
  const float coef = j < NY ? s0_coef<TG>(j) : 0.f;
  const int degj = degree_of(j);
  const RowRange rr = block_rows<kS0FwdWaves>(a.rows);
  for (int64_t slot = rr.first; slot < rr.end; slot += rr.stride) {
    const int64_t n = visit_row(a.csr, slot, a.rows);
    if (n < 0) continue;
    v4f acc[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[cb] = v4f{0.f, 0.f, 0.f, 0.f};
    const int32_t beg = a.csr.ptr[n], end = a.csr.ptr[n + 1];
    for (int32_t pos = beg; pos < end; pos += 64) {
      const int32_t count = min(end - pos, 64);
      const S0Chunk ch = s0_stage(a, pos, count);
      for (int t0 = 0; t0 < count; t0 += 16 * kS0FwdTiles) {
        // sub-tile u: projection rows = edge t0 + 16 u + j; D-layout edges t0 + 16 u + 4q + r
        Split A[kS0FwdTiles][2];
        float yv[kS0FwdTiles][4], xv[kS0FwdTiles][4][4];
#pragma unroll
        for (int u = 0; u < kS0FwdTiles; ++u) {
          const int ci = t0 + 16 * u + j;
          const int32_t ri = __shfl(ch.row, ci & 63);
          load_a(a.h, ci < count ? ri : 0, ci < count, A[u]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int k = t0 + 16 * u + 4 * q + r;
            const int32_t e = __shfl(ch.e, k & 63), s = __shfl(ch.s, k & 63);
            const float m = __shfl(ch.m, k & 63);
            const bool ok = k < count;
            yv[u][r] = ok && j < NY ? coef * m * a.sh[(int64_t)e * NY + j] : 0.f;
            const float* xs = a.x + (int64_t)s * C + c0 + j;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) xv[u][r][cb] = ok ? xs[16 * cb] : 0.f;
          }
        }
#pragma unroll
        for (int p = 0; p < PG; ++p) {
#pragma unroll
          for (int cb = 0; cb < 4; ++cb) {
            const SliceOps w = slice_ops(w4l, p, cb);
#pragma unroll
            for (int u = 0; u < kS0FwdTiles; ++u) {
              const v4f D = project_block<false>(w, A[u]);
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc[cb] = mfma_f32(degj == p ? yv[u][r] : 0.f, D[r] * xv[u][r][cb], acc[cb]);
            }
            // one slice's LDS operands live at a time
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    // lane (q, j): component 4q + r, channel 16 cb + j
    float* row = out + n * (int64_t)(NY * C) + c0 + j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int k = 4 * q + r;
      if (k < NY) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) row[(int64_t)k * C + 16 * cb] = acc[cb][r];
      }
    }
  }
}

// Receiver-owned gate-tangent adjoint (dsh and dr; no feature gradient).  The
// tail slot `rows` holds edges whose receiver is out of range: zero cotangent,
// so zero gradients.  `acc` adds to what an earlier channel group wrote.
template <class TG>
__global__ __launch_bounds__(kS0BwdWaves * 64, 1) void msg_s0_bwd_rcv_kernel(FusedArgs a,
                                                                           const float* __restrict__ grad,
                                                                           float* __restrict__ dsh,
                                                                           float* __restrict__ dr, int acc) {
  static_assert(TG::LI == 0 && TG::P0 == 0 && TG::NOG == TG::NY && TG::NO == TG::NY && TG::NY <= 16,
                "degree-0 input group with one output slot per harmonic component");
  extern __shared__ bf16x8 w4l[];
  constexpr int NY = TG::NY, PG = TG::PG;
  stage_slice<PG, 0>(a.w4s, a.C / 64, a.cg, w4l);
  __syncthreads();
  const int C = a.C, l = lane_id(), q = l >> 4, j = l & 15, c0 = 64 * a.cg;
  const float coef = j < NY ? s0_coef<TG>(j) : 0.f;
  const int degj = degree_of(j);
  const RowRange rr = block_rows<kS0BwdWaves>(a.rows + 1);
  for (int64_t slot = rr.first; slot < rr.end; slot += rr.stride) {
    const int64_t n = visit_row(a.csr, slot, a.rows);
    if (n < 0) continue;
    const bool tail = n == a.rows;
    // B operand: go[component j][channel 16 cb + 4 q + r] times the component's CG constant
    float gb[4][4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      v4f v = v4f{0.f, 0.f, 0.f, 0.f};
      if (!tail && j < NY) v = *reinterpret_cast<const v4f*>(grad + n * (int64_t)(NY * C) + (int64_t)j * C + c0 + 16 * cb + 4 * q);
#pragma unroll
      for (int r = 0; r < 4; ++r) gb[cb][r] = coef * v[r];
    }
    const int32_t beg = a.csr.ptr[n], end = a.csr.ptr[n + 1];
    for (int32_t pos = beg; pos < end; pos += 64) {
      const int32_t count = min(end - pos, 64);
      const S0Chunk ch = s0_stage(a, pos, count);
      for (int t0 = 0; t0 < count; t0 += 8) {
        // 8-edge tiles: projection column / contraction row j holds edge t0 + (j & 7), its h3 in rows 0..7 and
        // its t3 in rows 8..15, so one projection and one contraction chain give the gates' Q (rows 0..7) and
        // the tangents' R (rows 8..15) together
        const int ci = t0 + (j & 7);
        const bool oki = ci < count;
        const int32_t si = __shfl(ch.s, ci & 63);
        const float mi = __shfl(ch.m, ci & 63);
        const int64_t hr = oki ? __shfl(ch.row, ci & 63) : 0;
        Split A[2];
        load_a((j & 8) ? a.t : a.h, hr, oki, A);
        // sender features of the row's edge at channels 16 cb + 4 q .. + 3, times the mask
        float xv[4][4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
          v4f v = v4f{0.f, 0.f, 0.f, 0.f};
          if (oki) v = *reinterpret_cast<const v4f*>(a.x + (int64_t)si * C + c0 + 16 * cb + 4 * q);
#pragma unroll
          for (int r = 0; r < 4; ++r) xv[cb][r] = mi * v[r];
        }
        // harmonics of the rows' edges for dr (lanes q >= 2), loaded with the tile's other operands: a load
        // after the contraction would wait, with the same counter, for the stores before it
        float shv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int k = t0 + 4 * (q & 1) + r;
          const int32_t ek = __shfl(ch.e, k & 63);
          shv[r] = k < count && j < NY && q >= 2 ? a.sh[(int64_t)ek * NY + j] : 0.f;
        }
        v4f QR[PG];
#pragma unroll
        for (int p = 0; p < PG; ++p) {
          QR[p] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int cb = 0; cb < 4; ++cb) {
            const SliceOps w = slice_ops(w4l, p, cb);
            const v4f G = project_block<true>(w, A);
#pragma unroll
            for (int r = 0; r < 4; ++r) QR[p] = mfma_f32(G[r] * xv[cb][r], gb[cb][r], QR[p]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        // lane (q, j): rows 4q + r (q < 2: dsh of edge t0 + 4q + r; q >= 2: R of edge t0 + 4(q - 2) + r),
        // component j
        float dv[4];
        int32_t eo[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int k = t0 + 4 * (q & 1) + r;
          eo[r] = __shfl(ch.e, k & 63);
          float v = 0.f;
#pragma unroll
          for (int p = 0; p < PG; ++p) v = degj == p ? QR[p][r] : v;
          const bool ok = k < count && j < NY;
          dv[r] = ok && q >= 2 ? shv[r] * v : 0.f;
          if (ok && q < 2 && dsh) {
            float* d = dsh + (int64_t)eo[r] * NY + j;
            *d = acc ? *d + v : v;
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int off = 8; off > 0; off >>= 1) dv[r] += __shfl_xor(dv[r], off);
        }
        if (j == 0 && q >= 2) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (t0 + 4 * (q & 1) + r < count) {
              float* d = dr + eo[r];
              *d = acc ? *d + dv[r] : dv[r];
            }
          }
        }
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Species form of the degree-0-input message (the model's first layer).
//
// There the features are a function of the species alone, x[s] = X[sp(s)]
// (embedding, then linear_up), so with the gates g_e[l, c] = sum_k h3_e[k]
// W4[l C + c, k] the message of path (0, l, l) factorises:
//   out[d, lm, c] = coef_l sum_{e -> d} m_e Y_lm(e) X[sp(s_e), c] g_e[l, c]
//                 = sum_{sp, k} Wf_l[c, (sp, k)] H[d, lm, (sp, k)],
//   H[d, lm, (sp, k)] = sum_{e -> d, sp(s_e) = sp} m_e Y_lm(e) h3_e[k],
//   Wf_l[c, (sp, k)]  = coef_l X[sp, c] w[l, c] W4[l C + c, k]   (w: TP path weight).
// The edge loop only accumulates Y h3 outer products in the hidden space
// (9 FMAs per lane and edge, no per-edge gate projection), and one GEMM per
// output component (K = S * 64, FP32 MFMA) applies the projection per node.
// The energy-and-forces adjoint uses the same factorisation:
//   Z[d, lm, (sp, k)] = sum_c go[d, lm, c] Wf_l[c, (sp, k)]          (GEMM per component)
//   dsh[e, lm] = m_e sum_k h3_e[k] Z[d, lm, (sp_e, k)]
//   dr[e]      = m_e sum_lm Y_lm(e) sum_k t3_e[k] Z[d, lm, (sp_e, k)]
// one wave per receiver row, lane = hidden index k, Z of the row in registers.
// ---------------------------------------------------------------------------
constexpr int kSpeciesMax = 4;
constexpr int kSpWaves = 4;

struct SpeciesArgs {
  const float* sh;          // [E, NY]
  const float* h3;          // [G, 64] (rows through grow)
  const float* t3;          // [G, 64] (adjoint only)
  const float* mask;        // [E] or nullptr
  const int64_t* src;       // [E]
  const int64_t* species;   // [N] species index of each node
  const int32_t* grow;      // [E] gate row of each edge, nullptr = the edge itself
  int64_t rows, edges;
  int S;
  Csr csr;                  // receiver CSR
};

struct SpChunk {
  int32_t e, row, sp;
  float m;
};

__device__ __forceinline__ SpChunk sp_stage(const SpeciesArgs& a, int32_t pos, int32_t count) {
  const int l = lane_id();
  SpChunk ch{0, 0, 0, 0.f};
  if (l < count) {
    const int32_t e = a.csr.order ? a.csr.order[pos + l] : pos + l;
    const int64_t s = a.src[e];
    const int64_t sp = (s >= 0 && s < a.rows) ? a.species[s] : -1;
    const bool ok = sp >= 0 && sp < a.S;
    ch.e = e;
    ch.row = a.grow ? a.grow[e] : e;
    ch.sp = ok ? (int32_t)sp : 0;
    ch.m = ok ? (a.mask ? a.mask[e] : 1.f) : 0.f;
  }
  asm volatile("" : "+v"(ch.e), "+v"(ch.row), "+v"(ch.sp), "+v"(ch.m));
  return ch;
}

__device__ __forceinline__ int64_t sp_slot() { return xcd_block(blockIdx.x, gridDim.x) * kSpWaves + wave_id(); }

// Row of H / Z holding (node n, output component lm): the components of degree l
// are stored together, [N, 2l+1, K] after the blocks of the lower degrees, so
// that each degree's projection is one GEMM over contiguous rows.
__device__ __forceinline__ int64_t hz_row(int64_t n, int lm, int64_t N) {
  const int l = lm < 1 ? 0 : lm < 4 ? 1 : 2;
  return N * (int64_t)(l * l) + n * (2 * l + 1) + (lm - l * l);
}

// H[n, lm, (sp, k)] of every receiver row n on FP32 MFMA (v_mfma_f32_16x16x4f32), four edges per step:
// A[lm][edge] = m Y_lm [species == sp] (lane: row lm = l % 16, edge l / 16), B[edge][k] = h3[edge][k]
// (lane: edge l / 16, column k = 16 cb + l % 16); one accumulator per (species, 16-column block).
// PARTS waves share a row, each taking 4 / PARTS of the 16-column blocks of k: fewer accumulators per
// wave, so more waves (and more edges' loads) in flight on this latency-bound pass.
template <int NY, int S, int PARTS>
__global__ __launch_bounds__(kSpWaves * 64) void species_fwd_kernel(SpeciesArgs a, float* __restrict__ H) {
  constexpr int CBW = 4 / PARTS;
  const int64_t wslot = sp_slot();
  const int64_t slot = wslot / PARTS;
  const int cb0 = (int)(wslot % PARTS) * CBW;
  if (slot >= a.rows) return;
  const int64_t n = visit_row(a.csr, slot, a.rows);
  if (n < 0) return;
  const int l = lane_id(), col = l & 15, eg = l >> 4;
  v4f acc[S][CBW];
#pragma unroll
  for (int b = 0; b < S; ++b)
#pragma unroll
    for (int cb = 0; cb < CBW; ++cb) acc[b][cb] = v4f{0.f, 0.f, 0.f, 0.f};
  const int32_t beg = a.csr.ptr[n], end = a.csr.ptr[n + 1];
  for (int32_t pos = beg; pos < end; pos += 64) {
    const int32_t count = min(end - pos, 64);
    const SpChunk ch = sp_stage(a, pos, count);
    // two 4-edge steps per iteration: both steps' loads are in flight before the first MFMA
    for (int t0 = 0; t0 < count; t0 += 8) {
      float yv[2], hb[2][CBW];
      int32_t spv[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ci = t0 + 4 * u + eg;
        const bool ok = ci < count;
        const int src_lane = min(ci, 63);
        const int32_t e = __shfl(ch.e, src_lane), row = __shfl(ch.row, src_lane);
        spv[u] = __shfl(ch.sp, src_lane);
        const float m = __shfl(ch.m, src_lane);
        yv[u] = (ok && col < NY) ? m * a.sh[(int64_t)e * NY + col] : 0.f;
#pragma unroll
        for (int cb = 0; cb < CBW; ++cb) hb[u][cb] = ok ? a.h3[(int64_t)row * 64 + 16 * (cb0 + cb) + col] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int b = 0; b < S; ++b) {
          const float av = spv[u] == b ? yv[u] : 0.f;
#pragma unroll
          for (int cb = 0; cb < CBW; ++cb) acc[b][cb] = mfma_f32(av, hb[u][cb], acc[b][cb]);
        }
    }
  }
  // D: lane (q, j) holds rows lm = 4 q + r, column k = 16 cb + j
  const int q = l >> 4;
  const int64_t K = (int64_t)S * 64;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int lm = 4 * q + r;
    if (lm < NY) {
      float* out = H + hz_row(n, lm, a.rows) * K + col;
#pragma unroll
      for (int b = 0; b < S; ++b)
#pragma unroll
        for (int cb = 0; cb < CBW; ++cb) out[b * 64 + 16 * (cb0 + cb)] = acc[b][cb][r];
    }
  }
}

// dsh and dr of every edge, eight edges per tile on split-bf16 MFMA: A rows 0..7 are the tile edges' h3,
// rows 8..15 their t3 (k = 32 ks + 8 (l / 16) + e), B the receiver's Z of one species transposed (column
// lm = l % 16), so D[row][lm] gives sum_k h3 Z (dsh, before the mask) and sum_k t3 Z (dr's terms).  The
// tail slot `rows` holds edges whose receiver is out of range: zero Z, zero gradients.
template <int NY, int S>
__global__ __launch_bounds__(kSpWaves * 64) void species_bwd_kernel(SpeciesArgs a, const float* __restrict__ Z,
                                                                     float* __restrict__ dsh, float* __restrict__ dr) {
  const int64_t slot = sp_slot();
  if (slot > a.rows) return;
  const int64_t n = visit_row(a.csr, slot, a.rows);
  if (n < 0) return;
  const bool tail = n == a.rows;
  const int l = lane_id(), j = l & 15, q = l >> 4;
  const int64_t K = (int64_t)S * 64;
  SliceOps Bz[S];
#pragma unroll
  for (int b = 0; b < S; ++b) {
    Split part[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float v[8];
      if (!tail && j < NY) {
        const float* zp = Z + hz_row(n, j, a.rows) * K + b * 64 + 32 * ks + 8 * q;
        const v4f x0 = *reinterpret_cast<const v4f*>(zp), x1 = *reinterpret_cast<const v4f*>(zp + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = x0[e];
          v[4 + e] = x1[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.f;
      }
      part[ks] = split8(v);
    }
    Bz[b] = SliceOps{part[0].hi, part[0].mid, part[0].lo, part[1].hi, part[1].mid, part[1].lo};
  }
  const int32_t beg = a.csr.ptr[n], end = a.csr.ptr[n + 1];
  for (int32_t pos = beg; pos < end; pos += 64) {
    const int32_t count = min(end - pos, 64);
    const SpChunk ch = sp_stage(a, pos, count);
    for (int t0 = 0; t0 < count; t0 += 8) {
      const int ci = t0 + (j & 7);
      const bool oki = ci < count;
      const int32_t ri = __shfl(ch.row, min(ci, 63));
      Split A[2];
      load_a((j & 8) ? a.t3 : a.h3, oki ? ri : 0, oki, A);
      // the edges of this lane's D rows: t0 + 4 (q & 1) + r
      int32_t eo[4], so[4];
      float mo[4], yo[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = t0 + 4 * (q & 1) + r;
        const int kl = min(k, 63);
        eo[r] = __shfl(ch.e, kl);
        so[r] = __shfl(ch.sp, kl);
        const float mv = __shfl(ch.m, kl);
        mo[r] = k < count ? mv : 0.f;
        yo[r] = (k < count && j < NY && q >= 2) ? a.sh[(int64_t)eo[r] * NY + j] : 0.f;
      }
      v4f D[S];
#pragma unroll
      for (int b = 0; b < S; ++b) D[b] = project_block<false>(Bz[b], A);
      float w[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = D[0][r];
#pragma unroll
        for (int b = 1; b < S; ++b) v = so[r] == b ? D[b][r] : v;
        const int k = t0 + 4 * (q & 1) + r;
        if (q < 2) {
          if (k < count && j < NY) dsh[(int64_t)eo[r] * NY + j] = mo[r] * v;
          w[r] = 0.f;
        } else {
          w[r] = yo[r] * v;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        w[r] += dpp_mov<0x128>(w[r]);   // row_ror:8
        w[r] += dpp_mov<0x124>(w[r]);   // row_ror:4
        w[r] += dpp_mov<0x122>(w[r]);   // row_ror:2
        w[r] += dpp_mov<0x121>(w[r]);   // row_ror:1
      }
      if (q >= 2 && j == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (t0 + 4 * (q & 1) + r < count) dr[eo[r]] = mo[r] * w[r];
      }
    }
  }
}


// Projection GEMM of the species form, C = A . B^T with B [NB*16, KS*32] small and constant:
// B is split once per block into LDS in the MFMA operand layout (NB*KS*3 KB), and each wave streams
// 16-row tiles of A straight from HBM (lane l: row l % 16, k = 32 ks + 8 (l / 16) .. + 7), splits them
// and multiplies on split-bf16 MFMA (six products, FP32-level accuracy); no LDS traffic for A and no
// barriers after the staging.  Rows of A and C map through (group, group stride, pitch): row r at
// (r / g) * gs + (r % g) * ld.
struct ProjMap {
  int64_t ld, group, gstride;
  __device__ __forceinline__ int64_t off(int64_t r) const {
    const uint32_t g = (uint32_t)r / (uint32_t)group;
    return (int64_t)g * gstride + (int64_t)((uint32_t)r - g * (uint32_t)group) * ld;
  }
};

constexpr int kProjWaves = 8;

template <int KS, int NB>
__global__ __launch_bounds__(kProjWaves * 64) void species_proj_kernel(const float* __restrict__ A, int64_t M,
                                                                        ProjMap am, const float* __restrict__ B,
                                                                        float* __restrict__ C, ProjMap cm) {
  extern __shared__ bf16x8 bl[];   // [NB][KS][3][64]
  constexpr int K = KS * 32;
  for (int t = threadIdx.x; t < NB * KS * 64; t += blockDim.x) {
    const int lane = t & 63, ks = (t >> 6) % KS, j = (t >> 6) / KS;
    const float* p = B + (int64_t)(16 * j + (lane & 15)) * K + 32 * ks + 8 * (lane >> 4);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = p[e];
    const Split sp = split8(v);
    bf16x8* o = bl + ((j * KS + ks) * 3) * 64 + lane;
    o[0] = sp.hi;
    o[64] = sp.mid;
    o[128] = sp.lo;
  }
  __syncthreads();
  const int l = lane_id();
  const int64_t tiles = (M + 15) / 16;
  const int64_t wstride = (int64_t)gridDim.x * kProjWaves;
  for (int64_t tile = (int64_t)blockIdx.x * kProjWaves + wave_id(); tile < tiles; tile += wstride) {
    // B is re-read from LDS per tile: hoisted out of the loop it would take NB * KS * 12 VGPRs
    asm volatile("" ::: "memory");
    const int64_t row = tile * 16 + (l & 15);
    const bool ok = row < M;
    const float* ap = A + (ok ? am.off(row) : 0) + 8 * (l >> 4);
    v4f acc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
    float av[KS][8];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ok) {
        const v4f x0 = *reinterpret_cast<const v4f*>(ap + 32 * ks), x1 = *reinterpret_cast<const v4f*>(ap + 32 * ks + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          av[ks][e] = x0[e];
          av[ks][4 + e] = x1[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) av[ks][e] = 0.f;
      }
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const Split a = split8(av[ks]);
#pragma unroll
      for (int j = 0; j < NB; ++j) {
        const bf16x8* b = bl + ((j * KS + ks) * 3) * 64 + l;
        const bf16x8 bh = b[0], bm = b[64], blo = b[128];
        acc[j] = mfma_bf16(a.lo, bh, acc[j]);
        acc[j] = mfma_bf16(a.hi, blo, acc[j]);
        acc[j] = mfma_bf16(a.mid, bm, acc[j]);
        acc[j] = mfma_bf16(a.mid, bh, acc[j]);
        acc[j] = mfma_bf16(a.hi, bm, acc[j]);
        acc[j] = mfma_bf16(a.hi, bh, acc[j]);
      }
    }
    // D: lane (q, j16) holds rows 4 q + r of the tile, column 16 j + j16
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t rr = tile * 16 + 4 * (l >> 4) + r;
      if (rr < M) {
        float* c = C + cm.off(rr) + (l & 15);
#pragma unroll
        for (int j = 0; j < NB; ++j) c[16 * j] = acc[j][r];
      }
    }
  }
}

// Wf[p][c][sp*64 + k] = coef_p X[sp, c] w[p, c] W4[p C + c, k] and Wb[p][sp*64 + k][c] = the same value:
// the B operands of the forward (N = C, K = S*64) and adjoint (N = S*64, K = C) GEMMs of path p.
template <class TG>
__global__ void species_weight_kernel(const float* __restrict__ X, int S, int C, const float* __restrict__ W4,
                                      const float* __restrict__ tpw, float* __restrict__ Wf, float* __restrict__ Wb) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per = (int64_t)C * S * 64;
  if (t >= TG::PG * per) return;
  const int p = (int)(t / per), r = (int)(t % per);
  const int c = r / (S * 64), sk = r % (S * 64), sp = sk / 64, k = sk % 64;
  // the path's CG constant: the component coefficient of the path's first output slot (one slot per path)
  int first = 0;
  for (int q = 0; q < p; ++q) first += 2 * q + 1;
  const float coef = s0_coef<TG>(first);
  const float w = tpw ? tpw[(int64_t)p * C + c] : 1.f;
  const float v = coef * (X[(int64_t)sp * C + c] * w) * W4[((int64_t)p * C + c) * 64 + k];
  Wf[(int64_t)p * per + (int64_t)c * S * 64 + sk] = v;
  Wb[(int64_t)p * per + (int64_t)sk * C + c] = v;
}

int fail(int code, const char* msg) { return set_error(code, msg); }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return ICTC_OK;
  char buf[256];
  snprintf(buf, sizeof(buf), "%s: %s", what, hipGetErrorString(e));
  return fail(ICTC_ERR_RUNTIME, buf);
}

int cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}


// ---- species form: launch helpers ----
int64_t align256(int64_t b) { return (b + 255) & ~(int64_t)255; }

struct SpeciesLayout {
  int64_t hz, wf, wb, total;   // byte offsets of H (or Z), Wf, Wb; total bytes
};
SpeciesLayout species_layout(int ny, int paths, int S, int C, int64_t N) {
  SpeciesLayout L;
  L.hz = 0;
  L.wf = align256(N * ny * S * 64 * (int64_t)sizeof(float));
  L.wb = L.wf + align256((int64_t)paths * C * S * 64 * sizeof(float));
  L.total = L.wb + align256((int64_t)paths * C * S * 64 * sizeof(float));
  return L;
}

template <class TG>
int species_weights(const float* X, int S, int C, const float* W4, const float* tpw, float* Wf, float* Wb,
                    hipStream_t st) {
  const int64_t n = (int64_t)TG::PG * C * S * 64;
  hipLaunchKernelGGL(species_weight_kernel<TG>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, X, S, C, W4, tpw,
                     Wf, Wb);
  return launch_status("species weight launch");
}

int species_check(int le, int lo, int C, int S, int64_t N, int64_t E) {
  if (!(le == lo && le >= 0 && le <= 2))
    return fail(ICTC_ERR_UNSUPPORTED, "species message: edge_lmax == output_lmax <= 2 only");
  if (S < 1 || S > kSpeciesMax) return fail(ICTC_ERR_UNSUPPORTED, "species message: 1..4 species");
  if (C <= 0 || C > 64 * kMaxGroups) return fail(ICTC_ERR_UNSUPPORTED, "species message: channels 1..256");
  if (N < 0 || E < 0 || N > INT32_MAX || E > INT32_MAX) return fail(ICTC_ERR_ARGUMENT, "species message: bad sizes");
  return ICTC_OK;
}

template <int LE>
int species_weights_le(const float* X, int S, int C, const float* W4, const float* tpw, float* Wf, float* Wb,
                       hipStream_t st) {
  return species_weights<TpG<0, LE, LE, 0>>(X, S, C, W4, tpw, Wf, Wb, st);
}

int species_weights_any(int le, const float* X, int S, int C, const float* W4, const float* tpw, float* Wf, float* Wb,
                        hipStream_t st) {
  switch (le) {
    case 0: return species_weights_le<0>(X, S, C, W4, tpw, Wf, Wb, st);
    case 1: return species_weights_le<1>(X, S, C, W4, tpw, Wf, Wb, st);
    default: return species_weights_le<2>(X, S, C, W4, tpw, Wf, Wb, st);
  }
}


template <int NY, int S>
void species_fwd_launch(const SpeciesArgs& a, float* H, hipStream_t st) {
  constexpr int PARTS = 2;   // 766 -> 703 us at cfg4 (one wave per row); 4 parts: 1016 us
  const unsigned blocks = (unsigned)((a.rows * PARTS + kSpWaves - 1) / kSpWaves);
  hipLaunchKernelGGL((species_fwd_kernel<NY, S, PARTS>), dim3(blocks), dim3(kSpWaves * 64), 0, st, a, H);
}
template <int NY, int S>
void species_bwd_launch(const SpeciesArgs& a, const float* Z, float* dsh, float* dr, hipStream_t st) {
  const unsigned blocks = (unsigned)((a.rows + 1 + kSpWaves - 1) / kSpWaves);
  hipLaunchKernelGGL((species_bwd_kernel<NY, S>), dim3(blocks), dim3(kSpWaves * 64), 0, st, a, Z, dsh, dr);
}
template <int NY>
void species_fwd_ny(const SpeciesArgs& a, float* H, hipStream_t st) {
  switch (a.S) {
    case 1: species_fwd_launch<NY, 1>(a, H, st); break;
    case 2: species_fwd_launch<NY, 2>(a, H, st); break;
    case 3: species_fwd_launch<NY, 3>(a, H, st); break;
    default: species_fwd_launch<NY, 4>(a, H, st); break;
  }
}
template <int NY>
void species_bwd_ny(const SpeciesArgs& a, const float* Z, float* dsh, float* dr, hipStream_t st) {
  switch (a.S) {
    case 1: species_bwd_launch<NY, 1>(a, Z, dsh, dr, st); break;
    case 2: species_bwd_launch<NY, 2>(a, Z, dsh, dr, st); break;
    case 3: species_bwd_launch<NY, 3>(a, Z, dsh, dr, st); break;
    default: species_bwd_launch<NY, 4>(a, Z, dsh, dr, st); break;
  }
}


int proj_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}

// C [M, NB*16] = A [M, KS*32] . B^T through species_proj_kernel (B row-major [NB*16, KS*32]).
template <int KS, int NB>
int species_proj(const float* A, int64_t M, ProjMap am, const float* B, float* C, ProjMap cm, hipStream_t st) {
  if (M <= 0) return ICTC_OK;
  const int64_t tiles = (M + 15) / 16;
  const int64_t blocks = std::min<int64_t>((tiles + kProjWaves - 1) / kProjWaves, 2 * (int64_t)proj_cus());
  const size_t lds = (size_t)NB * KS * 3 * 64 * sizeof(bf16x8);
  hipLaunchKernelGGL((species_proj_kernel<KS, NB>), dim3((unsigned)blocks), dim3(kProjWaves * 64), lds, st, A, M, am,
                     B, C, cm);
  return launch_status("species projection launch");
}

// Channel counts with compiled projection kernels: the forward's output width and the adjoint's
// reduction length are C; species widths S*64 with S <= 4.
template <int CB>
int species_proj_fwd_c(int S, const float* A, int64_t M, ProjMap am, const float* B, float* C, ProjMap cm,
                       hipStream_t st) {
  switch (S) {
    case 1: return species_proj<2, CB>(A, M, am, B, C, cm, st);
    case 2: return species_proj<4, CB>(A, M, am, B, C, cm, st);
    case 3: return species_proj<6, CB>(A, M, am, B, C, cm, st);
    default: return species_proj<8, CB>(A, M, am, B, C, cm, st);
  }
}
template <int KS>
int species_proj_bwd_c(int S, const float* A, int64_t M, ProjMap am, const float* B, float* C, ProjMap cm,
                       hipStream_t st) {
  switch (S) {
    case 1: return species_proj<KS, 4>(A, M, am, B, C, cm, st);
    case 2: return species_proj<KS, 8>(A, M, am, B, C, cm, st);
    case 3: return species_proj<KS, 12>(A, M, am, B, C, cm, st);
    default: return species_proj<KS, 16>(A, M, am, B, C, cm, st);
  }
}

enum class Pass { kFwd, kBwdSrc, kBwdRcv };

struct Launch {
  Pass pass;
  FusedArgs a;
  const float* grad;
  float *out, *dx, *dsh, *dr;
  int acc;
  hipStream_t st;
};

template <class TG>
int launch_group(const Launch& L) {
  const size_t lds = (size_t)TG::PG * kSlice * sizeof(bf16x8);
  if constexpr (TG::LI == 0) {
    // degree-0 input: the MFMA contraction kernels (the source-owned adjoint keeps the generic kernel)
    if (L.pass == Pass::kFwd) {
      hipLaunchKernelGGL(msg_s0_fwd_kernel<TG>, dim3((unsigned)cus()), dim3(kS0FwdWaves * 64), lds, L.st, L.a, L.out);
      return launch_status("fused message launch");
    }
    if (L.pass == Pass::kBwdRcv) {
      hipLaunchKernelGGL(msg_s0_bwd_rcv_kernel<TG>, dim3((unsigned)cus()), dim3(kS0BwdWaves * 64), lds, L.st,
                         L.a, L.grad, L.dsh, L.dr, L.acc);
      return launch_status("fused message launch");
    }
  }
  const dim3 grid((unsigned)cus()), block(fused_waves<TG>() * 64);
  switch (L.pass) {
    case Pass::kFwd:
      hipLaunchKernelGGL(msg_fused_fwd_kernel<TG>, grid, block, lds, L.st, L.a, L.out);
      break;
    case Pass::kBwdSrc:
      hipLaunchKernelGGL(msg_fused_bwd_src_kernel<TG>, grid, block, lds, L.st, L.a, L.grad, L.dx, L.dsh, L.dr, L.acc);
      break;
    case Pass::kBwdRcv:
      hipLaunchKernelGGL(msg_fused_bwd_rcv_kernel<TG>, grid, block, lds, L.st, L.a, L.grad, L.dsh, L.dr, L.acc);
      break;
  }
  return launch_status("fused message launch");
}

// Path groups of the compiled degree triples, in launch order (l1 ascending).
#define ICTC_FUSED_SHAPES(X) \
  X(0, 2, 2) X(1, 2, 2) X(2, 2, 2)

template <int LI, int LE, int LO, int L1>
int run_groups(Launch L, int first) {
  if constexpr (L1 > LI) {
    return ICTC_OK;
  } else {
    L.acc = first ? 0 : 1;
    if (int rc = launch_group<TpG<LI, LE, LO, L1>>(L)) return rc;
    return run_groups<LI, LE, LO, L1 + 1>(L, 0);
  }
}

int run_all(int li, int le, int lo, const Launch& L, int first) {
#define ICTC_CASE(A, B, C) \
  if (li == A && le == B && lo == C) return run_groups<A, B, C, 0>(L, first);
  ICTC_FUSED_SHAPES(ICTC_CASE)
#undef ICTC_CASE
  return fail(ICTC_ERR_UNSUPPORTED, "fused message: degree triple not compiled");
}

bool fused_shape(int li, int le, int lo) {
#define ICTC_CASE(A, B, C) \
  if (li == A && le == B && lo == C) return true;
  ICTC_FUSED_SHAPES(ICTC_CASE)
#undef ICTC_CASE
  return false;
}

int check(int li, int le, int lo, int C, int64_t N, int64_t E) {
  if (!fused_shape(li, le, lo)) return fail(ICTC_ERR_UNSUPPORTED, "fused message: degree triple not compiled");
  if (C <= 0 || C % 64 || C > 64 * kMaxGroups)
    return fail(ICTC_ERR_UNSUPPORTED, "fused message: channels must be a multiple of 64 up to 256");
  if (N < 0 || E < 0 || N > INT32_MAX || E > INT32_MAX) return fail(ICTC_ERR_ARGUMENT, "fused message: bad sizes");
  return ICTC_OK;
}

}  // namespace
}  // namespace ictc

using namespace ictc;

extern "C" {

int ictc_fused_supported(int input_lmax, int edge_lmax, int output_lmax, int channels) {
  return fused_shape(input_lmax, edge_lmax, output_lmax) && channels > 0 && channels % 64 == 0 &&
         channels <= 64 * kMaxGroups;
}

int64_t ictc_fused_weight_bytes(int paths, int channels) {
  if (paths <= 0 || channels <= 0 || channels % 64) return -1;
  return (int64_t)paths * (channels / 64) * kSlice * (int64_t)sizeof(bf16x8);
}

int ictc_fused_weight_split(const float* W4, const float* tp_weight, int paths, int channels, void* out,
                            int64_t out_bytes, void* stream) {
  const int64_t need = ictc_fused_weight_bytes(paths, channels);
  if (need < 0) return fail(ICTC_ERR_ARGUMENT, "fused weight split: paths > 0 and channels a multiple of 64");
  if (!W4 || !out) return fail(ICTC_ERR_ARGUMENT, "fused weight split: null operand");
  if (out_bytes < need) return fail(ICTC_ERR_ARGUMENT, "fused weight split: output smaller than ictc_fused_weight_bytes");
  if (reinterpret_cast<uintptr_t>(out) & 15) return fail(ICTC_ERR_ARGUMENT, "fused weight split: output not 16-byte aligned");
  const int64_t threads = (int64_t)paths * (channels / 64) * 4 * 2 * 64;
  hipLaunchKernelGGL(fused_split_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     W4, tp_weight, paths, channels, (bf16x8*)out);
  return launch_status("ictc_fused_weight_split launch");
}

int ictc_msg_fused_fwd(int li, int le, int lo, int C, const float* x, const float* sh, const float* h3,
                       const void* w4split, const float* mask, const int64_t* src, int64_t N, int64_t E,
                       const int32_t* dptr, const int32_t* dorder, const int32_t* dst_rows, float* out,
                       const int32_t* gate_rows, void* stream) {
  if (int rc = check(li, le, lo, C, N, E)) return rc;
  if (N == 0) return ICTC_OK;
  if (!x || !out || !dptr || (E > 0 && (!sh || !h3 || !w4split || !src)))
    return fail(ICTC_ERR_ARGUMENT, "ictc_msg_fused_fwd: null operand");
  if ((reinterpret_cast<uintptr_t>(h3) | reinterpret_cast<uintptr_t>(w4split)) & 15)
    return fail(ICTC_ERR_ARGUMENT, "ictc_msg_fused_fwd: h3 and the split weight must be 16-byte aligned");
  Launch L{Pass::kFwd,
           FusedArgs{x, sh, h3, nullptr, (const bf16x8*)w4split, mask, src, N, E, C, 0, Csr{dptr, dorder, dst_rows},
                     gate_rows},
           nullptr, out, nullptr, nullptr, nullptr, 0, (hipStream_t)stream};
  for (int cg = 0; cg < C / 64; ++cg) {
    L.a.cg = cg;
    if (int rc = run_all(li, le, lo, L, 1)) return rc;
  }
  return ICTC_OK;
}

int ictc_msg_fused_bwd_tangent(int li, int le, int lo, int C, const float* x, const float* sh, const float* h3,
                               const float* t3, const void* w4split, const float* mask, const int64_t* src,
                               const int64_t* dst, int64_t N, int64_t E, const int32_t* dptr, const int32_t* dorder,
                               const int32_t* sptr, const int32_t* sorder, const int32_t* dst_rows,
                               const int32_t* src_rows, const float* grad, float* dx, float* dsh, float* dr,
                               const int32_t* gate_rows, void* stream) {
  if (int rc = check(li, le, lo, C, N, E)) return rc;
  if (E == 0) {
    // no edges: dsh and dr are empty, dx is zero
    const int64_t n = dx ? N * (int64_t)(C * (li + 1) * (li + 1)) : 0;
    if (n == 0) return ICTC_OK;
    hipLaunchKernelGGL(fused_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, dx, n);
    return launch_status("ictc_msg_fused_bwd_tangent dx fill");
  }
  if (!dr) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_fused_bwd_tangent: dr is required");
  if (!x || !sh || !h3 || !t3 || !w4split || !src || !dst || !grad || !dptr)
    return fail(ICTC_ERR_ARGUMENT, "ictc_msg_fused_bwd_tangent: null operand");
  if (dx && !sptr) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_fused_bwd_tangent: dfeatures needs the source CSR");
  if ((reinterpret_cast<uintptr_t>(h3) | reinterpret_cast<uintptr_t>(t3) | reinterpret_cast<uintptr_t>(w4split)) & 15)
    return fail(ICTC_ERR_ARGUMENT, "ictc_msg_fused_bwd_tangent: h3, t3 and the split weight must be 16-byte aligned");
  const bool src_owned = dx != nullptr;
  Launch L{src_owned ? Pass::kBwdSrc : Pass::kBwdRcv,
           FusedArgs{x, sh, h3, t3, (const bf16x8*)w4split, mask, src_owned ? dst : src, N, E, C, 0,
                     src_owned ? Csr{sptr, sorder, src_rows} : Csr{dptr, dorder, dst_rows}, gate_rows},
           grad, nullptr, dx, dsh, dr, 0, (hipStream_t)stream};
  for (int cg = 0; cg < C / 64; ++cg) {
    L.a.cg = cg;
    if (int rc = run_all(li, le, lo, L, cg == 0)) return rc;
  }
  return ICTC_OK;
}

int64_t ictc_species_message_workspace_bytes(int edge_lmax, int species, int channels, int64_t nodes) {
  if (edge_lmax < 0 || edge_lmax > 2 || species < 1 || species > kSpeciesMax || channels <= 0 || nodes < 0) return -1;
  const int ny = (edge_lmax + 1) * (edge_lmax + 1);
  return species_layout(ny, edge_lmax + 1, species, channels, nodes).total;
}

int ictc_species_message_fwd(int edge_lmax, int output_lmax, int C, int S, const float* xtab, const int64_t* species,
                             const float* sh, const float* h3, const float* W4, const float* tp_weight,
                             const float* mask, const int64_t* src, int64_t N, int64_t E, const int32_t* dptr,
                             const int32_t* dorder, const int32_t* dst_rows, const int32_t* gate_rows, float* out,
                             void* ws, int64_t ws_bytes, void* stream) {
  if (int rc = species_check(edge_lmax, output_lmax, C, S, N, E)) return rc;
  if (N == 0) return ICTC_OK;
  const int ny = (edge_lmax + 1) * (edge_lmax + 1), P = edge_lmax + 1;
  if (!xtab || !species || !W4 || !out || !dptr || !ws || (E > 0 && (!sh || !h3 || !src)))
    return fail(ICTC_ERR_ARGUMENT, "ictc_species_message_fwd: null operand");
  const SpeciesLayout L = species_layout(ny, P, S, C, N);
  if (ws_bytes < L.total) return fail(ICTC_ERR_ARGUMENT, "ictc_species_message_fwd: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  char* base = static_cast<char*>(ws);
  float *H = (float*)(base + L.hz), *Wf = (float*)(base + L.wf), *Wb = (float*)(base + L.wb);
  if (int rc = species_weights_any(edge_lmax, xtab, S, C, W4, tp_weight, Wf, Wb, st)) return rc;
  SpeciesArgs a{sh, h3, nullptr, mask, src, species, gate_rows, N, E, S, Csr{dptr, dorder, dst_rows}};
  switch (ny) {
    case 1: species_fwd_ny<1>(a, H, st); break;
    case 4: species_fwd_ny<4>(a, H, st); break;
    default: species_fwd_ny<9>(a, H, st); break;
  }
  if (int rc = launch_status("ictc_species_message_fwd launch")) return rc;
  // per degree l: out[n, l^2 + m, :] = H_l[n, m, :] . Wf_l^T, H_l the rows [N (2l+1), S*64] of degree l
  const int64_t K = (int64_t)S * 64;
  for (int l = 0; l <= edge_lmax; ++l) {
    const int64_t g = 2 * l + 1;
    const float* Al = H + N * (int64_t)(l * l) * K;
    const float* Bl = Wf + (int64_t)l * C * K;
    float* Cl = out + (int64_t)(l * l) * C;
    int rc;
    if (C == 64)
      rc = species_proj_fwd_c<4>(S, Al, N * g, ProjMap{K, 1, K}, Bl, Cl, ProjMap{C, g, (int64_t)ny * C}, st);
    else
      rc = gemm_nt_grouped(Al, N * g, K, K, 1, K, Bl, C, K, Cl, C, g, (int64_t)ny * C, 0, stream, 0);
    if (rc) return rc;
  }
  return ICTC_OK;
}

int ictc_species_message_bwd(int edge_lmax, int output_lmax, int C, int S, const float* xtab, const int64_t* species,
                             const float* sh, const float* h3, const float* t3, const float* W4,
                             const float* tp_weight, const float* mask, const int64_t* src, int64_t N, int64_t E,
                             const int32_t* dptr, const int32_t* dorder, const int32_t* dst_rows,
                             const int32_t* gate_rows, const float* grad, float* dsh, float* dr, void* ws,
                             int64_t ws_bytes, void* stream) {
  if (int rc = species_check(edge_lmax, output_lmax, C, S, N, E)) return rc;
  if (E == 0) return ICTC_OK;
  const int ny = (edge_lmax + 1) * (edge_lmax + 1), P = edge_lmax + 1;
  if (!xtab || !species || !W4 || !dptr || !ws || !sh || !h3 || !t3 || !src || !grad || !dsh || !dr)
    return fail(ICTC_ERR_ARGUMENT, "ictc_species_message_bwd: null operand (dsh and dr are both required)");
  const SpeciesLayout L = species_layout(ny, P, S, C, N);
  if (ws_bytes < L.total) return fail(ICTC_ERR_ARGUMENT, "ictc_species_message_bwd: workspace too small");
  hipStream_t st = (hipStream_t)stream;
  char* base = static_cast<char*>(ws);
  float *Z = (float*)(base + L.hz), *Wf = (float*)(base + L.wf), *Wb = (float*)(base + L.wb);
  if (int rc = species_weights_any(edge_lmax, xtab, S, C, W4, tp_weight, Wf, Wb, st)) return rc;
  const int64_t K = (int64_t)S * 64;
  if (N > 0) {
    // per degree l: Z_l[n, m, :] = go[n, l^2 + m, :] . Wb_l^T  (Wb_l = Wf_l^T, [S*64, C])
    for (int l = 0; l <= edge_lmax; ++l) {
      const int64_t g = 2 * l + 1;
      const float* Al = grad + (int64_t)(l * l) * C;
      const float* Bl = Wb + (int64_t)l * C * K;
      float* Cl = Z + N * (int64_t)(l * l) * K;
      int rc;
      if (C == 64)
        rc = species_proj_bwd_c<2>(S, Al, N * g, ProjMap{C, g, (int64_t)ny * C}, Bl, Cl, ProjMap{K, 1, K}, st);
      else
        rc = gemm_nt_grouped(Al, N * g, C, C, g, (int64_t)ny * C, Bl, K, C, Cl, K, 1, K, 0, stream, 0);
      if (rc) return rc;
    }
  }
  SpeciesArgs a{sh, h3, t3, mask, src, species, gate_rows, N, E, S, Csr{dptr, dorder, dst_rows}};
  switch (ny) {
    case 1: species_bwd_ny<1>(a, Z, dsh, dr, st); break;
    case 4: species_bwd_ny<4>(a, Z, dsh, dr, st); break;
    default: species_bwd_ny<9>(a, Z, dsh, dr, st); break;
  }
  return launch_status("ictc_species_message_bwd launch");
}

}  // extern "C"

