// Per-edge tensor product, CSR graph message and direction-harmonic kernels
// for gfx950 (CDNA4, wave64).
//
// Data layout in HBM (all FP32, row-major, "component-major, channel-minor"):
//   node / edge features  [rows, NX*C]   component k = l*l+m at k*C + c
//   harmonics             [E, NY]        NY = (LE+1)^2
//   gates                 [E, P*C]       path p at p*C + c
//   TP output             [rows, NO*C]   output slot k at k*C + c
// One wave owns one row (an edge for the edge TP, a node for the CSR message)
// and one group of 64 channels, lane l owning channel c = 64*group + l, so every feature,
// gate and output access is a fully coalesced 256-byte wave transaction and
// every per-edge scalar (indices, harmonics, mask) is wave-uniform.
//
// The graph message is deterministic and float-atomic free: the forward and
// the gate / harmonic adjoints run over the receiver-sorted CSR (one owner per
// output row); the feature adjoint runs over the source-sorted CSR.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "generated/ictc_tables.h"

namespace ictc {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlock = kWave * kWavesPerBlock;

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// DPP move within rows of 16 lanes (all rows and banks enabled).
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sums over the wave of v[0..N) (N <= 16) by reduce-scatter: a permlane32
// swap pairs component k with k+8 across the wave halves, a permlane16 swap
// pairs k with k+4 across rows, so row r ends up with partial sums of
// components 4r .. 4r+3 over 4 lanes each; four DPP row rotations (8, 4, 2, 1)
// finish each row sum.  About 3 VALU ops per component instead of a full wave
// reduction per component.  Lane 16r + k (k < 4) returns the total of
// component 4r + k (wave_sums_slot); the addition order is fixed.
template <int N>
__device__ __forceinline__ float wave_sums(const float* v) {
  static_assert(N >= 1 && N <= 16, "wave_sums covers up to 16 components");
  float w[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < N || k + 8 < N) {
      const float a = k < N ? v[k] : 0.f, b = k + 8 < N ? v[k + 8] : 0.f;
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
      w[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
      w[k] = 0.f;
    }
  }
  float u[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (k < N || k + 4 < N || k + 8 < N || k + 12 < N) {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[k]), __float_as_uint(w[k + 4]), false, false);
      u[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
      u[k] = 0.f;
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) u[k] += dpp_mov<0x128>(u[k]);   // row_ror:8
#pragma unroll
  for (int k = 0; k < 4; ++k) u[k] += dpp_mov<0x124>(u[k]);   // row_ror:4
#pragma unroll
  for (int k = 0; k < 4; ++k) u[k] += dpp_mov<0x122>(u[k]);   // row_ror:2
#pragma unroll
  for (int k = 0; k < 4; ++k) u[k] += dpp_mov<0x121>(u[k]);   // row_ror:1
  const int q = lane_id() & 3;
  return q == 0 ? u[0] : (q == 1 ? u[1] : (q == 2 ? u[2] : u[3]));
}

// Component whose total wave_sums returns in this lane, or -1.
__device__ __forceinline__ int wave_sums_slot() {
  const int l = lane_id();
  return (l & 15) < 4 ? 4 * (l >> 4) + (l & 15) : -1;
}

struct Operands {
  const float* x;       // features (edge rows for the edge TP, node rows for messages)
  const float* sh;      // [E, NY]
  const float* gates;   // [E, P*C]
  const float* weight;  // [P, C] or nullptr for unit coefficients
  const float* mask;    // [E] or nullptr
  int64_t rows;         // E (edge TP) or N (message)
  int64_t edges;
  int channels;
  // Gate row of each edge ([E], nullptr = the edge itself): the radial gates depend on the edge length
  // only, and an edge and its reverse have bitwise-equal lengths, so one row can serve both.
  const int32_t* grow = nullptr;
  // Gate-gradient outputs add to the rows already there (ictc_msg_bwd_accumulate) instead of overwriting them.
  int dg_acc = 0;
};

// Row of the gate (and gate-tangent) arrays that edge e reads.
__device__ __forceinline__ int64_t gate_row(const Operands& a, int64_t e) { return a.grow ? (int64_t)a.grow[e] : e; }

template <class T>
__device__ __forceinline__ void load_harmonics(const float* __restrict__ sh, int64_t e, float* y) {
  const float* p = sh + e * T::NY;
#pragma unroll
  for (int j = 0; j < T::NY; ++j) y[j] = p[j];
}

template <int N>
__device__ __forceinline__ void load_row(const float* __restrict__ base, int C, int c, float* v) {
  // wave-uniform row pointer stepped on the scalar unit + a 32-bit lane byte offset: the loads take
  // the SGPR-base form with no per-load 64-bit vector address arithmetic.  The empty asm keeps the
  // offset's zero extension next to the loads (hoisted out of a loop it hides the pattern).
  uint32_t off = (uint32_t)c * 4u;
  asm volatile("" : "+v"(off));
#pragma unroll
  for (int i = 0; i < N; ++i) {
    v[i] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + off);
    base += C;
  }
}

// load_row for a row read once: non-temporal loads, so that the streamed row does not displace
// the rows other waves gather again (the receiver cotangent rows of the source-owned adjoint).
template <int N>
__device__ __forceinline__ void load_row_stream(const float* __restrict__ base, int C, int c, float* v) {
  uint32_t off = (uint32_t)c * 4u;
  asm volatile("" : "+v"(off));
#pragma unroll
  for (int i = 0; i < N; ++i) {
    v[i] = __builtin_nontemporal_load(reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + off));
    base += C;
  }
}

template <int N>
__device__ __forceinline__ void zero_row(float* v) {
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = 0.f;
}

template <int N>
__device__ __forceinline__ void store_row(float* __restrict__ base, int C, int c, const float* v) {
  uint32_t off = (uint32_t)c * 4u;
  asm volatile("" : "+v"(off));
#pragma unroll
  for (int i = 0; i < N; ++i) {
    *reinterpret_cast<float*>(reinterpret_cast<char*>(base) + off) = v[i];
    base += C;
  }
}

// store_row of a gate-gradient row, or with a.dg_acc the sum of the row already there and v.
template <int N>
__device__ __forceinline__ void store_dg_row(const Operands& a, float* __restrict__ base, int C, int c, float* v) {
  if (a.dg_acc) {
    float o[N];
    load_row<N>(base, C, c, o);
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = o[i] + v[i];
  }
  store_row<N>(base, C, c, v);
}

// Gates of gate row `row` for channel c, times the per-path weight (if any) and `scale`.
// All P gate loads are issued before any use so they are in flight together;
// the optional weight is a separate uniform branch after them.
template <class T, bool STREAM = false>
__device__ __forceinline__ void load_gw(const Operands& a, int64_t row, int c, float scale, float* gw) {
  if (STREAM) load_row_stream<T::P>(a.gates + row * (int64_t)(T::P * a.channels), a.channels, c, gw);
  else load_row<T::P>(a.gates + row * (int64_t)(T::P * a.channels), a.channels, c, gw);
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

// ---------------------------------------------------------------------------
// Launch geometry.  A channel group is 64 consecutive channels, one per lane
// (c = 64 * group + lane); G = ceil(C / 64) groups, C <= 256.  Every kernel
// runs 4 rows per 256-thread block and takes the group from blockIdx.y.
// Kernels that reduce over channels (the harmonic gradient) write group 0's
// partial sum to the output and group g's to slab g-1 of a workspace; a
// second pass (launch_group_sum) adds the slabs in group order, so the result
// is deterministic and no block ever waits on another wave.
// Register budgets: the minimum waves per SIMD requested from the compiler
// drop for the wide degree triples so that their accumulators stay in VGPRs.
// ---------------------------------------------------------------------------
constexpr int kMaxGroups = 4;

// Minimum waves per SIMD requested for each (kernel, degree triple): the
// highest of 4, 3, 2, 1 at which the kernel compiles without register spills,
// found by tune_occupancy.py and recorded in ictc_occupancy.h.
enum KernelKind {
  kEdgeFwd, kEdgeBwd, kMsgFwd, kMsgBwdEdge, kMsgBwdX, kEdgeSecond, kMsgFwd2, kMsgBwdEdge2, kMsgBwdX2, kMsgBwdSrc
};
template <int K, int LI, int LE, int LO>
struct Occupancy {
#ifdef ICTC_OCCUPANCY_PROBE
  static constexpr int value = ICTC_OCCUPANCY_PROBE;
#else
  static constexpr int value = 4;
#endif
};

#ifndef ICTC_OCCUPANCY_PROBE
#include "ictc_occupancy.h"
#endif

struct RowGroup {
  int64_t row;
  int group;
};

// Workgroups are dispatched round-robin over the 8 XCDs (block b runs on XCD
// b % 8), each with its own L2.  The message kernels gather neighbour rows,
// and neighbouring rows have nearby indices, so hand each XCD a contiguous
// range of logical blocks: a bijection of [0, nb) that keeps the gathered
// rows of concurrently running blocks in one L2.
constexpr int kXcds = 8;
__device__ __forceinline__ int64_t xcd_block(int64_t b, int64_t nb) {
  const int64_t q = nb / kXcds, r = nb % kXcds, x = b % kXcds, i = b / kXcds;
  return x < r ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
}

__device__ __forceinline__ RowGroup row_group_y() {
  return {(int64_t)blockIdx.x * kWavesPerBlock + wave_id(), (int)blockIdx.y};
}

// Row-parallel kernels over graph rows (the CSR message): XCD-local row ranges.
__device__ __forceinline__ RowGroup row_group_y_xcd() {
  return {xcd_block(blockIdx.x, gridDim.x) * kWavesPerBlock + wave_id(), (int)blockIdx.y};
}

// Harmonic-gradient target of a channel group: group 0 writes the output,
// group g > 0 slab g-1 of the workspace ([G-1][rows][NY]).
__device__ __forceinline__ float* group_target(float* dsh, float* part, int group, int64_t rows, int ny) {
  return (dsh && group > 0) ? part + (int64_t)(group - 1) * rows * ny : dsh;
}

// ---------------------------------------------------------------------------
// Edge TP: one wave per (edge, channel group).
// ---------------------------------------------------------------------------
template <class T>
__global__ __launch_bounds__(kBlock, (Occupancy<kEdgeFwd, T::LI, T::LE, T::LO>::value)) void edge_fwd_kernel(
    Operands a, float* __restrict__ out) {
  const RowGroup rg = row_group_y();
  const int64_t e = rg.row;
  if (e >= a.rows) return;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  if (c >= C) return;
  float y[T::NY], xv[T::NX], gw[T::P], o[T::NO];
  load_harmonics<T>(a.sh, e, y);
  load_row<T::NX>(a.x + e * (int64_t)(T::NX * C), C, c, xv);
  load_gw<T>(a, gate_row(a, e), c, 1.f, gw);
#pragma unroll
  for (int k = 0; k < T::NO; ++k) o[k] = 0.f;
  T::fwd(xv, y, gw, o);
  store_row<T::NO>(out + e * (int64_t)(T::NO * C), C, c, o);
}

template <class T>
__global__ __launch_bounds__(kBlock, (Occupancy<kEdgeBwd, T::LI, T::LE, T::LO>::value)) void edge_bwd_kernel(
    Operands a, const float* __restrict__ grad, float* __restrict__ dx, float* __restrict__ dsh,
    float* __restrict__ dsh_part, float* __restrict__ dgates) {
  const RowGroup rg = row_group_y();
  const int64_t e = rg.row;
  if (e >= a.rows) return;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  const bool active = c < C;
  float y[T::NY], dyv[T::NY];
  load_harmonics<T>(a.sh, e, y);
#pragma unroll
  for (int j = 0; j < T::NY; ++j) dyv[j] = 0.f;
  if (active) {
    float xv[T::NX], gw[T::P], go[T::NO];
    load_row<T::NX>(a.x + e * (int64_t)(T::NX * C), C, c, xv);
    load_row<T::NO>(grad + e * (int64_t)(T::NO * C), C, c, go);
    load_gw<T>(a, gate_row(a, e), c, 1.f, gw);
    if (dx) {
      float d[T::NX];
#pragma unroll
      for (int i = 0; i < T::NX; ++i) d[i] = 0.f;
      T::dx_v(y, gw, go, d);
      store_row<T::NX>(dx + e * (int64_t)(T::NX * C), C, c, d);
    }
    float d[T::P];
    if (dsh && dgates) T::dydg(xv, y, gw, go, dyv, d);
    else if (dsh) T::dy(xv, gw, go, dyv);
    else if (dgates) T::dg(xv, y, go, d);
    if (dgates) {
      if (a.weight) {
#pragma unroll
        for (int p = 0; p < T::P; ++p) d[p] *= a.weight[p * C + c];
      }
      store_row<T::P>(dgates + e * (int64_t)(T::P * C), C, c, d);
    }
  }
  if (!dsh) return;
  float* out = group_target(dsh, dsh_part, rg.group, a.rows, T::NY);
  const float mine = wave_sums<T::NY>(dyv);
  const int j = wave_sums_slot();
  if (j >= 0 && j < T::NY) out[e * T::NY + j] = mine;
}

// ---------------------------------------------------------------------------
// CSR graph message.  ptr/order describe the receiver-sorted (dst) CSR: the
// edges into node n are order[ptr[n] .. ptr[n+1]) (order == nullptr: edges are
// already sorted and order is the identity).
// ---------------------------------------------------------------------------
struct Csr {
  const int32_t* ptr;    // [N+2]: ptr[N]..ptr[N+1] holds out-of-range edges
  const int32_t* order;  // [E] or nullptr
  const int32_t* rows;   // [N] row traversal order (a permutation of 0..N-1) or nullptr for 0..N-1
};

// Row visited by logical row slot `slot`.  A spatially ordered traversal keeps
// the neighbour rows gathered by concurrently running waves (and by the blocks
// of one XCD) in a compact region, so they hit in L2.  Slots at or past `rows`
// (the out-of-range tail slot) map to themselves; an entry outside [0, rows)
// yields -1 and its wave does nothing.
__device__ __forceinline__ int64_t visit_row(const Csr& csr, int64_t slot, int64_t rows) {
  if (!csr.rows || slot >= rows) return slot;
  const int64_t n = csr.rows[slot];
  return n >= 0 && n < rows ? n : -1;
}

// Part `part` of `parts` equal shares of row n's CSR segment (receiver-owned
// kernels whose outputs are per edge split long rows over several waves when
// the graph has too few rows to fill the GPU).  False when the share is empty.
__device__ __forceinline__ bool row_part(const Csr& csr, int64_t n, int part, int parts, int32_t& beg, int32_t& end) {
  const int32_t b = csr.ptr[n], e = csr.ptr[n + 1];
  const int32_t per = (e - b + parts - 1) / parts;
  beg = b + part * per;
  end = min(e, beg + per);
  return beg < end;
}

// Edge metadata of a chunk of up to 64 consecutive CSR positions, staged one
// edge per lane with coalesced loads; the edge loop then reads it with
// readlane (wave-uniform SGPR values, no memory latency inside the loop).
template <class T>
struct Chunk {
  int32_t e;        // edge id of this lane's position
  int32_t row;      // its gate row (staged with the chunk: a per-edge index load inside the edge loop
                    // would be a vector load whose wait also drains the rows already in flight)
  int32_t peer;     // src (receiver-sorted CSR) or dst (source-sorted CSR); 0 when out of range
  float m;          // mask, 0 when the peer is out of range or the lane is past the chunk
  float y[T::NY];   // harmonics of this lane's edge
};

template <class T>
__device__ __forceinline__ void stage_chunk(const Operands& a, const int64_t* __restrict__ peer_ids,
                                            const int32_t* __restrict__ order, int32_t pos, int32_t count,
                                            Chunk<T>& ch) {
  const int l = lane_id();
  ch.e = 0;
  ch.row = 0;
  ch.peer = 0;
  ch.m = 0.f;
#pragma unroll
  for (int j = 0; j < T::NY; ++j) ch.y[j] = 0.f;
  if (l < count) {
    const int32_t e = order ? order[pos + l] : pos + l;
    const int64_t p = peer_ids[e];
    const bool ok = p >= 0 && p < a.rows;
    ch.e = e;
    ch.row = a.grow ? a.grow[e] : e;
    ch.peer = ok ? (int32_t)p : 0;
    ch.m = ok ? (a.mask ? a.mask[e] : 1.f) : 0.f;
#pragma unroll
    for (int j = 0; j < T::NY; ++j) ch.y[j] = a.sh[(int64_t)e * T::NY + j];
  }
  // The chunk's loads complete here, once per chunk.  Left to their first use inside the edge loop,
  // the wait for them would recur at every edge (some paths through the loop body do not use them)
  // and would also drain the next edge's rows already in flight.
  asm volatile("" : "+v"(ch.e), "+v"(ch.row), "+v"(ch.peer), "+v"(ch.m));
#pragma unroll
  for (int j = 0; j < T::NY; ++j) asm volatile("" : "+v"(ch.y[j]));
}

__device__ __forceinline__ int32_t lane_i(int32_t v, int i) { return __builtin_amdgcn_readlane(v, i); }
__device__ __forceinline__ float lane_f(float v, int i) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}

// Compile-time flag for generic lambdas: the edge loops below are compiled once with and once without
// the per-path weight, chosen once per wave.  A weight branch inside the loop loads the weights per
// edge, and the wait where its paths merge drains the next edge's rows already in flight.
template <bool B>
struct Flag {
  static constexpr bool value = B;
};

// The forward keeps two edges' feature and gate rows in flight (loads of edge i + 1 issued before
// edge i's products) where the per-lane state stays small, NX + NY + P + NO <= 64 values with input
// degree <= 2: every such triple compiles without spills at the table's occupancy (Tp<2,2,2>: 128
// VGPRs at 4 waves per SIMD, cfg4 layer 1 3.34 -> 3.13 ms), while (3,3,1), (3,1,3), (3,2,2) and the
// degree-3 triples above spill.
template <class T>
constexpr bool msg_fwd_pipelined() {
  return T::LI <= 2 && T::NX + T::NY + T::P + T::NO <= 64;
}

template <class T>
__global__ __launch_bounds__(kBlock, (Occupancy<kMsgFwd, T::LI, T::LE, T::LO>::value)) void msg_fwd_kernel(
    Operands a, const int64_t* __restrict__ src, Csr csr, float* __restrict__ out) {
  const RowGroup rg = row_group_y_xcd();
  if (rg.row >= a.rows) return;
  const int64_t n = visit_row(csr, rg.row, a.rows);
  if (n < 0) return;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  const bool active = c < C;
  float o[T::NO];
#pragma unroll
  for (int k = 0; k < T::NO; ++k) o[k] = 0.f;
  const int32_t beg = csr.ptr[n], end = csr.ptr[n + 1];
  if constexpr (msg_fwd_pipelined<T>()) {
    auto run = [&](auto weighted) {
    constexpr bool W = decltype(weighted)::value;
    for (int32_t pos = beg; pos < end; pos += kWave) {
      const int32_t count = min(end - pos, kWave);
      Chunk<T> ch;
      stage_chunk<T>(a, src, csr.order, pos, count, ch);
      float x0[T::NX], g0[T::P], x1[T::NX], g1[T::P];
      auto fetch = [&](int i, float* xv, float* gr) {
        const int64_t s = lane_i(ch.peer, i), row = lane_i(ch.row, i);
        load_row<T::NX>(a.x + s * (int64_t)(T::NX * C), C, c, xv);
        load_row<T::P>(a.gates + row * (int64_t)(T::P * C), C, c, gr);
      };
      auto consume = [&](int i, const float* xv, const float* gr) {
        const float m = lane_f(ch.m, i);
        float y[T::NY], gw[T::P];
#pragma unroll
        for (int j = 0; j < T::NY; ++j) y[j] = lane_f(ch.y[j], i);
#pragma unroll
        for (int p = 0; p < T::P; ++p) gw[p] = gr[p];
        if constexpr (W) {
#pragma unroll
          for (int p = 0; p < T::P; ++p) gw[p] *= a.weight[p * C + c];
        }
#pragma unroll
        for (int p = 0; p < T::P; ++p) gw[p] *= m;
        T::fwd_b(xv, y, gw, o);
      };
      if (!active) continue;
      fetch(0, x0, g0);
      for (int i = 0; i < count; i += 2) {
        if (i + 1 < count) fetch(i + 1, x1, g1);
        consume(i, x0, g0);
        if (i + 1 >= count) break;
        if (i + 2 < count) fetch(i + 2, x0, g0);
        consume(i + 1, x1, g1);
      }
    }
    };
    if (a.weight) run(Flag<true>{});
    else run(Flag<false>{});
    if (active) store_row<T::NO>(out + n * (int64_t)(T::NO * C), C, c, o);
    return;
  }
  for (int32_t pos = beg; pos < end; pos += kWave) {
    const int32_t count = min(end - pos, kWave);
    Chunk<T> ch;
    stage_chunk<T>(a, src, csr.order, pos, count, ch);
    for (int i = 0; i < count; ++i) {
      const int64_t e = lane_i(ch.e, i);
      const int64_t s = lane_i(ch.peer, i);
      const float m = lane_f(ch.m, i);
      float y[T::NY];
#pragma unroll
      for (int j = 0; j < T::NY; ++j) y[j] = lane_f(ch.y[j], i);
      if (active) {
        float xv[T::NX], gw[T::P];
        load_row<T::NX>(a.x + s * (int64_t)(T::NX * C), C, c, xv);
        load_gw<T>(a, lane_i(ch.row, i), c, m, gw);
        T::fwd_b(xv, y, gw, o);
      }
    }
  }
  if (active) store_row<T::NO>(out + n * (int64_t)(T::NO * C), C, c, o);
}

// Gate-tangent mode of the first adjoint: per edge, the harmonic gradient (when
// dsh_g) and dr = sum over paths and channels of dgates * gdot, reduced over the
// wave's 64 channels in one wave_sums where the components fit.
template <int NY>
__device__ __forceinline__ void store_dsh_dr(float* __restrict__ dsh_g, float* __restrict__ dr_g, int64_t e,
                                             const float* dyv, float dgt) {
  const int j = wave_sums_slot();
  if constexpr (NY + 1 <= 16) {
    if (dsh_g) {
      float v[NY + 1];
#pragma unroll
      for (int k = 0; k < NY; ++k) v[k] = dyv[k];
      v[NY] = dgt;
      const float t = wave_sums<NY + 1>(v);
      if (j >= 0 && j < NY) dsh_g[e * NY + j] = t;
      else if (j == NY) dr_g[e] = t;
      return;
    }
  } else {
    if (dsh_g) {
      const float t = wave_sums<NY>(dyv);
      if (j >= 0 && j < NY) dsh_g[e * NY + j] = t;
    }
  }
  const float t = wave_sums<1>(&dgt);
  if (j == 0) dr_g[e] = t;
}

// This lane's share of the gate-tangent dot: sum_p dg[p] w[p] gdot[p] (dg unweighted, unmasked).
// W: 1 / 0 = with / without the per-path weight, known at compile time; -1 = tested at run time.
template <class T, int W = -1>
__device__ __forceinline__ float gate_tangent_dot(const Operands& a, const float* __restrict__ gdot, int64_t e, int c,
                                                  const float* gt, const float* dg) {
  float t = 0.f;
  if (W == 1 || (W < 0 && a.weight)) {
#pragma unroll
    for (int p = 0; p < T::P; ++p) t += dg[p] * a.weight[p * a.channels + c] * gt[p];
  } else {
#pragma unroll
    for (int p = 0; p < T::P; ++p) t += dg[p] * gt[p];
  }
  return t;
}

// Receiver-owned adjoint: per-edge gate and harmonic gradients.  Waves of
// row `rows` own the out-of-range tail segment ptr[rows]..ptr[rows+1] and
// write zero gradients for it (mask 0, zero cotangent).
// Waves per SIMD of the receiver-owned adjoint: the gate-tangent form holds the
// tangent row besides the gate row and the full dy/dg contraction, so it asks
// for one wave per SIMD fewer than the table (at the table's level up to 113
// VGPRs spill, e.g. Tp<2,3,3>; one fewer leaves at most 5).
template <class T, bool TAN>
constexpr int edge_adjoint_waves() {
  constexpr int w = Occupancy<kMsgBwdEdge, T::LI, T::LE, T::LO>::value;
  return (TAN && w > 1) ? w - 1 : w;
}

// With TAN, gdot [E, P*C] (d gates / dr) replaces the gate gradient output:
// dr[e] = sum dgates * gdot is written instead (group g > 0: slab g-1 of dr_part).
template <class T, bool TAN>
__global__ __launch_bounds__(kBlock, (edge_adjoint_waves<T, TAN>())) void msg_bwd_edge_kernel(
    Operands a, const int64_t* __restrict__ src, Csr csr, const float* __restrict__ grad, float* __restrict__ dsh,
    float* __restrict__ dsh_part, float* __restrict__ dgates, int parts, const float* __restrict__ gdot,
    float* __restrict__ dr, float* __restrict__ dr_part) {
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
  float* dr_g = rg.group > 0 ? dr_part + (int64_t)(rg.group - 1) * a.edges : dr;
  float go[T::NO];
  if (active && !tail) load_row<T::NO>(grad + n * (int64_t)(T::NO * C), C, c, go);
  else {
#pragma unroll
    for (int k = 0; k < T::NO; ++k) go[k] = 0.f;
  }
  for (int32_t pos = beg; pos < end; pos += kWave) {
    const int32_t count = min(end - pos, kWave);
    Chunk<T> ch;
    stage_chunk<T>(a, src, csr.order, pos, count, ch);
    for (int i = 0; i < count; ++i) {
      const int64_t e = lane_i(ch.e, i);
      const int64_t s = lane_i(ch.peer, i);
      const float m = lane_f(ch.m, i);
      float y[T::NY], dyv[T::NY];
#pragma unroll
      for (int j = 0; j < T::NY; ++j) {
        y[j] = lane_f(ch.y[j], i);
        dyv[j] = 0.f;
      }
      float dgt = 0.f;
      if (TAN && active) {
        float xv[T::NX], gw[T::P], gt[T::P], d[T::P];
        load_row<T::NX>(a.x + s * (int64_t)(T::NX * C), C, c, xv);
        load_gw<T>(a, lane_i(ch.row, i), c, m, gw);
        load_row<T::P>(gdot + lane_i(ch.row, i) * (int64_t)(T::P * C), C, c, gt);
        if (dsh) T::dydg(xv, y, gw, go, dyv, d);
        else T::dg(xv, y, go, d);
        dgt = m * gate_tangent_dot<T>(a, gdot, e, c, gt, d);
      }
      if (TAN) {
        store_dsh_dr<T::NY>(dsh_g, dr_g, e, dyv, dgt);
        continue;
      }
      if (active) {
        float xv[T::NX], gw[T::P];
        load_row<T::NX>(a.x + s * (int64_t)(T::NX * C), C, c, xv);
        load_gw<T>(a, lane_i(ch.row, i), c, m, gw);
        float d[T::P];
        if (dsh && dgates) T::dydg(xv, y, gw, go, dyv, d);
        else if (dsh) T::dy(xv, gw, go, dyv);
        else if (dgates) T::dg(xv, y, go, d);
        if (dgates) {
#pragma unroll
          for (int p = 0; p < T::P; ++p) d[p] *= m;
          if (a.weight) {
#pragma unroll
            for (int p = 0; p < T::P; ++p) d[p] *= a.weight[p * C + c];
          }
          store_dg_row<T::P>(a, dgates + e * (int64_t)(T::P * C), C, c, d);
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

// Source-owned adjoint: node feature gradient over the source-sorted CSR.
template <class T>
__global__ __launch_bounds__(kBlock, (Occupancy<kMsgBwdX, T::LI, T::LE, T::LO>::value)) void msg_bwd_x_kernel(
    Operands a, const int64_t* __restrict__ dst, Csr scsr, const float* __restrict__ grad, float* __restrict__ dx) {
  const RowGroup rg = row_group_y_xcd();
  if (rg.row >= a.rows) return;
  const int64_t n = visit_row(scsr, rg.row, a.rows);
  if (n < 0) return;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  const bool active = c < C;
  float d[T::NX];
#pragma unroll
  for (int i = 0; i < T::NX; ++i) d[i] = 0.f;
  const int32_t beg = scsr.ptr[n], end = scsr.ptr[n + 1];
  // An out-of-range receiver contributes zero (mask 0, row 0 read).
  for (int32_t pos = beg; pos < end; pos += kWave) {
    const int32_t count = min(end - pos, kWave);
    Chunk<T> ch;
    stage_chunk<T>(a, dst, scsr.order, pos, count, ch);
    for (int i = 0; i < count; ++i) {
      const int64_t e = lane_i(ch.e, i);
      const int64_t r = lane_i(ch.peer, i);
      const float m = lane_f(ch.m, i);
      float y[T::NY];
#pragma unroll
      for (int j = 0; j < T::NY; ++j) y[j] = lane_f(ch.y[j], i);
      if (active) {
        float go[T::NO], gw[T::P];
        load_row<T::NO>(grad + r * (int64_t)(T::NO * C), C, c, go);
        load_gw<T>(a, lane_i(ch.row, i), c, m, gw);
        T::dx_v(y, gw, go, d);
      }
    }
  }
  if (active) store_row<T::NX>(dx + n * (int64_t)(T::NX * C), C, c, d);
}

// Source-owned complete adjoint: the feature gradient of each source row and,
// on the way, the gate and harmonic gradients of its out-edges (per-edge
// outputs, so any owner may write them).  One pass reads the gate stream once
// and gathers only the receiver cotangent rows the feature gradient needs;
// the sender's own features are loaded once per row.  Row slot `rows` covers
// the out-of-range tail segment of the source CSR and writes zero gate and
// harmonic gradients for it (no feature row).
// Waves per SIMD of the source-owned adjoint.  The gate-tangent form streams the
// tangent rows as well; where the table allows 3 it runs better at 2, with fewer
// receiver rows in flight (cfg4 layer-1 shape: 8.62 ms at 2, 9.6 ms at 3 with 13
// spilled VGPRs).
template <class T, bool TAN>
constexpr int src_adjoint_waves() {
  return (TAN && Occupancy<kMsgBwdSrc, T::LI, T::LE, T::LO>::value == 3)
             ? 2
             : Occupancy<kMsgBwdSrc, T::LI, T::LE, T::LO>::value;
}

// The gate-tangent form keeps two edges' cotangent, gate and gate-tangent rows in flight where it runs
// at 2 waves per SIMD (up to 256 VGPRs) and the second set of rows is at most 57 values per lane
// (NO + 2 P): at 60, the (1,3,3) and (3,1,3) triples spill.
template <class T, bool TAN>
constexpr bool src_adjoint_pipelined() {
  return TAN && src_adjoint_waves<T, TAN>() == 2 && T::NO + 2 * T::P <= 57;
}

// TAN: as in msg_bwd_edge_kernel, dr from gdot in place of the gate gradient.
// W: the per-path weight a.weight is set (chosen at launch).  One loop per kernel: with both forms in one
// kernel they share one register allocation, and the gate-tangent form of Tp<2,2,2> spilled 15 VGPRs
// (226 without a spill for the unweighted form alone).
template <class T, bool TAN, bool W = false>
__global__ __launch_bounds__(kBlock, (src_adjoint_waves<T, TAN>())) void msg_bwd_src_kernel(
    Operands a, const int64_t* __restrict__ dst, Csr scsr, const float* __restrict__ grad, float* __restrict__ dx,
    float* __restrict__ dsh, float* __restrict__ dsh_part, float* __restrict__ dgates, const float* __restrict__ gdot,
    float* __restrict__ dr, float* __restrict__ dr_part) {
  const RowGroup rg = row_group_y_xcd();
  if (rg.row > a.rows) return;
  const int64_t n = visit_row(scsr, rg.row, a.rows);
  if (n < 0) return;
  const bool tail = n == a.rows;
  const int C = a.channels, c = 64 * rg.group + lane_id();
  const bool active = c < C;
  float* dsh_g = group_target(dsh, dsh_part, rg.group, a.edges, T::NY);
  float* dr_g = rg.group > 0 ? dr_part + (int64_t)(rg.group - 1) * a.edges : dr;
  float xv[T::NX], d[T::NX];
  if (active && !tail) load_row<T::NX>(a.x + n * (int64_t)(T::NX * C), C, c, xv);
  else zero_row<T::NX>(xv);
  zero_row<T::NX>(d);
  const int32_t beg = scsr.ptr[n], end = scsr.ptr[n + 1];
  if constexpr (src_adjoint_pipelined<T, TAN>()) {
    // Two edges in flight: the cotangent, gate and gate-tangent rows of edge i + 1 load while edge i
    // computes (2 waves per SIMD leave room for the second set of rows).  Per-edge arithmetic is that
    // of the unpipelined form, operand for operand.
    auto run = [&](auto weighted) {
    for (int32_t pos = beg; pos < end; pos += kWave) {
      const int32_t count = min(end - pos, kWave);
      Chunk<T> ch;
      stage_chunk<T>(a, dst, scsr.order, pos, count, ch);
      float go0[T::NO], gr0[T::P], gt0[T::P], go1[T::NO], gr1[T::P], gt1[T::P];
      auto fetch = [&](int i, float* go, float* gr, float* gt) {
        const int64_t r = lane_i(ch.peer, i), row = lane_i(ch.row, i);
        load_row<T::NO>(grad + r * (int64_t)(T::NO * C), C, c, go);
        load_row_stream<T::P>(a.gates + row * (int64_t)(T::P * C), C, c, gr);
        load_row_stream<T::P>(gdot + row * (int64_t)(T::P * C), C, c, gt);
      };
      auto consume = [&](int i, const float* go, const float* gr, const float* gt) {
        const int64_t e = lane_i(ch.e, i);
        const float m = lane_f(ch.m, i);
        float y[T::NY], dyv[T::NY], gw[T::P], dg[T::P];
#pragma unroll
        for (int j = 0; j < T::NY; ++j) {
          y[j] = lane_f(ch.y[j], i);
          dyv[j] = 0.f;
        }
        float dgt = 0.f;
        if (active) {
#pragma unroll
          for (int p = 0; p < T::P; ++p) gw[p] = gr[p];
          if constexpr (W) {
#pragma unroll
            for (int p = 0; p < T::P; ++p) gw[p] *= a.weight[p * C + c];
          }
#pragma unroll
          for (int p = 0; p < T::P; ++p) gw[p] *= m;
          if (dsh) {
            T::dxdydg(xv, y, gw, go, d, dyv, dg);   // (the tail row's d is never stored)
          } else {
            if (!tail) T::dx_v(y, gw, go, d);
            T::dg(xv, y, go, dg);
          }
          dgt = m * gate_tangent_dot<T, W ? 1 : 0>(a, gdot, e, c, gt, dg);
        }
        store_dsh_dr<T::NY>(dsh_g, dr_g, e, dyv, dgt);
      };
      if (active) fetch(0, go0, gr0, gt0);
      for (int i = 0; i < count; i += 2) {
        if (active && i + 1 < count) fetch(i + 1, go1, gr1, gt1);
        consume(i, go0, gr0, gt0);
        if (i + 1 >= count) break;
        if (active && i + 2 < count) fetch(i + 2, go0, gr0, gt0);
        consume(i + 1, go1, gr1, gt1);
      }
    }
    };
    run(Flag<W>{});
    if (active && !tail && dx) store_row<T::NX>(dx + n * (int64_t)(T::NX * C), C, c, d);
    return;
  }
  // An out-of-range receiver contributes zero (mask 0, row 0 read).
  for (int32_t pos = beg; pos < end; pos += kWave) {
    const int32_t count = min(end - pos, kWave);
    Chunk<T> ch;
    stage_chunk<T>(a, dst, scsr.order, pos, count, ch);
    for (int i = 0; i < count; ++i) {
      const int64_t e = lane_i(ch.e, i);
      const int64_t r = lane_i(ch.peer, i);
      const float m = lane_f(ch.m, i);
      float y[T::NY], dyv[T::NY];
#pragma unroll
      for (int j = 0; j < T::NY; ++j) {
        y[j] = lane_f(ch.y[j], i);
        dyv[j] = 0.f;
      }
      float dgt = 0.f;
      if (TAN && active) {
        float go[T::NO], gw[T::P], gt[T::P], dg[T::P];
        load_row<T::NO>(grad + r * (int64_t)(T::NO * C), C, c, go);
        load_gw<T, true>(a, lane_i(ch.row, i), c, m, gw);
        load_row_stream<T::P>(gdot + lane_i(ch.row, i) * (int64_t)(T::P * C), C, c, gt);
        if (!tail) T::dx_v(y, gw, go, d);
        if (dsh) T::dydg(xv, y, gw, go, dyv, dg);
        else T::dg(xv, y, go, dg);
        dgt = m * gate_tangent_dot<T>(a, gdot, e, c, gt, dg);
      }
      if (TAN) {
        store_dsh_dr<T::NY>(dsh_g, dr_g, e, dyv, dgt);
        continue;
      }
      if (active) {
        float go[T::NO], gw[T::P], dg[T::P];
        load_row<T::NO>(grad + r * (int64_t)(T::NO * C), C, c, go);
        load_gw<T>(a, lane_i(ch.row, i), c, m, gw);
        if (!tail) T::dx_v(y, gw, go, d);
        if (dsh && dgates) T::dydg(xv, y, gw, go, dyv, dg);
        else if (dsh) T::dy(xv, gw, go, dyv);
        else if (dgates) T::dg(xv, y, go, dg);
        if (dgates) {
#pragma unroll
          for (int p = 0; p < T::P; ++p) dg[p] *= m;
          if (a.weight) {
#pragma unroll
            for (int p = 0; p < T::P; ++p) dg[p] *= a.weight[p * C + c];
          }
          store_dg_row<T::P>(a, dgates + e * (int64_t)(T::P * C), C, c, dg);
        }
      }
      if (dsh) {
        const float v = wave_sums<T::NY>(dyv);
        const int j = wave_sums_slot();
        if (j >= 0 && j < T::NY) dsh_g[e * T::NY + j] = v;
      }
    }
  }
  if (active && !tail && dx) store_row<T::NX>(dx + n * (int64_t)(T::NX * C), C, c, d);
}

// ---------------------------------------------------------------------------
// Direction harmonics: one thread per edge.
// ---------------------------------------------------------------------------
template <int L>
__global__ __launch_bounds__(256) void sh_fwd_kernel(const float* __restrict__ n, int64_t E, float* __restrict__ Y) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float v[Sh<L>::N];
  Sh<L>::fwd(n[3 * e], n[3 * e + 1], n[3 * e + 2], v);
#pragma unroll
  for (int k = 0; k < Sh<L>::N; ++k) Y[e * Sh<L>::N + k] = v[k];
}

template <int L>
__global__ __launch_bounds__(256) void sh_bwd_kernel(const float* __restrict__ n, const float* __restrict__ gY,
                                                     int64_t E, float* __restrict__ gn) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float g[Sh<L>::N];
#pragma unroll
  for (int k = 0; k < Sh<L>::N; ++k) g[k] = gY[e * Sh<L>::N + k];
  float gx, gy, gz;
  Sh<L>::bwd(n[3 * e], n[3 * e + 1], n[3 * e + 2], g, gx, gy, gz);
  gn[3 * e] = gx;
  gn[3 * e + 1] = gy;
  gn[3 * e + 2] = gz;
}

template <int L>
__global__ __launch_bounds__(256) void sh_jvp_kernel(const float* __restrict__ n, const float* __restrict__ hn,
                                                     int64_t E, float* __restrict__ dY) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float v[Sh<L>::N];
  Sh<L>::jvp(n[3 * e], n[3 * e + 1], n[3 * e + 2], hn[3 * e], hn[3 * e + 1], hn[3 * e + 2], v);
#pragma unroll
  for (int k = 0; k < Sh<L>::N; ++k) dY[e * Sh<L>::N + k] = v[k];
}

template <int L>
__global__ __launch_bounds__(256) void sh_hvp_kernel(const float* __restrict__ n, const float* __restrict__ gY,
                                                     const float* __restrict__ hn, int64_t E, float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  float g[Sh<L>::N];
#pragma unroll
  for (int k = 0; k < Sh<L>::N; ++k) g[k] = gY[e * Sh<L>::N + k];
  float ox, oy, oz;
  Sh<L>::hvp(n[3 * e], n[3 * e + 1], n[3 * e + 2], g, hn[3 * e], hn[3 * e + 1], hn[3 * e + 2], ox, oy, oz);
  out[3 * e] = ox;
  out[3 * e + 1] = oy;
  out[3 * e + 2] = oz;
}

}  // namespace ictc
