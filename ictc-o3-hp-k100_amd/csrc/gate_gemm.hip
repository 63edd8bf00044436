// Gate projection of the radial MLP on bf16 MFMA with a three-way operand split:
//   gates[E, M] = h[E, 64] . W^T,  W [M, 64] (nn.Linear layout)
// (the last Linear of `fc`, mace_ictc/models/mace/layers.py:826-835; the
// reference runs it as a library GEMM, streamed_gate_message.py:51-57).
//
// FP32 accuracy from bf16 MFMA: each operand is written exactly as
// x = hi + mid + lo + r with hi, mid, lo bf16 (round-to-nearest-even at each
// level) and |r| <= 2^-27 |x|.  The product keeps the six terms whose size is
// at least 2^-24 of hi*hi (lo*hi, hi*lo, mid*mid, mid*hi, hi*mid, hi*hi,
// accumulated smallest first in FP32 across both k-steps); the dropped terms are below 2^-25
// relative, under FP32 rounding.  bf16 has FP32's exponent range, so there is
// no overflow or scaling concern.  Six v_mfma_f32_16x16x32_bf16 (16 cycles
// each) replace eight v_mfma_f32_16x16x4_f32 (32 cycles each) per 16x16x32
// block, which makes the projection HBM-bound (it writes E * M floats).
//
// Tiling: a block owns 256 edges, split from HBM into LDS once; its 8 waves
// take 64-row slices of W in turn.  A wave holds its slice pre-split in
// registers (A operand: 4 row blocks x 2 k-steps x 3 parts) and streams the
// pre-split 16-edge tiles of h from LDS (B operand), so every gate is produced
// by one wave and stored as a 16-byte vector per lane.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/ictc_mi355x.h"
#include "split_bf16.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kK = 64;           // hidden width (reduction length)
constexpr int kEdgesPerBlock = 256;
constexpr int kTiles = kEdgesPerBlock / 16;


__device__ __forceinline__ v4f mfma(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void load8(const float* __restrict__ p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

// The block's 16-edge tiles of h, split once into bf16 parts in the B operand
// layout ([tile][k-step][hi, mid, lo][lane]); every slice reads them from LDS.
struct HTiles {
  bf16x8 b[kTiles][2][3][64];
};

// The tiles [t0, t1) of one 64-row slice.  The NRB row blocks are independent
// accumulator chains, interleaved so that no MFMA waits on its predecessor.
template <int NRB>
__device__ __forceinline__ void slice_tiles(const Split (&A)[4][2], const HTiles& ht, int t0, int t1, int64_t e_base,
                                            int64_t E, int M, int s, float* __restrict__ out) {
  const int l = threadIdx.x & 63, i = l & 15, g = l >> 4;
  for (int t = t0; t < t1; ++t) {
    const int64_t e = e_base + 16 * t + i;
    Split B0, B1;
    B0.hi = ht.b[t][0][0][l], B0.mid = ht.b[t][0][1][l], B0.lo = ht.b[t][0][2][l];
    B1.hi = ht.b[t][1][0][l], B1.mid = ht.b[t][1][1][l], B1.lo = ht.b[t][1][2][l];
    v4f acc[NRB];
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) acc[rb] = v4f{0.f, 0.f, 0.f, 0.f};
#define ICTC_STEP(PA, PB, KS, BB) \
  _Pragma("unroll") for (int rb = 0; rb < NRB; ++rb) acc[rb] = mfma(A[rb][KS].PA, BB.PB, acc[rb]);
    ICTC_STEP(lo, hi, 0, B0) ICTC_STEP(hi, lo, 0, B0) ICTC_STEP(mid, mid, 0, B0)
    ICTC_STEP(lo, hi, 1, B1) ICTC_STEP(hi, lo, 1, B1) ICTC_STEP(mid, mid, 1, B1)
    ICTC_STEP(mid, hi, 0, B0) ICTC_STEP(hi, mid, 0, B0) ICTC_STEP(mid, hi, 1, B1)
    ICTC_STEP(hi, mid, 1, B1) ICTC_STEP(hi, hi, 0, B0) ICTC_STEP(hi, hi, 1, B1)
#undef ICTC_STEP
    if (e < E) {
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) *reinterpret_cast<v4f*>(out + e * M + 64 * s + 16 * rb + 4 * g) = acc[rb];
    }
  }
}

// MFMA operand layout (both operands use the same k order, which is all the
// instruction requires): lane l holds row/column l % 16 and k = 32*ks + 8*(l/16) + e.
// D: lane l holds column l % 16 (an edge) and rows 4*(l/16) + r (gate outputs).
// The block's 256 hidden rows are split into LDS once (each slice used to
// split them again), so the gate stream cannot evict them between the slices
// that reuse them.  With fewer slices than waves, the waves of a slice share
// its tiles (a power-of-two number of waves per slice).
constexpr int kNtWaves = 8;
__global__ __launch_bounds__(64 * kNtWaves, 1) void gate_gemm_nt_kernel(const float* __restrict__ h, int64_t E,
                                                                         const float* __restrict__ W, int M,
                                                                         float* __restrict__ out) {
  __shared__ HTiles ht;
  const int l = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = l & 15, g = l >> 4;
  const int64_t e_base = (int64_t)blockIdx.x * kEdgesPerBlock;
  for (int t = wave; t < kTiles; t += kNtWaves) {
    const int64_t e = e_base + 16 * t + i;
    float cur[16];
    if (e < E) {
      load8(h + e * kK + 8 * g, cur);
      load8(h + e * kK + 32 + 8 * g, cur + 8);
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) cur[q] = 0.f;
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const Split B = split8(cur + 8 * ks);
      ht.b[t][ks][0][l] = B.hi;
      ht.b[t][ks][1][l] = B.mid;
      ht.b[t][ks][2][l] = B.lo;
    }
  }
  __syncthreads();
  const int slices = (M + 63) / 64;
  int wps = 1;  // waves per slice
  while (2 * wps * slices <= kNtWaves) wps *= 2;
  const int per = kTiles / wps, t0 = (wave % wps) * per;
  for (int s = wave / wps; s < slices; s += kNtWaves / wps) {
    const int nrb = min(4, (M - 64 * s) / 16);
    Split A[4][2];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (rb < nrb) load8(W + (int64_t)(64 * s + 16 * rb + i) * kK + 32 * ks + 8 * g, v);
        A[rb][ks] = split8(v);
      }
    }
    switch (nrb) {
      case 4: slice_tiles<4>(A, ht, t0, t0 + per, e_base, E, M, s, out); break;
      case 3: slice_tiles<3>(A, ht, t0, t0 + per, e_base, E, M, s, out); break;
      case 2: slice_tiles<2>(A, ht, t0, t0 + per, e_base, E, M, s, out); break;
      default: slice_tiles<1>(A, ht, t0, t0 + per, e_base, E, M, s, out); break;
    }
  }
}

// ---- adjoint: dh[E, 64] = dg[E, M] . W (W [M, 64]) ------------------------
// Transposed product D[k][e] = sum_m W[m][k] dg[e][m].  Wave s of a block owns
// the reduction slice m in [64 s, 64 s + 64), holds W's slice pre-split as the
// A operand (4 row blocks x 2 k-steps x 3 parts) and reads its 16 x 64 block
// of dg per 16-edge tile (B operand: lane l reads 32 contiguous bytes of edge
// l % 16), so dg streams from HBM exactly once.  The slices' partial sums meet
// in LDS and are added in slice order (deterministic); the LDS tile is double
// buffered so one barrier per tile suffices.  The next D tiles' dg blocks
// are loaded while the current one is multiplied (D = 1 at up to 12 waves,
// D = 3 at up to 8, whose register budget holds the deeper ring).
constexpr int kMaxSlices = 12;  // up to 768 gates: 12 waves per block leave 170 VGPRs per lane
constexpr int kRedRow = 68;  // LDS row pitch (floats) of a partial 16 x 64 tile

__device__ __forceinline__ void load_dg(const float* __restrict__ dg, int64_t e, int64_t E, int64_t ldg, int s,
                                        float* v) {
  const int g = (threadIdx.x & 63) >> 4;
  if (e < E) {
    load8(dg + e * ldg + 64 * s + 8 * g, v);
    load8(dg + e * ldg + 64 * s + 32 + 8 * g, v + 8);
  } else {
#pragma unroll
    for (int q = 0; q < 16; ++q) v[q] = 0.f;
  }
}

// dg rows have pitch ldg (a column block of a wider gradient); accumulate != 0 adds to dh.
// D: tiles of dg in flight per wave (a ring of register buffers); MAXS: waves per block at most.
template <int D, int MAXS>
__global__ __launch_bounds__(64 * MAXS) void gate_gemm_nn_kernel(const float* __restrict__ dg, int64_t ldg,
                                                                 int64_t E, const float* __restrict__ W, int M,
                                                                 float* __restrict__ dh, int accumulate) {
  extern __shared__ float red[];  // [2][S][16][kRedRow]
  const int l = threadIdx.x & 63, s = threadIdx.x >> 6, S = blockDim.x >> 6;
  const int i = l & 15, g = l >> 4;
  // A operand: row k = 16 kb + i, reduction index m = 64 s + 32 ks + 8 g + e  ->  W[m][k]
  Split A[4][2];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = W[(int64_t)(64 * s + 32 * ks + 8 * g + e) * kK + 16 * kb + i];
      A[kb][ks] = split8(v);
    }
  const int64_t tiles = (E + 15) / 16;
  const int64_t G = gridDim.x;
  float ring[D][16];
#pragma unroll
  for (int j = 0; j < D; ++j)
    if (blockIdx.x + j * G < tiles) load_dg(dg, 16 * (blockIdx.x + j * G) + i, E, ldg, s, ring[j]);
  int buf = 0;
  for (int64_t t0 = blockIdx.x; t0 < tiles; t0 += D * G) {
#pragma unroll
  for (int j = 0; j < D; ++j, buf ^= 1) {
    const int64_t t = t0 + j * G;
    if (t >= tiles) break;
    float cur[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) cur[q] = ring[j][q];
    if (t + D * G < tiles) load_dg(dg, 16 * (t + D * G) + i, E, ldg, s, ring[j]);
    const Split B0 = split8(cur), B1 = split8(cur + 8);
    v4f acc[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) acc[kb] = v4f{0.f, 0.f, 0.f, 0.f};
#define ICTC_STEP(PA, PB, KS, BB) \
  _Pragma("unroll") for (int kb = 0; kb < 4; ++kb) acc[kb] = mfma(A[kb][KS].PA, BB.PB, acc[kb]);
    ICTC_STEP(lo, hi, 0, B0) ICTC_STEP(hi, lo, 0, B0) ICTC_STEP(mid, mid, 0, B0)
    ICTC_STEP(lo, hi, 1, B1) ICTC_STEP(hi, lo, 1, B1) ICTC_STEP(mid, mid, 1, B1)
    ICTC_STEP(mid, hi, 0, B0) ICTC_STEP(hi, mid, 0, B0) ICTC_STEP(mid, hi, 1, B1)
    ICTC_STEP(hi, mid, 1, B1) ICTC_STEP(hi, hi, 0, B0) ICTC_STEP(hi, hi, 1, B1)
#undef ICTC_STEP
    // D: lane holds edge i, k = 16 kb + 4 g + r
    float* part = red + ((int64_t)(buf * S + s) * 16 + i) * kRedRow;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) *reinterpret_cast<v4f*>(part + 16 * kb + 4 * g) = acc[kb];
    __syncthreads();
    for (int q = threadIdx.x; q < 16 * 16; q += blockDim.x) {  // 16 edges x 16 float4 of k
      const int edge = q >> 4, kq = q & 15;
      const float* src = red + ((int64_t)(buf * S) * 16 + edge) * kRedRow + 4 * kq;
      v4f sum = *reinterpret_cast<const v4f*>(src);
      for (int w = 1; w < S; ++w) sum += *reinterpret_cast<const v4f*>(src + (int64_t)w * 16 * kRedRow);
      const int64_t e = 16 * t + edge;
      if (e < E) {
        v4f* o = reinterpret_cast<v4f*>(dh + e * kK + 4 * kq);
        *o = accumulate ? *o + sum : sum;
      }
    }
  }
  }
}

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

}  // namespace

extern "C" {

int ictc_gate_gemm_fwd(const float* hidden, int64_t edges, int hidden_width, const float* weight, int gates,
                       float* out, void* stream) {
  if (hidden_width != kK) return fail(ICTC_ERR_UNSUPPORTED, "gate projection is compiled for a 64-wide hidden layer");
  if (edges < 0 || gates <= 0 || gates % 16 != 0)
    return fail(ICTC_ERR_ARGUMENT, "gate projection: edges >= 0 and a positive multiple of 16 gates required");
  if (edges == 0) return ICTC_OK;
  if (!hidden || !weight || !out) return fail(ICTC_ERR_ARGUMENT, "gate projection: null operand");
  if ((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(out)) &
      15)
    return fail(ICTC_ERR_ARGUMENT, "gate projection: operands must be 16-byte aligned");
  const unsigned blocks = (unsigned)((edges + kEdgesPerBlock - 1) / kEdgesPerBlock);
  hipLaunchKernelGGL(gate_gemm_nt_kernel, dim3(blocks), dim3(64 * kNtWaves), 0, (hipStream_t)stream, hidden, edges, weight,
                     gates, out);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof(buf), "ictc_gate_gemm_fwd launch: %s", hipGetErrorString(e));
    return fail(ICTC_ERR_RUNTIME, buf);
  }
  return ICTC_OK;
}

int ictc_gate_gemm_bwd(const float* grad, int64_t edges, int gates, const float* weight, int hidden_width,
                       float* dhidden, void* stream) {
  return ictc_gate_gemm_bwd_strided(grad, gates, edges, gates, weight, hidden_width, dhidden, 0, stream);
}

int ictc_gate_gemm_bwd_strided(const float* grad, int64_t grad_pitch, int64_t edges, int gates, const float* weight,
                               int hidden_width, float* dhidden, int accumulate, void* stream) {
  if (hidden_width != kK) return fail(ICTC_ERR_UNSUPPORTED, "gate adjoint is compiled for a 64-wide hidden layer");
  if (edges < 0 || gates <= 0 || gates % 64 != 0 || gates > 64 * kMaxSlices)
    return fail(ICTC_ERR_UNSUPPORTED, "gate adjoint: gates must be a positive multiple of 64, at most 768");
  if (grad_pitch < gates || grad_pitch % 4) return fail(ICTC_ERR_ARGUMENT, "gate adjoint: grad pitch >= gates, a multiple of 4");
  if (edges == 0) return ICTC_OK;
  if (!grad || !weight || !dhidden) return fail(ICTC_ERR_ARGUMENT, "gate adjoint: null operand");
  if ((reinterpret_cast<uintptr_t>(grad) | reinterpret_cast<uintptr_t>(dhidden)) & 15)
    return fail(ICTC_ERR_ARGUMENT, "gate adjoint: operands must be 16-byte aligned");
  const int S = gates / 64;
  const int64_t tiles = (edges + 15) / 16;
  const size_t lds = sizeof(float) * 2 * S * 16 * kRedRow;
  // persistent blocks: as many as are resident at once (LDS and registers), so none waits for a second round
  // up to 512 gates: 8 waves with three tiles of dg in flight each (242 -> 214 us for 424k edges x 512);
  // wider blocks keep 12 waves with one tile in flight (the register budget of 3 waves per SIMD)
  const bool use_deep = S <= 8;
  int per_cu = 0;
  const hipError_t oe = use_deep ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gate_gemm_nn_kernel<3, 8>, 64 * S, lds)
                                 : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gate_gemm_nn_kernel<1, kMaxSlices>, 64 * S, lds);
  if (oe != hipSuccess || per_cu <= 0) per_cu = 1;
  if (per_cu > 4) per_cu = 4;
  const int64_t want = (int64_t)cu_count() * per_cu;
  const unsigned blocks = (unsigned)(tiles < want ? tiles : want);
  if (use_deep)
    hipLaunchKernelGGL((gate_gemm_nn_kernel<3, 8>), dim3(blocks), dim3(64 * S), lds, (hipStream_t)stream, grad,
                       grad_pitch, edges, weight, gates, dhidden, accumulate);
  else
    hipLaunchKernelGGL((gate_gemm_nn_kernel<1, kMaxSlices>), dim3(blocks), dim3(64 * S), lds, (hipStream_t)stream,
                       grad, grad_pitch, edges, weight, gates, dhidden, accumulate);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof(buf), "ictc_gate_gemm_bwd launch: %s", hipGetErrorString(e));
    return fail(ICTC_ERR_RUNTIME, buf);
  }
  return ICTC_OK;
}

}  // extern "C"
