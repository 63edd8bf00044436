// Channel-mixing linears on the packed component-major layout, on split-bf16
// MFMA (v_mfma_f32_16x16x32_bf16, six products: FP32-level accuracy) where the
// weight panel fits LDS (K <= 256, every linear of the cfg4 model) and on FP32
// MFMA (v_mfma_f32_16x16x4_f32) beyond.  One kernel covers
//   EquivariantChannelLinearSO3 / product o3.Linear (ictd_irreps.py:207-227, products.py:817):
//       out[n, l, m, :] = s_l W_l x[n, l, m, :]                       (1 path in, 1 path out)
//   PathPreservingLinearSO3 (layers.py:317-355, common.py:368-374):
//       out[n, l, m, :] = s_l W_l concat_k msg[n, l, k, m, :]         (K_l paths in)
//   and their input adjoints (W_l^T, the path count moved to the output).
// Row layout of every degree block: [paths][2l+1][channels] (the message
// kernels' output order), so no transpose or concatenation is materialized.
//
// A degree block is a GEMM of (N rows per component m) x (paths_in * Cin) by
// (paths_in * Cin) x (paths_out * Cout).  A wave computes 16 nodes x 64
// output columns of one component; the block's waves share the weight
// panel (64 output columns x K) staged in LDS.  FP32 operand k
// order (consistent for A and B, which is all the MFMA needs): at k-step j,
// lane group g = l/16 supplies k = 16 g + j of the chunk, so each lane reads
// 16 contiguous floats of its row (four 16-byte loads).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>

#include "../../include/ictc_mi355x.h"
#include "split_bf16.h"

namespace ictc {
int set_error(int code, const char* msg);
}

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kMaxDeg = 4;
constexpr int kPanel = 64 + 4;  // LDS row pitch of the weight panel

struct LinearDesc {
  const float* w[kMaxDeg];   // [paths_out * Cout, paths_in * Cin] row-major
  int64_t in_off[kMaxDeg];   // column offset of the degree block in an input row
  int64_t out_off[kMaxDeg];
  int pin[kMaxDeg], pout[kMaxDeg];
  int wld[kMaxDeg];          // weight row length (paths_in * Cin of the whole map; a launch may take a slice)
  float scale[kMaxDeg];
  int lmax;
  int accumulate;            // add to the output rows instead of writing them
};

__device__ __forceinline__ v4f mfma(float a, float b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// FP32 MFMA form for panels too wide for LDS (K > kBf16MaxK with more channels than a slice holds; K <= kBf16MaxK runs the split-bf16 kernel
// below).  WHOLE: the block's whole weight panel (64 output columns x K) is staged in LDS once, and the
// block loops over 64-node tiles (grid.x persistent blocks); otherwise the panel is staged per 64-wide
// k-chunk.  MFMA operands: A = weights (M = 16 output columns), B = inputs (N = 16 nodes),
// so each lane ends with 4 consecutive output columns of one node and stores them as one 16-byte write.
constexpr int kWholeK = 256;
// Widest panel of the split-bf16 kernel: its three bf16 parts of 64 columns x 384 take 147 KB of LDS (one
// 16-wave block per CU either way, as at 256).
constexpr int kBf16MaxK = 384;

template <bool WHOLE>
__global__ __launch_bounds__(256) void packed_linear_kernel(const float* __restrict__ in, int64_t in_stride,
                                                            float* __restrict__ out, int64_t out_stride, int Ci,
                                                            int Co, int64_t N, LinearDesc d, int64_t node_blocks) {
  extern __shared__ float panel[];
  // blockIdx.y enumerates the (degree, component) pairs in order.
  int l = 0, m = blockIdx.y;
  while (m >= 2 * l + 1) {
    m -= 2 * l + 1;
    ++l;
  }
  const int w = 2 * l + 1;
  const int K = d.pin[l] * Ci, ncols = d.pout[l] * Co;
  const int col0 = 64 * blockIdx.z;
  if (col0 >= ncols) return;
  const float* __restrict__ W = d.w[l];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int Kr = (K + 63) / 64 * 64;  // K rounded to the k-chunk; the panel is zero past K
  const int pitch = WHOLE ? Kr + 4 : kPanel;
  auto stage = [&](int kc, int kn) {  // W[col0 .. col0+64) x [kc .. kc+kn) -> panel[r][k - kc] (zero outside)
    const int q4 = kn / 4;
    for (int t = threadIdx.x; t < 64 * q4; t += 256) {
      const int r = t / q4, q = t % q4;
      const int col = col0 + r, k = kc + 4 * q;
      float4 v = {0.f, 0.f, 0.f, 0.f};
      if (col < ncols && k < K) v = *reinterpret_cast<const float4*>(W + (int64_t)col * K + k);
      *reinterpret_cast<float4*>(panel + r * pitch + 4 * q) = v;
    }
  };
  if (WHOLE) {
    stage(0, Kr);
    __syncthreads();
  }
  const float s = d.scale[l];
  for (int64_t nb = blockIdx.x; nb < node_blocks; nb += gridDim.x) {
    const int64_t n0 = (nb * 4 + wave) * 16;
    const int64_t n = n0 + i;
    v4f acc[4];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) acc[cb] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int kc = 0; kc < K; kc += 64) {
      if (!WHOLE) {
        __syncthreads();
        stage(kc, 64);
        __syncthreads();
      }
      // B: node n, k = kc + 16 g + j (16 contiguous channels of one input path).
      float a[16];
      const int k0 = kc + 16 * g;
      if (n < N && k0 < K) {
        const int p = k0 / Ci, c = k0 % Ci;
        const float* src = in + n * in_stride + d.in_off[l] + ((int64_t)p * w + m) * Ci + c;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 v = *reinterpret_cast<const float4*>(src + 4 * q);
          a[4 * q] = v.x, a[4 * q + 1] = v.y, a[4 * q + 2] = v.z, a[4 * q + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) a[j] = 0.f;
      }
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        float b[16];
        const float* row = panel + (16 * cb + i) * pitch + (WHOLE ? kc : 0) + 16 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 v = *reinterpret_cast<const float4*>(row + 4 * q);
          b[4 * q] = v.x, b[4 * q + 1] = v.y, b[4 * q + 2] = v.z, b[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[cb] = mfma(b[j], a[j], acc[cb]);
      }
    }
    // D: lane holds output columns col0 + 16 cb + 4 g .. + 3 of node n0 + i.
    if (n < N) {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const int col = col0 + 16 * cb + 4 * g;
        if (col >= ncols) continue;
        const int p = col / Co, c = col % Co;
        *reinterpret_cast<v4f*>(out + n * out_stride + d.out_off[l] + ((int64_t)p * w + m) * Co + c) = s * acc[cb];
      }
    }
  }
}

// Split-bf16 form of the whole-panel path (K <= kBf16MaxK): the weight panel is split once into three bf16
// parts in LDS (the A operand of v_mfma_f32_16x16x32_bf16, lane l: output column 16 cb + l % 16,
// k = 32 ks + 8 (l / 16) .. + 7), each 16-node tile's inputs are split once per 32-wide k-step (B
// operand: node l % 16, the same k), and each 16 x 16 x 32 block keeps the six products whose size is at
// least 2^-24 of hi*hi (split_bf16.h), smallest first: FP32-level accuracy at a third of the FP32 MFMA
// time.  kLinWaves waves per block share the panel.
constexpr int kLinWaves = 16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4f mfma_bf16(bf16x8 a, bf16x8 b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// NZ: 64-column blocks per workgroup (all of a narrow linear's output columns, so its inputs are read once).
template <int NZ>
constexpr int lin_waves() { return NZ == 1 ? kLinWaves : kLinWaves / 2; }  // 64 accumulator VGPRs at NZ = 4

template <int NZ>
__global__ __launch_bounds__(lin_waves<NZ>() * 64, 1) void packed_linear_bf16_kernel(
    const float* __restrict__ in, int64_t in_stride, float* __restrict__ out, int64_t out_stride, int Ci, int Co,
    int64_t N, LinearDesc d, int64_t node_tiles) {
  constexpr int NCB = 4 * NZ;  // 16-column blocks
  extern __shared__ bf16x8 wpanel[];  // [ks][cb][part][lane]
  int l = 0, m = blockIdx.y;
  while (m >= 2 * l + 1) {
    m -= 2 * l + 1;
    ++l;
  }
  const int w = 2 * l + 1;
  const int K = d.pin[l] * Ci, ncols = d.pout[l] * Co;
  const int col0 = 64 * NZ * blockIdx.z;
  if (col0 >= ncols) return;
  const float* __restrict__ W = d.w[l];
  const int nks = (K + 31) / 32;
  for (int t = threadIdx.x; t < nks * NCB * 64; t += blockDim.x) {
    const int lane = t & 63, cb = (t >> 6) % NCB, ks = (t >> 6) / NCB;
    const int col = col0 + 16 * cb + (lane & 15), k = 32 * ks + 8 * (lane >> 4);
    float v[8];
    if (col < ncols && k < K) {
      const float4 a = *reinterpret_cast<const float4*>(W + (int64_t)col * d.wld[l] + k);
      const float4 b = *reinterpret_cast<const float4*>(W + (int64_t)col * d.wld[l] + k + 4);
      v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
    const Split sp = split8(v);
    bf16x8* o = wpanel + ((ks * NCB + cb) * 3) * 64 + lane;
    o[0] = sp.hi;
    o[64] = sp.mid;
    o[128] = sp.lo;
  }
  __syncthreads();
  const float sc = d.scale[l];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, i = lane & 15, g = lane >> 4;
  constexpr int NW = lin_waves<NZ>();
  for (int64_t tile = (int64_t)blockIdx.x * NW + wave; tile < node_tiles; tile += (int64_t)gridDim.x * NW) {
    const int64_t n = tile * 16 + i;
    v4f acc[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) acc[cb] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < nks; ++ks) {
      const int k0 = 32 * ks + 8 * g;
      float a[8];
      if (n < N && k0 < K) {
        const int p = k0 / Ci, c = k0 % Ci;
        const float* src = in + n * in_stride + d.in_off[l] + ((int64_t)p * w + m) * Ci + c;
        const float4 x0 = *reinterpret_cast<const float4*>(src), x1 = *reinterpret_cast<const float4*>(src + 4);
        a[0] = x0.x, a[1] = x0.y, a[2] = x0.z, a[3] = x0.w, a[4] = x1.x, a[5] = x1.y, a[6] = x1.z, a[7] = x1.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = 0.f;
      }
      const Split B = split8(a);
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const bf16x8* pp = wpanel + ((ks * NCB + cb) * 3) * 64 + lane;
        const bf16x8 wh = pp[0], wm = pp[64], wl = pp[128];
        // weight part x input part: lo*hi, hi*lo, mid*mid, mid*hi, hi*mid, hi*hi (smallest first)
        acc[cb] = mfma_bf16(wl, B.hi, acc[cb]);
        acc[cb] = mfma_bf16(wh, B.lo, acc[cb]);
        acc[cb] = mfma_bf16(wm, B.mid, acc[cb]);
        acc[cb] = mfma_bf16(wm, B.hi, acc[cb]);
        acc[cb] = mfma_bf16(wh, B.mid, acc[cb]);
        acc[cb] = mfma_bf16(wh, B.hi, acc[cb]);
      }
    }
    // D: lane holds output columns col0 + 16 cb + 4 g .. + 3 of node n0 + i.
    if (n < N) {
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const int col = col0 + 16 * cb + 4 * g;
        if (col >= ncols) continue;
        const int p = col / Co, c = col % Co;
        v4f* dst = reinterpret_cast<v4f*>(out + n * out_stride + d.out_off[l] + ((int64_t)p * w + m) * Co + c);
        *dst = d.accumulate ? *dst + sc * acc[cb] : sc * acc[cb];
      }
    }
  }
}

int fail(int code, const char* msg) { return ictc::set_error(code, msg); }

// The split-bf16 kernel over every (component, column block) pair: one 16-wave block per CU.
int launch_bf16(const float* in, int64_t in_stride, float* out, int64_t out_stride, int channels_in,
                int channels_out, int64_t nodes, const LinearDesc& d, int maxk, int maxcols, unsigned gy, unsigned gz,
                hipStream_t stream) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                               hipSuccess || cus <= 0)
    cus = 256;
  const int64_t node_tiles = (nodes + 15) / 16;
  // a narrow linear with up to 256 output columns covers them all in one workgroup (inputs read once)
  const bool wide4 = maxk <= 64 && maxcols > 64 && maxcols <= 256;
  const unsigned gzw = wide4 ? 1u : gz;
  const int nw = wide4 ? lin_waves<4>() : lin_waves<1>();
  const int64_t most = (node_tiles + nw - 1) / nw;
  // Blocks per (component, column block): one block per CU over all pairs; where that leaves more than a fifth
  // of the CUs idle (many pairs), the fewest whose estimated makespan (rounds of one block per CU times node
  // tiles per wave) is least.  cfg5's message-linear adjoint (16 components x 10 column blocks): 249 us with
  // one block per pair, 160 us with eight.
  const int64_t pairs = (int64_t)gy * gzw;
  int64_t gx = (int64_t)cus / pairs;
  gx = gx < 1 ? 1 : (gx > most ? most : gx);
  if (5 * gx * pairs < 4 * (int64_t)cus) {
    int64_t best = INT64_MAX;
    for (int64_t x = 1; x <= most && x <= 4 * cus; ++x) {
      const int64_t rounds = (x * pairs + cus - 1) / cus, per_wave = (node_tiles + x * nw - 1) / (x * nw);
      if (rounds * per_wave < best) {
        best = rounds * per_wave;
        gx = x;
      }
    }
  }
  const size_t lds = (size_t)(maxk / 32) * 4 * (wide4 ? 4 : 1) * 3 * 64 * sizeof(bf16x8);
  if (wide4)
    hipLaunchKernelGGL(packed_linear_bf16_kernel<4>, dim3((unsigned)gx, gy, 1), dim3(lin_waves<4>() * 64), lds, stream,
                       in, in_stride, out, out_stride, channels_in, channels_out, nodes, d, node_tiles);
  else
    hipLaunchKernelGGL(packed_linear_bf16_kernel<1>, dim3((unsigned)gx, gy, gz), dim3(lin_waves<1>() * 64), lds,
                       stream, in, in_stride, out, out_stride, channels_in, channels_out, nodes, d, node_tiles);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof(buf), "ictc_packed_linear launch: %s", hipGetErrorString(e));
    return fail(ICTC_ERR_RUNTIME, buf);
  }
  return ICTC_OK;
}

}  // namespace

extern "C" {

int ictc_packed_linear(int lmax, int channels_in, int channels_out, const float* in, int64_t in_stride,
                       const int* in_paths, const int64_t* in_offsets, float* out, int64_t out_stride,
                       const int* out_paths, const int64_t* out_offsets, const float* const* weights,
                       const float* scales, int64_t nodes, void* stream) {
  if (lmax < 0 || lmax >= kMaxDeg) return fail(ICTC_ERR_UNSUPPORTED, "packed linear: lmax must be 0..3");
  if (channels_in < 16 || channels_out < 16 || channels_in % 16 || channels_out % 16)
    return fail(ICTC_ERR_UNSUPPORTED, "packed linear: channel counts must be positive multiples of 16");
  if (nodes < 0 || in_stride < 0 || out_stride < 0 || !in_paths || !in_offsets || !out_paths || !out_offsets ||
      !weights || !scales)
    return fail(ICTC_ERR_ARGUMENT, "packed linear: invalid arguments");
  if (in_stride % 4 || out_stride % 4)
    return fail(ICTC_ERR_ARGUMENT, "packed linear: row strides must be multiples of 4 floats");
  LinearDesc d{};
  d.lmax = lmax;
  int maxcols = 0;
  for (int l = 0; l <= lmax; ++l) {
    if (in_paths[l] < 1 || out_paths[l] < 1 || in_offsets[l] % 4 || out_offsets[l] % 4 || out_offsets[l] < 0 ||
        in_offsets[l] < 0)
      return fail(ICTC_ERR_ARGUMENT, "packed linear: bad path counts or offsets");
    if (!weights[l]) return fail(ICTC_ERR_ARGUMENT, "packed linear: null weight");
    d.w[l] = weights[l];
    d.in_off[l] = in_offsets[l];
    d.out_off[l] = out_offsets[l];
    d.pin[l] = in_paths[l];
    d.pout[l] = out_paths[l];
    d.wld[l] = in_paths[l] * channels_in;
    d.scale[l] = scales[l];
    if (out_paths[l] * channels_out > maxcols) maxcols = out_paths[l] * channels_out;
  }
  if (nodes == 0) return ICTC_OK;
  if (!in || !out) return fail(ICTC_ERR_ARGUMENT, "packed linear: null operand");
  int maxk = 0;  // largest K, rounded to the 64-wide k-chunk
  for (int l = 0; l <= lmax; ++l) {
    const int kr = (in_paths[l] * channels_in + 63) / 64 * 64;
    maxk = kr > maxk ? kr : maxk;
  }
  const int64_t node_blocks = (nodes + 63) / 64;
  const unsigned gy = (unsigned)((lmax + 1) * (lmax + 1)), gz = (unsigned)((maxcols + 63) / 64);
  // Panels wider than the LDS holds run as consecutive launches over slices of the input paths (at most
  // kBf16MaxK / Cin paths each), the later ones adding to the output rows.
  const int slice = channels_in <= kBf16MaxK ? kBf16MaxK / channels_in : 0;
  if (maxk > kBf16MaxK && slice > 0) {
    int slices = 1;
    for (int l = 0; l <= lmax; ++l) slices = std::max(slices, (in_paths[l] + slice - 1) / slice);
    for (int j = 0; j < slices; ++j) {
      LinearDesc dj = d;
      dj.accumulate = j > 0;
      int kj = 0;
      for (int l = 0; l <= lmax; ++l) {
        const int p0 = std::min(j * slice, in_paths[l]), p1 = std::min((j + 1) * slice, in_paths[l]);
        dj.pin[l] = p1 - p0;
        dj.w[l] = weights[l] + (int64_t)p0 * channels_in;
        dj.in_off[l] = in_offsets[l] + (int64_t)p0 * (2 * l + 1) * channels_in;
        kj = std::max(kj, (dj.pin[l] * channels_in + 63) / 64 * 64);
      }
      if (int rc = launch_bf16(in, in_stride, out, out_stride, channels_in, channels_out, nodes, dj, kj, maxcols,
                               gy, gz, (hipStream_t)stream))
        return rc;
    }
    return ICTC_OK;
  }
  if (maxk <= kBf16MaxK) {
    if (int rc = launch_bf16(in, in_stride, out, out_stride, channels_in, channels_out, nodes, d, maxk, maxcols, gy,
                             gz, (hipStream_t)stream))
      return rc;
  } else {
    hipLaunchKernelGGL(packed_linear_kernel<false>, dim3((unsigned)node_blocks, gy, gz), dim3(256),
                       (size_t)64 * kPanel * sizeof(float), (hipStream_t)stream, in, in_stride, out, out_stride,
                       channels_in, channels_out, nodes, d, node_blocks);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char buf[256];
    snprintf(buf, sizeof(buf), "ictc_packed_linear launch: %s", hipGetErrorString(e));
    return fail(ICTC_ERR_RUNTIME, buf);
  }
  return ICTC_OK;
}

}  // extern "C"
