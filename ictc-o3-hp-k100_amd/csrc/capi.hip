// extern "C" entry points of libictc_mi355x.so (declared in include/ictc_mi355x.h).
#include <hipcub/hipcub.hpp>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>

#include "../../include/ictc_mi355x.h"
#include "ictc_launch.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return ICTC_OK;
  return fail(ICTC_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(err));
}

// Natural-parity path count and output components (operators.py:206-207).
bool tp_counts(int li, int le, int lo, int* P, int* NO) {
  if (li < 0 || le < 0 || lo < 0 || li > 3 || le > 3 || lo > 3) return false;
  int p = 0, no = 0;
  for (int a = 0; a <= li; ++a)
    for (int b = 0; b <= le; ++b)
      for (int c = 0; c <= lo; ++c)
        if (((a - b) <= c && (b - a) <= c) && c <= a + b && ((a + b + c) % 2 == 0)) {
          ++p;
          no += 2 * c + 1;
        }
  if (P) *P = p;
  if (NO) *NO = no;
  return p > 0;
}

int check_shape(int li, int le, int lo, int C) {
  int P = 0;
  if (!tp_counts(li, le, lo, &P, nullptr))
    return fail(ICTC_ERR_UNSUPPORTED, "degrees (%d, %d, %d) are outside the compiled coverage (0..3, nonempty paths)",
                li, le, lo);
  if (ictc::channel_groups(C) == 0)
    return fail(ICTC_ERR_UNSUPPORTED, "channels=%d outside the supported range 1..256", C);
  return ICTC_OK;
}

ictc::Operands operands(const float* x, const float* sh, const float* g, const float* w, const float* mask,
                        int64_t rows, int64_t edges, int C, const int32_t* gate_rows = nullptr) {
  ictc::Operands a;
  a.grow = gate_rows;
  a.x = x;
  a.sh = sh;
  a.gates = g;
  a.weight = w;
  a.mask = mask;
  a.rows = rows;
  a.edges = edges;
  a.channels = C;
  return a;
}

// ---- CSR build kernels ----------------------------------------------------
__global__ void csr_keys_kernel(const int64_t* __restrict__ keys, int64_t E, int64_t N, int32_t* __restrict__ k32,
                                int32_t* __restrict__ ids) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= E) return;
  const int64_t k = keys[e];
  k32[e] = (k >= 0 && k < N) ? (int32_t)k : (int32_t)N;
  ids[e] = (int32_t)e;
}

// ptr[n] = first position whose sorted key >= n, for n in [0, N]; ptr[N+1] = E.
__global__ void csr_ptr_kernel(const int32_t* __restrict__ sorted, int64_t E, int64_t N, int32_t* __restrict__ ptr) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n > N + 1) return;
  if (n == N + 1) {
    ptr[n] = (int32_t)E;
    return;
  }
  int64_t lo = 0, hi = E;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (sorted[mid] < n) lo = mid + 1;
    else hi = mid;
  }
  ptr[n] = (int32_t)lo;
}

// ptr of keys that are already sorted (non-decreasing, all in [0, N)): ptr[n] = first position with key >= n
// for n in [0, N]; ptr[N+1] = E.
__global__ void csr_ptr_sorted_kernel(const int64_t* __restrict__ keys, int64_t E, int64_t N, int32_t* __restrict__ ptr) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n > N + 1) return;
  if (n == N + 1) {
    ptr[n] = (int32_t)E;
    return;
  }
  int64_t lo = 0, hi = E;
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (keys[mid] < n) lo = mid + 1;
    else hi = mid;
  }
  ptr[n] = (int32_t)lo;
}

int key_bits(int64_t N) {
  int bits = 1;
  while (bits < 31 && (int64_t(1) << bits) <= N) ++bits;
  return bits;
}

// Temporary-storage queries of the library sorts and scans ask the runtime for device properties on
// every call (tens of microseconds of host time per step); the answer is kept per thread for the last
// (device, size) asked.
struct TempMemo {
  int dev = -1;
  int64_t a = -1, b = -1;
  size_t bytes = 0;
  bool hit(int64_t x, int64_t y, int* d) {
    if (hipGetDevice(d) != hipSuccess) *d = -1;
    return *d == dev && x == a && y == b;
  }
  size_t keep(int d, int64_t x, int64_t y, size_t v) {
    dev = d, a = x, b = y, bytes = v;
    return v;
  }
};

size_t sort_temp_bytes(int64_t E, int64_t N) {
  thread_local TempMemo memo;
  int dev;
  if (memo.hit(E, key_bits(N), &dev)) return memo.bytes;
  size_t bytes = 0;
  (void)hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const int32_t*)nullptr, (int32_t*)nullptr,
                                     (const int32_t*)nullptr, (int32_t*)nullptr, (int)E, 0, key_bits(N));
  return memo.keep(dev, E, key_bits(N), bytes);
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// ---- Spatial (Morton) row order -------------------------------------------
// Spread the low 10 bits of v so that bit i moves to bit 3i.
__device__ __forceinline__ uint32_t spread3(uint32_t v) {
  v &= 0x3FFu;
  v = (v | (v << 16)) & 0x030000FFu;
  v = (v | (v << 8)) & 0x0300F00Fu;
  v = (v | (v << 4)) & 0x030C30C3u;
  v = (v | (v << 2)) & 0x09249249u;
  return v;
}

// 30-bit Morton key of the grid cell floor(pos / spacing) (each coordinate
// taken modulo 1024: a wrap only costs locality, never correctness).
__global__ void morton_keys_kernel(const float* __restrict__ pos, int64_t N, float inv_spacing,
                                   int32_t* __restrict__ keys, int32_t* __restrict__ ids) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  uint32_t q[3];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    const float v = pos[3 * i + d] * inv_spacing;
    // NaN / huge coordinates fall into cell 0 (locality only)
    const float f = (v == v && fabsf(v) < 1.0e9f) ? floorf(v) : 0.f;
    q[d] = (uint32_t)((int64_t)f & 0x3FF);
  }
  keys[i] = (int32_t)(spread3(q[0]) | (spread3(q[1]) << 1) | (spread3(q[2]) << 2));
  ids[i] = (int32_t)i;
}

size_t morton_temp_bytes(int64_t N) {
  thread_local TempMemo memo;
  int dev;
  if (memo.hit(N, 30, &dev)) return memo.bytes;
  size_t bytes = 0;
  (void)hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, (const int32_t*)nullptr, (int32_t*)nullptr,
                                     (const int32_t*)nullptr, (int32_t*)nullptr, (int)N, 0, 30);
  return memo.keep(dev, N, 30, bytes);
}

// Receiver row order: partial sums of |pos[i+1] - pos[i]| (index order) and |pos[rows[i+1]] - pos[rows[i]]|
// (the candidate order) per block, in a fixed order (deterministic), then every block of the second kernel
// forms both means from the partials and writes rows or the identity.
constexpr int kStepBlocks = 256;

__global__ __launch_bounds__(256) void step_partial_kernel(const float* __restrict__ pos, int64_t N,
                                                           const int32_t* __restrict__ rows,
                                                           double* __restrict__ part) {
  double a = 0.0, b = 0.0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i + 1 < N; i += (int64_t)gridDim.x * 256) {
    const int64_t r0 = rows[i], r1 = rows[i + 1];
    float da = 0.f, db = 0.f;
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const float u = pos[3 * (i + 1) + d] - pos[3 * i + d];
      const float v = pos[3 * r1 + d] - pos[3 * r0 + d];
      da += u * u;
      db += v * v;
    }
    a += sqrtf(da);
    b += sqrtf(db);
  }
  __shared__ double sa[256], sb[256];
  sa[threadIdx.x] = a;
  sb[threadIdx.x] = b;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) {
      sa[threadIdx.x] += sa[threadIdx.x + w];
      sb[threadIdx.x] += sb[threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    part[2 * blockIdx.x] = sa[0];
    part[2 * blockIdx.x + 1] = sb[0];
  }
}

__global__ __launch_bounds__(256) void step_choose_kernel(const double* __restrict__ part, int parts,
                                                          const int32_t* __restrict__ rows, int64_t N,
                                                          int32_t* __restrict__ out) {
  __shared__ int use_rows;
  if (threadIdx.x < 64) {   // one wave: strided partial sums, then a butterfly (a fixed order)
    double a = 0.0, b = 0.0;
    for (int k = threadIdx.x; k < parts; k += 64) {
      a += part[2 * k];
      b += part[2 * k + 1];
    }
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) {
      a += __shfl_xor(a, m, 64);
      b += __shfl_xor(b, m, 64);
    }
    if (threadIdx.x == 0) use_rows = a > 2.0 * b;   // the mean steps share the divisor N - 1
  }
  __syncthreads();
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < N) out[i] = use_rows ? rows[i] : (int32_t)i;
}

// Zero fill as a kernel (not hipMemsetAsync) so the call stays valid under
// HIP graph capture.
__global__ void fill_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

__global__ void fill_zero_i32_kernel(int32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

hipError_t route_edge_fwd(const ictc::TpShape& s, const ictc::Operands& a, float* out, hipStream_t st) {
  return ictc::launch_edge_fwd(s, a, out, st);
}
hipError_t route_edge_bwd(const ictc::TpShape& s, const ictc::Operands& a, const float* grad, float* dx, float* dsh,
                          float* dg, float* ws, hipStream_t st) {
  return ictc::launch_edge_bwd(s, a, grad, dx, dsh, dg, ws, st);
}
hipError_t route_msg_fwd(const ictc::TpShape& s, const ictc::Operands& a, const int64_t* src, ictc::Csr c,
                         float* out, hipStream_t st) {
  return ictc::launch_msg_fwd(s, a, src, c, out, st);
}
hipError_t route_edge_second(const ictc::TpShape& s, const ictc::Operands& a, const ictc::Tangents& t,
                             const float* grad, float* dgrad, float* dx, float* dsh, float* dg, float* ws,
                             hipStream_t st) {
  return ictc::launch_edge_second(s, a, t, grad, dgrad, dx, dsh, dg, ws, st);
}
hipError_t route_msg_bwd(const ictc::TpShape& s, const ictc::Operands& a, const int64_t* src, const int64_t* dst,
                         ictc::Csr dc, ictc::Csr sc, const float* grad, float* dx, float* dsh, float* dg, float* ws,
                         hipStream_t st) {
  return ictc::launch_msg_bwd(s, a, src, dst, dc, sc, grad, dx, dsh, dg, ws, st);
}

// Workspace floats for the channel groups' partial harmonic gradients.
int64_t group_ws_floats(int le, int C, int64_t E) {
  const int G = ictc::channel_groups(C);
  return G > 1 ? (int64_t)(G - 1) * E * (le + 1) * (le + 1) : 0;
}

int check_ws(const float* dsh, const float* ws, int64_t ws_bytes, int le, int C, int64_t E, const char* who) {
  const int64_t need = group_ws_floats(le, C, E) * (int64_t)sizeof(float);
  if (!dsh || need == 0) return ICTC_OK;
  if (!ws || ws_bytes < need)
    return fail(ICTC_ERR_ARGUMENT, "%s: dharmonics with %d channels needs a workspace of %lld bytes", who, C,
                (long long)need);
  return ICTC_OK;
}

__global__ void group_sum_kernel(float* __restrict__ out, const float* __restrict__ part, int64_t n, int slabs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float v = out[i];
  for (int s = 0; s < slabs; ++s) v += part[s * n + i];
  out[i] = v;
}

}  // namespace

namespace ictc {
hipError_t launch_group_sum(float* out, const float* part, int64_t n, int slabs, hipStream_t st) {
  if (slabs <= 0 || n <= 0) return hipSuccess;
  hipLaunchKernelGGL(group_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, out, part, n, slabs);
  return hipGetLastError();
}

int set_error(int code, const char* msg) {
  g_error = msg;
  return code;
}
}  // namespace ictc

extern "C" {

int ictc_version(void) { return 100; }

const char* ictc_last_error(void) { return g_error.c_str(); }

int ictc_tp_shape(int input_lmax, int edge_lmax, int output_lmax, int* num_paths, int* out_components) {
  if (!tp_counts(input_lmax, edge_lmax, output_lmax, num_paths, out_components))
    return fail(ICTC_ERR_UNSUPPORTED, "degrees (%d, %d, %d) unsupported", input_lmax, edge_lmax, output_lmax);
  return ICTC_OK;
}

int ictc_tp_fwd(int li, int le, int lo, int C, const float* x, const float* sh, const float* g, const float* w,
                int64_t E, float* out, void* stream) {
  if (int rc = check_shape(li, le, lo, C)) return rc;
  if (E < 0) return fail(ICTC_ERR_ARGUMENT, "edges must be nonnegative");
  if (E == 0) return ICTC_OK;
  if (!x || !sh || !g || !out) return fail(ICTC_ERR_ARGUMENT, "ictc_tp_fwd: null operand");
  const ictc::TpShape s{li, le, lo, C};
  return check_hip(route_edge_fwd(s, operands(x, sh, g, w, nullptr, E, E, C), out, (hipStream_t)stream),
                   "ictc_tp_fwd launch");
}

int64_t ictc_tp_workspace_bytes(int edge_lmax, int channels, int64_t edges) {
  if (edge_lmax < 0 || edge_lmax > 3 || ictc::channel_groups(channels) == 0 || edges < 0) return -1;
  return group_ws_floats(edge_lmax, channels, edges) * (int64_t)sizeof(float);
}

int ictc_tp_bwd(int li, int le, int lo, int C, const float* x, const float* sh, const float* g, const float* w,
                const float* grad, int64_t E, float* dx, float* dsh, float* dg, void* workspace,
                int64_t workspace_bytes, void* stream) {
  if (int rc = check_shape(li, le, lo, C)) return rc;
  if (E < 0) return fail(ICTC_ERR_ARGUMENT, "edges must be nonnegative");
  if (E == 0 || (!dx && !dsh && !dg)) return ICTC_OK;
  if (!x || !sh || !g || !grad) return fail(ICTC_ERR_ARGUMENT, "ictc_tp_bwd: null operand");
  if (int rc = check_ws(dsh, (const float*)workspace, workspace_bytes, le, C, E, "ictc_tp_bwd")) return rc;
  const ictc::TpShape s{li, le, lo, C};
  return check_hip(route_edge_bwd(s, operands(x, sh, g, w, nullptr, E, E, C), grad, dx, dsh, dg, (float*)workspace,
                                         (hipStream_t)stream),
                   "ictc_tp_bwd launch");
}

int64_t ictc_csr_workspace_bytes(int64_t E, int64_t N) {
  if (E < 0 || N < 0 || E >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) - 2) return -1;
  return (int64_t)(3 * align256(sizeof(int32_t) * (size_t)(E > 0 ? E : 1)) + align256(sort_temp_bytes(E, N)));
}

int ictc_csr_build(const int64_t* keys, int64_t E, int64_t N, int32_t* ptr, int32_t* order, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  if (E < 0 || N < 0) return fail(ICTC_ERR_ARGUMENT, "csr: negative size");
  if (E >= (int64_t(1) << 31) || N >= (int64_t(1) << 31) - 2)
    return fail(ICTC_ERR_UNSUPPORTED, "csr: more than 2^31 edges or nodes");
  if (!ptr) return fail(ICTC_ERR_ARGUMENT, "csr: null ptr");
  hipStream_t st = (hipStream_t)stream;
  if (E == 0) {
    hipLaunchKernelGGL(fill_zero_i32_kernel, dim3((unsigned)((N + 2 + 255) / 256)), dim3(256), 0, st, ptr, N + 2);
    return check_hip(hipGetLastError(), "csr fill");
  }
  if (!keys) return fail(ICTC_ERR_ARGUMENT, "csr: null keys");
  if (!order) {   // the caller's keys are already sorted and in range: the order is the identity
    hipLaunchKernelGGL(csr_ptr_sorted_kernel, dim3((unsigned)((N + 2 + 255) / 256)), dim3(256), 0, st, keys, E, N,
                       ptr);
    return check_hip(hipGetLastError(), "csr ptr (sorted keys)");
  }
  if (!workspace) return fail(ICTC_ERR_ARGUMENT, "csr: null workspace");
  const int64_t need = ictc_csr_workspace_bytes(E, N);
  if (workspace_bytes < need)
    return fail(ICTC_ERR_ARGUMENT, "csr: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
  char* ws = (char*)workspace;
  const size_t slab = align256(sizeof(int32_t) * (size_t)E);
  int32_t* k_in = (int32_t*)ws;
  int32_t* k_out = (int32_t*)(ws + slab);
  int32_t* ids = (int32_t*)(ws + 2 * slab);
  void* temp = ws + 3 * slab;
  size_t temp_bytes = sort_temp_bytes(E, N);
  hipLaunchKernelGGL(csr_keys_kernel, dim3((unsigned)((E + 255) / 256)), dim3(256), 0, st, keys, E, N, k_in, ids);
  if (int rc = check_hip(hipGetLastError(), "csr keys")) return rc;
  // Radix sort is stable: equal keys keep increasing edge order.
  if (int rc = check_hip(hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, k_in, k_out, ids, order, (int)E, 0,
                                                            key_bits(N), st),
                         "csr sort"))
    return rc;
  hipLaunchKernelGGL(csr_ptr_kernel, dim3((unsigned)((N + 2 + 255) / 256)), dim3(256), 0, st, k_out, E, N, ptr);
  return check_hip(hipGetLastError(), "csr ptr");
}

int64_t ictc_morton_workspace_bytes(int64_t N) {
  if (N < 0 || N >= (int64_t(1) << 31)) return -1;
  return (int64_t)(3 * align256(sizeof(int32_t) * (size_t)(N > 0 ? N : 1)) + align256(morton_temp_bytes(N)));
}

int ictc_morton_order(const float* pos, int64_t N, float spacing, int32_t* order, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  if (N < 0) return fail(ICTC_ERR_ARGUMENT, "morton order: negative size");
  if (N >= (int64_t(1) << 31)) return fail(ICTC_ERR_UNSUPPORTED, "morton order: more than 2^31 rows");
  if (!(spacing > 0.f)) return fail(ICTC_ERR_ARGUMENT, "morton order: spacing must be positive");
  if (N == 0) return ICTC_OK;
  if (!pos || !order || !workspace) return fail(ICTC_ERR_ARGUMENT, "morton order: null operand");
  const int64_t need = ictc_morton_workspace_bytes(N);
  if (workspace_bytes < need)
    return fail(ICTC_ERR_ARGUMENT, "morton order: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                (long long)need);
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)workspace;
  const size_t slab = align256(sizeof(int32_t) * (size_t)N);
  int32_t* keys = (int32_t*)ws;
  int32_t* ids = (int32_t*)(ws + slab);
  int32_t* sorted_keys = (int32_t*)(ws + 2 * slab);
  void* temp = ws + 3 * slab;
  size_t temp_bytes = morton_temp_bytes(N);
  hipLaunchKernelGGL(morton_keys_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, st, pos, N, 1.f / spacing,
                     keys, ids);
  if (int rc = check_hip(hipGetLastError(), "morton keys")) return rc;
  return check_hip(hipcub::DeviceRadixSort::SortPairs(temp, temp_bytes, keys, sorted_keys, ids, order, (int)N, 0, 30, st),
                   "morton sort");
}

int64_t ictc_receiver_rows_workspace_bytes(int64_t N) {
  if (N < 0 || N >= (int64_t(1) << 31)) return -1;
  return (int64_t)(2 * kStepBlocks * sizeof(double));
}

int ictc_receiver_rows(const float* pos, int64_t N, const int32_t* rows, int32_t* out, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  if (N < 0) return fail(ICTC_ERR_ARGUMENT, "receiver rows: negative size");
  if (N >= (int64_t(1) << 31)) return fail(ICTC_ERR_UNSUPPORTED, "receiver rows: more than 2^31 rows");
  if (N == 0) return ICTC_OK;
  if (!pos || !rows || !out || !workspace) return fail(ICTC_ERR_ARGUMENT, "receiver rows: null operand");
  if (workspace_bytes < ictc_receiver_rows_workspace_bytes(N))
    return fail(ICTC_ERR_ARGUMENT, "receiver rows: workspace smaller than ictc_receiver_rows_workspace_bytes");
  hipStream_t st = (hipStream_t)stream;
  double* part = (double*)workspace;
  const int parts = (int)std::min<int64_t>(kStepBlocks, (N + 255) / 256);
  hipLaunchKernelGGL(step_partial_kernel, dim3(parts), dim3(256), 0, st, pos, N, rows, part);
  if (int rc = check_hip(hipGetLastError(), "receiver rows partial")) return rc;
  hipLaunchKernelGGL(step_choose_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, st, part, parts, rows, N,
                     out);
  return check_hip(hipGetLastError(), "receiver rows");
}

int ictc_msg_fwd(int li, int le, int lo, int C, const float* x, const float* sh, const float* g, const float* w,
                 const float* mask, const int64_t* src, int64_t N, int64_t E, const int32_t* dptr,
                 const int32_t* dorder, const int32_t* dst_rows, float* out, const int32_t* gate_rows, void* stream) {
  if (int rc = check_shape(li, le, lo, C)) return rc;
  if (N < 0 || E < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  if (N == 0) return ICTC_OK;
  if (!x || !out || !dptr || (E > 0 && (!sh || !g || !src)))
    return fail(ICTC_ERR_ARGUMENT, "ictc_msg_fwd: null operand");
  const ictc::TpShape s{li, le, lo, C};
  return check_hip(route_msg_fwd(s, operands(x, sh, g, w, mask, N, E, C, gate_rows), src, ictc::Csr{dptr, dorder, dst_rows}, out,
                                        (hipStream_t)stream),
                   "ictc_msg_fwd launch");
}

static int msg_bwd(int li, int le, int lo, int C, const float* x, const float* sh, const float* g, const float* w,
                   const float* mask, const int64_t* src, const int64_t* dst, int64_t N, int64_t E,
                   const int32_t* dptr, const int32_t* dorder, const int32_t* sptr, const int32_t* sorder,
                   const int32_t* dst_rows, const int32_t* src_rows, const float* grad, float* dx, float* dsh,
                   float* dg, void* workspace, int64_t workspace_bytes, void* stream, int dg_acc) {
  if (int rc = check_shape(li, le, lo, C)) return rc;
  if (N < 0 || E < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  if (E == 0) {
    // no edges: dsh and dg are empty, dx is zero
    const int64_t n = dx ? N * (int64_t)(C * (li + 1) * (li + 1)) : 0;
    if (n == 0) return ICTC_OK;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, dx, n);
    return check_hip(hipGetLastError(), "dx fill");
  }
  if (!x || !sh || !g || !src || !dst || !grad || !dptr) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_bwd: null operand");
  if (dx && !sptr) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_bwd: dfeatures needs the source CSR");
  if (int rc = check_ws(dsh, (const float*)workspace, workspace_bytes, le, C, E, "ictc_msg_bwd")) return rc;
  const ictc::TpShape s{li, le, lo, C};
  ictc::Operands a = operands(x, sh, g, w, mask, N, E, C);
  a.dg_acc = dg_acc;
  return check_hip(route_msg_bwd(s, a, src, dst, ictc::Csr{dptr, dorder, dst_rows}, ictc::Csr{sptr, sorder, src_rows},
                                 grad, dx, dsh, dg, (float*)workspace, (hipStream_t)stream),
                   "ictc_msg_bwd launch");
}

int ictc_msg_bwd(int li, int le, int lo, int C, const float* x, const float* sh, const float* g, const float* w,
                 const float* mask, const int64_t* src, const int64_t* dst, int64_t N, int64_t E,
                 const int32_t* dptr, const int32_t* dorder, const int32_t* sptr, const int32_t* sorder,
                 const int32_t* dst_rows, const int32_t* src_rows, const float* grad, float* dx, float* dsh, float* dg,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  return msg_bwd(li, le, lo, C, x, sh, g, w, mask, src, dst, N, E, dptr, dorder, sptr, sorder, dst_rows, src_rows,
                 grad, dx, dsh, dg, workspace, workspace_bytes, stream, 0);
}

int ictc_msg_bwd_accumulate(int li, int le, int lo, int C, const float* x, const float* sh, const float* g,
                            const float* w, const float* mask, const int64_t* src, const int64_t* dst, int64_t N,
                            int64_t E, const int32_t* dptr, const int32_t* dorder, const int32_t* sptr,
                            const int32_t* sorder, const int32_t* dst_rows, const int32_t* src_rows,
                            const float* grad, float* dx, float* dsh, float* dg, void* workspace,
                            int64_t workspace_bytes, void* stream) {
  if (!dg) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_bwd_accumulate: dgates is required");
  return msg_bwd(li, le, lo, C, x, sh, g, w, mask, src, dst, N, E, dptr, dorder, sptr, sorder, dst_rows, src_rows,
                 grad, dx, dsh, dg, workspace, workspace_bytes, stream, 1);
}

int64_t ictc_msg_bwd_tangent_workspace_bytes(int edge_lmax, int C, int64_t E) {
  const int G = ictc::channel_groups(C);
  if (G == 0 || E < 0) return -1;
  return G > 1 ? (int64_t)(G - 1) * E * ((edge_lmax + 1) * (edge_lmax + 1) + 1) * (int64_t)sizeof(float) : 0;
}

int ictc_msg_bwd_tangent(int li, int le, int lo, int C, const float* x, const float* sh, const float* g,
                         const float* w, const float* mask, const int64_t* src, const int64_t* dst, int64_t N,
                         int64_t E, const int32_t* dptr, const int32_t* dorder, const int32_t* sptr,
                         const int32_t* sorder, const int32_t* dst_rows, const int32_t* src_rows, const float* grad,
                         const float* gdot, float* dx, float* dsh, float* dr, void* workspace,
                         int64_t workspace_bytes, const int32_t* gate_rows, void* stream) {
  if (int rc = check_shape(li, le, lo, C)) return rc;
  if (N < 0 || E < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  if (E == 0) {
    // no edges: dsh and dr are empty, dx is zero
    const int64_t n = dx ? N * (int64_t)(C * (li + 1) * (li + 1)) : 0;
    if (n == 0) return ICTC_OK;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, dx, n);
    return check_hip(hipGetLastError(), "dx fill");
  }
  if (!dr) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_bwd_tangent: dr is required");
  if (!x || !sh || !g || !gdot || !src || !dst || !grad || !dptr)
    return fail(ICTC_ERR_ARGUMENT, "ictc_msg_bwd_tangent: null operand");
  if (dx && !sptr) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_bwd_tangent: dfeatures needs the source CSR");
  const int64_t need = ictc_msg_bwd_tangent_workspace_bytes(le, C, E);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(ICTC_ERR_ARGUMENT, "ictc_msg_bwd_tangent: %d channels need a workspace of %lld bytes", C,
                (long long)need);
  const ictc::TpShape s{li, le, lo, C};
  return check_hip(ictc::launch_msg_bwd_tangent(s, operands(x, sh, g, w, mask, N, E, C, gate_rows), src, dst,
                                                ictc::Csr{dptr, dorder, dst_rows}, ictc::Csr{sptr, sorder, src_rows},
                                                grad, gdot, dx, dsh, dr, (float*)workspace, (hipStream_t)stream),
                   "ictc_msg_bwd_tangent launch");
}

int ictc_tp_second(int li, int le, int lo, int C, const float* x, const float* sh, const float* g, const float* w,
                   const float* grad, const float* tx, const float* tsh, const float* tg, int64_t E, float* dgrad,
                   float* dx, float* dsh, float* dg, void* workspace, int64_t workspace_bytes, void* stream) {
  if (int rc = check_shape(li, le, lo, C)) return rc;
  if (E < 0) return fail(ICTC_ERR_ARGUMENT, "edges must be nonnegative");
  if (E == 0 || (!dgrad && !dx && !dsh && !dg)) return ICTC_OK;
  if (!x || !sh || !g) return fail(ICTC_ERR_ARGUMENT, "ictc_tp_second: null operand");
  if ((dx || dsh || dg) && !grad) return fail(ICTC_ERR_ARGUMENT, "ictc_tp_second: dfeatures/dharmonics/dgates need grad");
  if (int rc = check_ws(dsh, (const float*)workspace, workspace_bytes, le, C, E, "ictc_tp_second")) return rc;
  const ictc::TpShape s{li, le, lo, C};
  const ictc::Tangents t{tx, tsh, tg};
  return check_hip(route_edge_second(s, operands(x, sh, g, w, nullptr, E, E, C), t, grad, dgrad, dx, dsh, dg,
                                     (float*)workspace, (hipStream_t)stream),
                   "ictc_tp_second launch");
}

int ictc_msg_second(int li, int le, int lo, int C, const float* x, const float* sh, const float* g, const float* w,
                    const float* mask, const int64_t* src, const int64_t* dst, int64_t N, int64_t E,
                    const int32_t* dptr, const int32_t* dorder, const int32_t* sptr, const int32_t* sorder,
                    const int32_t* dst_rows, const int32_t* src_rows, const float* grad, const float* tx,
                    const float* tsh, const float* tg, float* dgrad, float* dx, float* dsh, float* dg, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  if (int rc = check_shape(li, le, lo, C)) return rc;
  if (N < 0 || E < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  hipStream_t st = (hipStream_t)stream;
  if (E == 0) {  // node outputs are zero; there are no edge outputs
    int P = 0, NO = 0;
    tp_counts(li, le, lo, &P, &NO);
    const int64_t sizes[2] = {N * (int64_t)(C * NO), N * (int64_t)(C * (li + 1) * (li + 1))};
    float* outs[2] = {dgrad, dx};
    for (int k = 0; k < 2; ++k) {
      if (!outs[k] || sizes[k] == 0) continue;
      hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((sizes[k] + 255) / 256)), dim3(256), 0, st, outs[k],
                         sizes[k]);
      if (int rc = check_hip(hipGetLastError(), "ictc_msg_second fill")) return rc;
    }
    return ICTC_OK;
  }
  if (N == 0 || (!dgrad && !dx && !dsh && !dg)) return ICTC_OK;
  if (!x || !sh || !g || !src || !dst || !dptr) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_second: null operand");
  if ((dx || dsh || dg) && !grad)
    return fail(ICTC_ERR_ARGUMENT, "ictc_msg_second: dfeatures/dharmonics/dgates need grad");
  if (dx && !sptr) return fail(ICTC_ERR_ARGUMENT, "ictc_msg_second: dfeatures needs the source CSR");
  if (int rc = check_ws(dsh, (const float*)workspace, workspace_bytes, le, C, E, "ictc_msg_second")) return rc;
  const ictc::TpShape s{li, le, lo, C};
  const ictc::Tangents t{tx, tsh, tg};
  const ictc::Operands a = operands(x, sh, g, w, mask, N, E, C);
  if (dgrad || dsh || dg) {
    if (int rc = check_hip(ictc::launch_msg_second_rcv(s, a, t, src, ictc::Csr{dptr, dorder, dst_rows}, grad, dgrad,
                                                       dsh, dg, (float*)workspace, st),
                           "ictc_msg_second launch"))
      return rc;
  }
  if (dx)
    return check_hip(ictc::launch_msg_second_src(s, a, t, dst, ictc::Csr{sptr, sorder, src_rows}, grad, dx, st),
                     "ictc_msg_second launch");
  return ICTC_OK;
}

int ictc_sh_fwd(const float* n, int64_t E, int lmax, float* out, void* stream) {
  if (lmax < 0 || lmax > 3) return fail(ICTC_ERR_UNSUPPORTED, "harmonics lmax=%d outside 0..3", lmax);
  if (E < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  if (E == 0) return ICTC_OK;
  if (!n || !out) return fail(ICTC_ERR_ARGUMENT, "ictc_sh_fwd: null operand");
  const dim3 grid((unsigned)((E + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  switch (lmax) {
    case 0: hipLaunchKernelGGL(ictc::sh_fwd_kernel<0>, grid, dim3(256), 0, st, n, E, out); break;
    case 1: hipLaunchKernelGGL(ictc::sh_fwd_kernel<1>, grid, dim3(256), 0, st, n, E, out); break;
    case 2: hipLaunchKernelGGL(ictc::sh_fwd_kernel<2>, grid, dim3(256), 0, st, n, E, out); break;
    default: hipLaunchKernelGGL(ictc::sh_fwd_kernel<3>, grid, dim3(256), 0, st, n, E, out); break;
  }
  return check_hip(hipGetLastError(), "ictc_sh_fwd launch");
}

int ictc_sh_bwd(const float* n, const float* grad, int64_t E, int lmax, float* dn, void* stream) {
  if (lmax < 0 || lmax > 3) return fail(ICTC_ERR_UNSUPPORTED, "harmonics lmax=%d outside 0..3", lmax);
  if (E < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  if (E == 0) return ICTC_OK;
  if (!n || !grad || !dn) return fail(ICTC_ERR_ARGUMENT, "ictc_sh_bwd: null operand");
  const dim3 grid((unsigned)((E + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  switch (lmax) {
    case 0: hipLaunchKernelGGL(ictc::sh_bwd_kernel<0>, grid, dim3(256), 0, st, n, grad, E, dn); break;
    case 1: hipLaunchKernelGGL(ictc::sh_bwd_kernel<1>, grid, dim3(256), 0, st, n, grad, E, dn); break;
    case 2: hipLaunchKernelGGL(ictc::sh_bwd_kernel<2>, grid, dim3(256), 0, st, n, grad, E, dn); break;
    default: hipLaunchKernelGGL(ictc::sh_bwd_kernel<3>, grid, dim3(256), 0, st, n, grad, E, dn); break;
  }
  return check_hip(hipGetLastError(), "ictc_sh_bwd launch");
}

int ictc_sh_jvp(const float* n, const float* hn, int64_t E, int lmax, float* out, void* stream) {
  if (lmax < 0 || lmax > 3) return fail(ICTC_ERR_UNSUPPORTED, "harmonics lmax=%d outside 0..3", lmax);
  if (E < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  if (E == 0) return ICTC_OK;
  if (!n || !hn || !out) return fail(ICTC_ERR_ARGUMENT, "ictc_sh_jvp: null operand");
  const dim3 grid((unsigned)((E + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  switch (lmax) {
    case 0: hipLaunchKernelGGL(ictc::sh_jvp_kernel<0>, grid, dim3(256), 0, st, n, hn, E, out); break;
    case 1: hipLaunchKernelGGL(ictc::sh_jvp_kernel<1>, grid, dim3(256), 0, st, n, hn, E, out); break;
    case 2: hipLaunchKernelGGL(ictc::sh_jvp_kernel<2>, grid, dim3(256), 0, st, n, hn, E, out); break;
    default: hipLaunchKernelGGL(ictc::sh_jvp_kernel<3>, grid, dim3(256), 0, st, n, hn, E, out); break;
  }
  return check_hip(hipGetLastError(), "ictc_sh_jvp launch");
}

int ictc_sh_hvp(const float* n, const float* grad, const float* hn, int64_t E, int lmax, float* out, void* stream) {
  if (lmax < 0 || lmax > 3) return fail(ICTC_ERR_UNSUPPORTED, "harmonics lmax=%d outside 0..3", lmax);
  if (E < 0) return fail(ICTC_ERR_ARGUMENT, "negative size");
  if (E == 0) return ICTC_OK;
  if (!n || !grad || !hn || !out) return fail(ICTC_ERR_ARGUMENT, "ictc_sh_hvp: null operand");
  const dim3 grid((unsigned)((E + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  switch (lmax) {
    case 0: hipLaunchKernelGGL(ictc::sh_hvp_kernel<0>, grid, dim3(256), 0, st, n, grad, hn, E, out); break;
    case 1: hipLaunchKernelGGL(ictc::sh_hvp_kernel<1>, grid, dim3(256), 0, st, n, grad, hn, E, out); break;
    case 2: hipLaunchKernelGGL(ictc::sh_hvp_kernel<2>, grid, dim3(256), 0, st, n, grad, hn, E, out); break;
    default: hipLaunchKernelGGL(ictc::sh_hvp_kernel<3>, grid, dim3(256), 0, st, n, grad, hn, E, out); break;
  }
  return check_hip(hipGetLastError(), "ictc_sh_hvp launch");
}

}  // extern "C"
