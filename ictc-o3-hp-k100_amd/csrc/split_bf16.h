// FP32-level products on bf16 MFMA: each operand is written exactly as
// x = hi + mid + lo + r with hi, mid, lo bf16 (round-to-nearest-even at each
// level) and |r| <= 2^-27 |x|.  A product keeps the six terms whose size is
// at least 2^-24 of hi*hi (lo*hi, hi*lo, mid*mid, mid*hi, hi*mid, hi*hi,
// accumulated smallest first in FP32); the dropped terms are below 2^-25
// relative, under FP32 rounding.  bf16 has FP32's exponent range, so there is
// no overflow or scaling concern.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

union Bf8 {
  bf16x8 v;
  uint16_t u[8];
};

struct Split {
  bf16x8 hi, mid, lo;
};

// bf16 (as the upper half of an FP32 bit pattern) nearest to x, ties to even.
__device__ __forceinline__ uint32_t round_bf16(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u & 0xFFFF0000u;
}

__device__ __forceinline__ Split split8(const float* v) {
  Bf8 h, m, l;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t hb = round_bf16(v[e]);
    const float r1 = v[e] - __uint_as_float(hb);
    const uint32_t mb = round_bf16(r1);
    const float r2 = r1 - __uint_as_float(mb);
    const uint32_t lb = round_bf16(r2);
    h.u[e] = (uint16_t)(hb >> 16);
    m.u[e] = (uint16_t)(mb >> 16);
    l.u[e] = (uint16_t)(lb >> 16);
  }
  return {h.v, m.v, l.v};
}

}  // namespace
