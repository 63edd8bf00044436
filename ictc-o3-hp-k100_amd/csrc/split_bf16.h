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

struct Split {
  bf16x8 hi, mid, lo;
};

// The conversions use gfx950's f32 -> bf16 convert (v_cvt_pk_bf16_f32, round
// to nearest even): the same parts as rounding the bit pattern by hand, in
// about a third of the VALU operations.
__device__ __forceinline__ Split split8(const float* v) {
  bf16x8 h, m, l;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 hb = (__bf16)v[e];
    const float r1 = v[e] - (float)hb;
    const __bf16 mb = (__bf16)r1;
    const float r2 = r1 - (float)mb;
    h[e] = hb;
    m[e] = mb;
    l[e] = (__bf16)r2;
  }
  return {h, m, l};
}

}  // namespace
