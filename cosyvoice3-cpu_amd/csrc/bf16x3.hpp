// Three-plane bfloat16 form of float32 values: x = hi + mid + lo, each plane the
// round-to-nearest bfloat16 of what the planes before it leave.  Each residual is
// exact in float32 (x minus a rounding of x to fewer bits), so |x - (hi + mid + lo)|
// <= 2^-8 |x - hi - mid| <= 2^-24 |x|: the planes carry all 24 bits of the float.
// A product a.b is then the six plane products whose weights reach 2^-16
// (hh, hm, mh, hl, mm, lh), each exact in the matrix core's float32 accumulate;
// the three dropped (ml, lm, ll) weigh at most ~2^-23 |a b|.
#pragma once

#include "common.hpp"

namespace cv3 {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> their hi, mid and lo planes, two bfloat16 per 32-bit word (a in the
// low half).  v_cvt_pk_bf16_f32 rounds to nearest even.
__device__ __forceinline__ void split_x3(float a, float b, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
  const f32x2_t x = {a, b};
  const bf16x2_t h = __builtin_convertvector(x, bf16x2_t);
  const f32x2_t r1 = x - __builtin_convertvector(h, f32x2_t);
  const bf16x2_t m = __builtin_convertvector(r1, bf16x2_t);
  const f32x2_t r2 = r1 - __builtin_convertvector(m, f32x2_t);
  const bf16x2_t l = __builtin_convertvector(r2, bf16x2_t);
  hi = __builtin_bit_cast(uint32_t, h);
  mid = __builtin_bit_cast(uint32_t, m);
  lo = __builtin_bit_cast(uint32_t, l);
}

// Eight floats (two float4) -> one 16-byte word of each plane.
__device__ __forceinline__ void split_x3(const float4& a, const float4& b, uint4& hi, uint4& mid, uint4& lo) {
  split_x3(a.x, a.y, hi.x, mid.x, lo.x);
  split_x3(a.z, a.w, hi.y, mid.y, lo.y);
  split_x3(b.x, b.y, hi.z, mid.z, lo.z);
  split_x3(b.z, b.w, hi.w, mid.w, lo.w);
}

}  // namespace cv3
