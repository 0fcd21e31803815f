// Shared device helpers of the FP8 (OCP e4m3fn) kernels: the fp32 -> e4m3
// encoder and 16-bit activation loads.
#pragma once

#include "ti_common.h"

namespace ti {
namespace fp8 {

constexpr float kE4M3Max = 448.0f;

// fp32 -> e4m3fn code, round to nearest even.  |x| >= 480 (the midpoint above
// the largest finite value) and NaN give the NaN code 0x7F with x's sign, the
// behaviour of torch's non-saturating float8_e4m3fn cast; callers scale into
// [-448, 448] first, so only the rounding matters on the product path.
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
  const uint32_t bits = __float_as_uint(x);
  const uint32_t sign = (bits >> 24) & 0x80u;
  const float a = fabsf(x);
  const uint32_t abits = __float_as_uint(a);
  uint32_t mag;
  if (!(a < 480.0f)) {  // also NaN
    mag = 0x7Fu;
  } else if (a < 0.015625f) {  // below 2^-6: subnormal step 2^-9, exact scaling
    mag = (uint32_t)__builtin_rintf(a * 512.0f);
  } else {
    const uint32_t lsb = (abits >> 20) & 1u;
    mag = ((abits + 0x7FFFFu + lsb) >> 20) - (120u << 3);
    mag = mag > 0x7Fu ? 0x7Fu : mag;
  }
  return mag | sign;
}

// Two fp32 -> e4m3fn codes by the gfx950 conversion instruction (round to
// nearest even): low byte x0, high byte x1.  Agrees with e4m3_encode for every
// finite |x| < 480 (ti_fp8_e4m3_selfcheck compares all 2^32 inputs); callers
// keep their inputs in that range.
__device__ __forceinline__ uint32_t e4m3_encode2_hw(float x0, float x1) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x0, x1, 0, false) & 0xFFFFu;
}

// Eight values (each finite, |y| < 480) -> eight e4m3fn bytes, in order.
__device__ __forceinline__ uint2 e4m3_pack8_hw(const float (&y)[8]) {
  return make_uint2(e4m3_encode2_hw(y[0], y[1]) | (e4m3_encode2_hw(y[2], y[3]) << 16),
                    e4m3_encode2_hw(y[4], y[5]) | (e4m3_encode2_hw(y[6], y[7]) << 16));
}

// x / sc as the e4m3 conversion sees it, without a division per element.  r is
// the correctly rounded 1/sc.  q = fl(x * r) lies within one fp32 ulp of the
// correctly rounded quotient fl(x / sc), so both round to the same e4m3 value
// unless they sit within a few ulps of an e4m3 rounding midpoint (low 20
// mantissa bits near 0x80000), below the e4m3 normal range (2^-6, where the
// rounding position moves), or near the top of the range (447 and above); there
// the quotient itself is returned.  The e4m3 codes are therefore those of the
// IEEE quotient; the returned float itself may differ from it by an ulp.
__device__ __forceinline__ float quot_for_e4m3(float x, float sc, float r) {
  const float q = x * r;
  const float a = fabsf(q);
  const uint32_t lo = __float_as_uint(q) & 0xFFFFFu;
  const bool clear = a >= 0.015625f && a < 447.0f && (lo - 0x7FFF8u) > 0x10u;  // |lo - 0x80000| > 8
  return clear ? q : x / sc;
}

template <int DT>
__device__ __forceinline__ float act_to_f32(uint16_t h) {
  if constexpr (DT == TI_DTYPE_F16) return f16_bits_to_f32(h);
  else return bf16_bits_to_f32(h);
}

}  // namespace fp8
}  // namespace ti
