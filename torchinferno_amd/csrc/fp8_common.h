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

template <int DT>
__device__ __forceinline__ float act_to_f32(uint16_t h) {
  if constexpr (DT == TI_DTYPE_F16) return f16_bits_to_f32(h);
  else return bf16_bits_to_f32(h);
}

}  // namespace fp8
}  // namespace ti
