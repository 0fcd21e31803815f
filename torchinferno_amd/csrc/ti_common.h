// Shared helpers for the gfx950 quantized-linear kernels: status reporting,
// vector types for MFMA operands, and dtype conversions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>
#include <stdlib.h>

#include "../../include/ti_quant.h"

namespace ti {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

// Thread-local last-error text for ti_last_error().
void set_error(const char* fmt, ...);

#define TI_CHECK_ARG(cond, ...)                  \
  do {                                           \
    if (!(cond)) {                               \
      ::ti::set_error(__VA_ARGS__);              \
      return TI_ERR_INVALID;                     \
    }                                            \
  } while (0)

#define TI_CHECK_SHAPE(cond, ...)                \
  do {                                           \
    if (!(cond)) {                               \
      ::ti::set_error(__VA_ARGS__);              \
      return TI_ERR_UNSUPPORTED;                 \
    }                                            \
  } while (0)

#define TI_CHECK_LAUNCH(name)                                          \
  do {                                                                 \
    hipError_t e_ = hipGetLastError();                                 \
    if (e_ != hipSuccess) {                                            \
      ::ti::set_error("%s: launch failed: %s", name, hipGetErrorString(e_)); \
      return TI_ERR_HIP;                                               \
    }                                                                  \
  } while (0)

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
// fp32 -> bf16, round to nearest even; NaN -> quiet NaN.  The integer form;
// the kernels use f32_to_bf16_bits, one gfx950 v_cvt_pk_bf16_f32, which gives
// the same bits for all 2^32 inputs (ti_bf16_round_selfcheck compares them).
__device__ __forceinline__ uint16_t f32_to_bf16_bits_sw(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;  // v_cvt_f16_f32: IEEE round to nearest even
  return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

template <int DT>
__device__ __forceinline__ float load_act(const uint16_t* p) {
  if constexpr (DT == TI_DTYPE_F16) return f16_bits_to_f32(*p);
  else return bf16_bits_to_f32(*p);
}

template <int DT>
__device__ __forceinline__ uint16_t to_bits(float f) {
  if constexpr (DT == TI_DTYPE_F16) return f32_to_f16_bits(f);
  else return f32_to_bf16_bits(f);
}

__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace ti
