// Device helpers shared by the int4 W4A16 kernels (int4_gemm.hip, int4_decode.hip):
// the in-register nibble unpack, the bf16/fp16 MFMA step, and the per-group
// compute of one wave (bias-corrected MFMA sums scaled into fp32 accumulators).
#pragma once

#include "ti_common.h"

namespace ti {
namespace int4 {

constexpr int kGroup = 128;

template <int DT>
struct Magic;
template <>
struct Magic<TI_DTYPE_F16> {
  static constexpr uint32_t kOr = 0x64006400u;            // 1024 + q
  static constexpr float kBias = 1032.0f;                 // 1024 + zero point 8
  static constexpr uint32_t kNegBiasPair = 0xE408E408u;   // fp16 -1032 x2
};
template <>
struct Magic<TI_DTYPE_BF16> {
  static constexpr uint32_t kOr = 0x43004300u;            // 128 + q
  static constexpr float kBias = 136.0f;                  // 128 + zero point 8
  static constexpr uint32_t kNegBiasPair = 0xC308C308u;   // bf16 -136 x2
};

// (x & mask) | magic in one v_and_or_b32 (the compiler otherwise splits it).
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm volatile("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(mask), "v"(magic));
  return r;
}

template <int DT>
__device__ __forceinline__ i32x4 unpack8(uint32_t w, uint32_t mask, uint32_t magic) {
  i32x4 r;
  r[0] = (int)and_or(w, mask, magic);
  r[1] = (int)and_or(w >> 4, mask, magic);
  r[2] = (int)and_or(w >> 8, mask, magic);
  r[3] = (int)and_or(w >> 12, mask, magic);
  return r;
}

// Two words at once: one 64-bit shift yields both words' shifted copies (the
// low word's top bits pick up the high word's low nibbles, which the mask
// discards), so a pair costs 3 shifts instead of 6.
__device__ __forceinline__ void unpack16(uint32_t w0, uint32_t w1, uint32_t mask, uint32_t magic, i32x4& r0,
                                         i32x4& r1) {
  const uint64_t x = ((uint64_t)w1 << 32) | w0;
  uint64_t s4, s8, s12;
  asm("v_lshrrev_b64 %0, 4, %1" : "=v"(s4) : "v"(x));
  asm("v_lshrrev_b64 %0, 8, %1" : "=v"(s8) : "v"(x));
  asm("v_lshrrev_b64 %0, 12, %1" : "=v"(s12) : "v"(x));
  r0[0] = (int)and_or(w0, mask, magic);
  r0[1] = (int)and_or((uint32_t)s4, mask, magic);
  r0[2] = (int)and_or((uint32_t)s8, mask, magic);
  r0[3] = (int)and_or((uint32_t)s12, mask, magic);
  r1[0] = (int)and_or(w1, mask, magic);
  r1[1] = (int)and_or((uint32_t)(s4 >> 32), mask, magic);
  r1[2] = (int)and_or((uint32_t)(s8 >> 32), mask, magic);
  r1[3] = (int)and_or((uint32_t)(s12 >> 32), mask, magic);
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16x16x32(i32x4 a, i32x4 b, f32x4 c) {
  if constexpr (DT == TI_DTYPE_F16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

template <int DT>
__device__ __forceinline__ float scale_to_f32(uint32_t bits) {
  return DT == TI_DTYPE_F16 ? f16_bits_to_f32((uint16_t)bits) : bf16_bits_to_f32((uint16_t)bits);
}

template <int DT, int MT, int NT>
__device__ __forceinline__ void compute_group(const i32x4 (&w)[NT], const i32x4 (&a)[MT][4],
                                              const float (&sc)[NT], f32x4 (&acc)[NT][MT]) {
  const uint32_t mask = 0x000F000Fu, magic = Magic<DT>::kOr;
  const i32x4 negbias = {(int)Magic<DT>::kNegBiasPair, (int)Magic<DT>::kNegBiasPair,
                         (int)Magic<DT>::kNegBiasPair, (int)Magic<DT>::kNegBiasPair};
  f32x4 nbias[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    nbias[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) nbias[mt] = mfma16x16x32<DT>(a[mt][j], negbias, nbias[mt]);
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    // The 64-bit-shift unpack: measured 1-4% faster in the skinny kernels
    // (M <= 32); the tall-tile compute below keeps the 32-bit form, where it
    // measured neutral to slightly slower.
    i32x4 b[4];
    unpack16((uint32_t)w[t][0], (uint32_t)w[t][1], mask, magic, b[0], b[1]);
    unpack16((uint32_t)w[t][2], (uint32_t)w[t][3], mask, magic, b[2], b[3]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 cc = nbias[mt];
#pragma unroll
      for (int j = 0; j < 4; ++j) cc = mfma16x16x32<DT>(a[mt][j], b[j], cc);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][mt][i] = __builtin_fmaf(sc[t], cc[i], acc[t][mt][i]);
    }
  }
}


// The same per-group compute for tall tiles (MT >= 4): each weight tile is
// unpacked once, then the 16-row activation tiles are read from LDS one at a
// time (get_a(mt, j)), so only one row tile's A operand is live at a time.
template <int DT, int MT, int NT, typename GetA>
__device__ __forceinline__ void compute_group_rows(const i32x4 (&w)[NT], GetA&& get_a, const float (&sc)[NT],
                                                   f32x4 (&acc)[NT][MT]) {
  const uint32_t mask = 0x000F000Fu, magic = Magic<DT>::kOr;
  const i32x4 negbias = {(int)Magic<DT>::kNegBiasPair, (int)Magic<DT>::kNegBiasPair,
                         (int)Magic<DT>::kNegBiasPair, (int)Magic<DT>::kNegBiasPair};
  i32x4 b[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) b[t][j] = unpack8<DT>((uint32_t)w[t][j], mask, magic);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    i32x4 a[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = get_a(mt, j);
    f32x4 nb = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) nb = mfma16x16x32<DT>(a[j], negbias, nb);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 cc = nb;
#pragma unroll
      for (int j = 0; j < 4; ++j) cc = mfma16x16x32<DT>(a[j], b[t][j], cc);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][mt][i] = __builtin_fmaf(sc[t], cc[i], acc[t][mt][i]);
    }
  }
}

}  // namespace int4
}  // namespace ti
