// FP8 e4m3 activation quantizers for gfx950.
//
//   per-token (one scale per row; also the per-output-channel weight quant,
//     which is the same formula over a weight's rows):
//     s[m] = max(amax_k |x[m,k]| / 448, eps), q = e4m3(x / s)
//     -- src/torchinferno/kernels/fp8.py:53-72 (Triton _row_scale_cast_fp8),
//        fp8.py:129-138 (quantize_weight_fp8_per_channel, eps 1e-10)
//   1x128 block (DeepSeek act_quant):
//     s = max(amax_blk, 1e-4) * (1/448)  [or 2^ceil(log2(amax*(1/448)))],
//     q = e4m3(clamp(x / s, -448, 448))
//     -- src/torchinferno/kernels/deepseek_v4_tilelang_definitions.py:255-331
//   tensor scale (static or precomputed dynamic scale):
//     q = e4m3(x * inv_scale)  -- fp8.py:43-51 (_scale_cast_fp8)
//
// All arithmetic is fp32.  Scales come from IEEE division; the per-element
// quotients x / s reach the e4m3 cast as a product with 1/s where that provably
// rounds to the same code, else as the quotient (quot_for_e4m3).  The cast is
// round-to-nearest-even, so codes and scales are bit-identical to the same
// formulas evaluated by torch on the host.
#include <type_traits>

#include "fp8_common.h"

namespace ti {
namespace fp8 {
namespace {

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

template <int DT>
__device__ __forceinline__ void load8(const uint16_t* p, float (&f)[8]) {
  const uint4 v = *(const uint4*)p;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = act_to_f32<DT>((uint16_t)(w[i] & 0xFFFFu));
    f[2 * i + 1] = act_to_f32<DT>((uint16_t)(w[i] >> 16));
  }
}

__device__ __forceinline__ uint2 pack8(const uint32_t (&c)[8]) {
  return make_uint2(c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24),
                    c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24));
}

// Workgroup (row, chunk) of 256 threads; K % 8 == 0.  Every workgroup of a row
// reads the whole row for its max (the same value in each: max is exact), then
// quantizes its gridDim.y-th share of the row -- few rows (decode, small M)
// still spread over many workgroups.  RECIP forms the scale as
// amax * fl32(1/448) -- what torch computes for ``amax.float() / 448.0`` on a GPU
// tensor (a host-scalar divisor becomes a reciprocal multiply), the per-channel
// weight quant of fp8.py:129-138 -- instead of the quotient amax / 448.
template <int DT, bool RECIP>
__global__ __launch_bounds__(256) void quant_per_token_kernel(const uint16_t* __restrict__ x, int K,
                                                              uint8_t* __restrict__ q,
                                                              float* __restrict__ s, float eps) {
  __shared__ float red[4];
  const long row = blockIdx.x;
  const uint16_t* xr = x + row * K;
  float amax = 0.f;
  for (int i = threadIdx.x * 8; i < K; i += 256 * 8) {
    float f[8];
    load8<DT>(xr + i, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = fmaxf(RECIP ? amax * (1.0f / kE4M3Max) : amax / kE4M3Max, eps);
  if (threadIdx.x == 0 && blockIdx.y == 0) s[row] = sc;
  uint8_t* qr = q + row * K;
  const int chunk = ((K / 8 + gridDim.y - 1) / gridDim.y) * 8;
  const int i0 = blockIdx.y * chunk, i1 = min(K, i0 + chunk);
  for (int i = i0 + threadIdx.x * 8; i < i1; i += 256 * 8) {
    float f[8];
    load8<DT>(xr + i, f);
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = f[e] / sc;  // |y| <= 448 by the choice of sc
    *(uint2*)(qr + i) = e4m3_pack8_hw(y);
  }
}

// The same per-token quant for one workgroup per row with the row held in
// registers between the max and the quantization (NI 8-element loads per
// thread, K <= NI * 2048): x is read from memory once.  Codes as above (the
// quotient through quot_for_e4m3).
template <int DT, bool RECIP, int NI>
__global__ __launch_bounds__(256) void quant_per_token_reg_kernel(const uint16_t* __restrict__ x, int K,
                                                                  uint8_t* __restrict__ q,
                                                                  float* __restrict__ s, float eps) {
  __shared__ float red[4];
  const long row = blockIdx.x;
  const uint16_t* xr = x + row * K;
  uint4 v[NI];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int i = (j * 256 + (int)threadIdx.x) * 8;
    v[j] = i < K ? *(const uint4*)(xr + i) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      amax = fmaxf(amax, fmaxf(fabsf(act_to_f32<DT>((uint16_t)(w[e] & 0xFFFFu))),
                               fabsf(act_to_f32<DT>((uint16_t)(w[e] >> 16)))));
  }
  amax = wave_max(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = fmaxf(RECIP ? amax * (1.0f / kE4M3Max) : amax / kE4M3Max, eps);
  const float r = 1.0f / sc;
  if (threadIdx.x == 0) s[row] = sc;
  uint8_t* qr = q + row * K;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int i = (j * 256 + (int)threadIdx.x) * 8;
    if (i < K) {
      const uint32_t w[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
      float y[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y[2 * e] = quot_for_e4m3(act_to_f32<DT>((uint16_t)(w[e] & 0xFFFFu)), sc, r);
        y[2 * e + 1] = quot_for_e4m3(act_to_f32<DT>((uint16_t)(w[e] >> 16)), sc, r);
      }
      *(uint2*)(qr + i) = e4m3_pack8_hw(y);
    }
  }
}

// One wave per (row, 128-column block): 2 elements per lane.
template <int DT, bool POW2>
__global__ __launch_bounds__(256) void quant_block_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                          uint8_t* __restrict__ q,
                                                          float* __restrict__ s, int s_layout) {
  const int lane = threadIdx.x & 63;
  const int KB = K / 128;
  const long blk = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= (long)M * KB) return;
  const long row = blk / KB;
  const int kb = (int)(blk % KB);
  const long off = row * K + (long)kb * 128 + lane * 2;
  const uint32_t w = *(const uint32_t*)(x + off);
  const float f0 = act_to_f32<DT>((uint16_t)(w & 0xFFFFu));
  const float f1 = act_to_f32<DT>((uint16_t)(w >> 16));
  float amax = wave_max(fmaxf(fabsf(f0), fabsf(f1)));
  amax = fmaxf(amax, 1e-4f);
  const float inv_max = 1.0f / kE4M3Max;  // fp32 constant, as the reference's fp8_max_inv
  float sc;
  if constexpr (POW2) {
    // 2^ceil(log2(amax / 448)) from the exponent and mantissa bits.
    const uint32_t b = __float_as_uint(amax * inv_max);
    const int e = (int)((b >> 23) & 0xFF) - 127 + ((b & 0x7FFFFFu) != 0 ? 1 : 0);
    sc = __uint_as_float((uint32_t)(e + 127) << 23);
  } else {
    sc = amax * inv_max;
  }
  const float y0 = fminf(fmaxf(f0 / sc, -kE4M3Max), kE4M3Max);
  const float y1 = fminf(fmaxf(f1 / sc, -kE4M3Max), kE4M3Max);
  *(uint16_t*)(q + off) = (uint16_t)e4m3_encode2_hw(y0, y1);
  if (lane == 0) s[s_layout ? (long)kb * M + row : row * KB + kb] = sc;
}

// The same quant with 16-byte accesses: one wave per (row, four 128-wide
// blocks), a 16-lane group per block, 8 elements per lane (x 16-byte and q
// 8-byte aligned).  Same per-element arithmetic.
template <int DT, bool POW2>
__global__ __launch_bounds__(256) void quant_block_wide_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                               uint8_t* __restrict__ q, float* __restrict__ s,
                                                               int s_layout) {
  const int lane = threadIdx.x & 63;
  const int KB = K / 128;
  const int QB = (KB + 3) / 4;
  const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (long)M * QB) return;
  const long row = item / QB;
  const int kb = (int)(item % QB) * 4 + (lane >> 4);
  const bool on = kb < KB;
  const long off = row * K + (long)min(kb, KB - 1) * 128 + (lane & 15) * 8;
  float f[8];
  load8<DT>(x + off, f);
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  amax = fmaxf(amax, 1e-4f);
  const float inv_max = 1.0f / kE4M3Max;
  float sc;
  if constexpr (POW2) {
    const uint32_t b = __float_as_uint(amax * inv_max);
    const int e = (int)((b >> 23) & 0xFF) - 127 + ((b & 0x7FFFFFu) != 0 ? 1 : 0);
    sc = __uint_as_float((uint32_t)(e + 127) << 23);
  } else {
    sc = amax * inv_max;
  }
  // Power-of-two scales: the product with the exact reciprocal is the quotient.
  // (With other scales quot_for_e4m3 measured slower here than the division:
  // eight quotients per lane do not repay the reciprocal.)
  float y[8];
  if constexpr (POW2) {
    const float r = 1.0f / sc;
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = fminf(fmaxf(f[e] * r, -kE4M3Max), kE4M3Max);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = fminf(fmaxf(f[e] / sc, -kE4M3Max), kE4M3Max);
  }
  if (on) {
    *(uint2*)(q + off) = e4m3_pack8_hw(y);
    if ((lane & 15) == 0) s[s_layout ? (long)kb * M + row : row * KB + kb] = sc;
  }
}

// q = e4m3(x * inv_scale[0]); n % 8 == 0.
template <int DT>
__global__ __launch_bounds__(256) void quant_tensor_kernel(const uint16_t* __restrict__ x, long n,
                                                           const float* __restrict__ inv_scale,
                                                           uint8_t* __restrict__ q) {
  const float inv = *inv_scale;
  for (long i = ((long)blockIdx.x * 256 + threadIdx.x) * 8; i < n; i += (long)gridDim.x * 256 * 8) {
    float f[8];
    load8<DT>(x + i, f);
    uint32_t c[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) c[e] = e4m3_encode(f[e] * inv);
    *(uint2*)(q + i) = pack8(c);
  }
}


// ---- fused producers: one 1024-thread workgroup per row, the row held in
// registers (V vectors of 8 per thread, n <= 8192 * V), so HBM is read once and
// each element's arithmetic is done once.
constexpr int kRowThreads = 1024;
constexpr int kRowWaves = kRowThreads / 64;

__device__ __forceinline__ double row_sum_f64(double v, double* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int i = 0; i < kRowWaves; ++i) t += red[i];
  return t;
}

__device__ __forceinline__ float row_max_f32(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < kRowWaves; ++i) t = fmaxf(t, red[i]);
  return t;
}

// fp32 -> activation dtype -> fp32.  The empty asm pins f as an fp32 register
// value: without it the compiler folds a producing multiply and the fp16
// conversion into one mixed-precision FMA (v_fma_mixlo_f16), which skips the
// fp32 rounding of the product and changes results at fp16 ties.
template <int DT>
__device__ __forceinline__ float round_act(float f) {
  asm volatile("" : "+v"(f));
  return DT == TI_DTYPE_F16 ? f16_bits_to_f32(f32_to_f16_bits(f)) : bf16_bits_to_f32(f32_to_bf16_bits(f));
}

template <int DT>
__device__ __forceinline__ uint4 pack_act8(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = (uint32_t)to_bits<DT>(f[2 * i]) | ((uint32_t)to_bits<DT>(f[2 * i + 1]) << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Quantize the row held in v with scale max(amax / 448, 1e-10) and store it.
template <int V>
__device__ __forceinline__ void row_quant_store(float (&v)[V][8], float amax, int n, uint8_t* __restrict__ qr,
                                                float* __restrict__ s_out) {
  const float sc = fmaxf(amax / kE4M3Max, 1e-10f);
  const float r = 1.0f / sc;
  if (threadIdx.x == 0) *s_out = sc;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int i = (j * kRowThreads + threadIdx.x) * 8;
    if (i < n) {
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = quot_for_e4m3(v[j][e], sc, r);  // |y| <= 448 by the choice of sc
      *(uint2*)(qr + i) = e4m3_pack8_hw(y);
    }
  }
}

// (add +) RMSNorm -> per-token e4m3; n % 8 == 0, n <= 8192 * V.  Sum of
// squares in fp64 rounded once to fp32; rsqrt = 1/sqrtf (IEEE); the normalized
// row is rounded to the activation dtype before the quant.
template <int DT, int V, bool ADD>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_quant_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res, const uint16_t* __restrict__ w, int n,
    float eps, uint16_t* __restrict__ hidden, uint8_t* __restrict__ q, float* __restrict__ s) {
  __shared__ double redd[kRowWaves];
  __shared__ float redf[kRowWaves];
  const long row = blockIdx.x;
  float h[V][8];
  double ss = 0.0;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int i = (j * kRowThreads + threadIdx.x) * 8;
    if (i < n) {
      load8<DT>(x + row * n + i, h[j]);
      if constexpr (ADD) {
        float r[8];
        load8<DT>(res + row * n + i, r);
#pragma unroll
        for (int e = 0; e < 8; ++e) h[j][e] = h[j][e] + r[e];
        *(uint4*)(hidden + row * n + i) = pack_act8<DT>(h[j]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += (double)h[j][e] * (double)h[j][e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) h[j][e] = 0.f;
    }
  }
  ss = row_sum_f64(ss, redd);
  const float var = (float)ss / (float)n;
  const float rs = 1.0f / sqrtf(var + eps);
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < V; ++j) {
    const int i = (j * kRowThreads + threadIdx.x) * 8;
    if (i < n) {
      float wt[8];
      load8<DT>(w + i, wt);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        h[j][e] = round_act<DT>(h[j][e] * rs * wt[e]);
        amax = fmaxf(amax, fabsf(h[j][e]));
      }
    }
  }
  amax = row_max_f32(amax, redf);
  row_quant_store<V>(h, amax, n, q + row * n, s + row);
}

// silu(g) = g / (1 + exp(-g)) for bf16 g, exactly as the per-element
// expression computes it (exp in fp64 rounded to fp32, then an IEEE fp32
// quotient).  A bf16 value has 2^16 bit patterns; only those with
// 2^-25 <= |g| < 128 (exponent field 102..133, 8192 patterns) need the full
// expression: kSiluBf16 holds them, generated at build time by the same
// expression in numpy (build_lib.py:write_silu_table; fp64 exp lies far enough
// from every fp32 rounding boundary there that host and device round alike,
// and a GPU test checks all 2^16 inputs).  Each workgroup copies the table to
// LDS.  Elsewhere exp(-g) rounds to exactly 1 (|g| < 2^-25), 0 (g >= 128) or
// inf (g <= -128), so silu(g) is g * 0.5, g or -0; inf and NaN take the full
// expression.
constexpr int kExpE0 = 102;       // first tabulated exponent field
constexpr int kExpTab = 2 * 32 * 128;

__device__ __align__(16) const uint32_t kSiluBf16[kExpTab] = {
#include "silu_bf16_table.h"
};

__device__ __forceinline__ float silu_f64exp(float g) { return g / (1.0f + (float)exp(-(double)g)); }

__device__ __forceinline__ float silu_bf16(float g, const float* tab) {
  const uint32_t b = __float_as_uint(g) >> 16;
  const uint32_t e = (b >> 7) & 0xFFu;
  if (e - kExpE0 < 32u) return tab[((b >> 15) << 12) | ((e - kExpE0) << 7) | (b & 127u)];
  if (e < (uint32_t)kExpE0) return g * 0.5f;
  if (e == 0xFFu) return silu_f64exp(g);
  return (b >> 15) ? -0.0f : g;
}

// SwiGLU -> per-token e4m3: act = g / (1 + exp(-g)) * u (exp in fp64, rounded
// to fp32; bf16 inputs read the quotient from the table above), rounded to the
// activation dtype.  Rows of gate/up are strided; workgroups stride over rows.
template <int DT, int V>
__global__ __launch_bounds__(kRowThreads) void swiglu_quant_kernel(const uint16_t* __restrict__ gate, long gstride,
                                                                   const uint16_t* __restrict__ up, long ustride,
                                                                   int n, long rows, uint8_t* __restrict__ q,
                                                                   float* __restrict__ s) {
  constexpr bool TAB = DT == TI_DTYPE_BF16;
  __shared__ float redf[kRowWaves];
  __shared__ __align__(16) float etab[TAB ? kExpTab : 1];
  if constexpr (TAB) {
    for (int i = threadIdx.x * 4; i < kExpTab; i += kRowThreads * 4)
      *(uint4*)(etab + i) = *(const uint4*)(kSiluBf16 + i);
    __syncthreads();
  }
  for (long row = blockIdx.x; row < rows; row += gridDim.x) {
    float a[V][8];
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int i = (j * kRowThreads + threadIdx.x) * 8;
      if (i < n) {
        float g[8], u[8];
        load8<DT>(gate + row * gstride + i, g);
        load8<DT>(up + row * ustride + i, u);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float sg;
          if constexpr (TAB) sg = silu_bf16(g[e], etab);
          else sg = silu_f64exp(g[e]);
          a[j][e] = round_act<DT>(sg * u[e]);
          amax = fmaxf(amax, fabsf(a[j][e]));
        }
      }
    }
    amax = row_max_f32(amax, redf);
    row_quant_store<V>(a, amax, n, q + row * n, s + row);
    __syncthreads();  // redf is rewritten by the next row
  }
}

// Every fp32 bit pattern through both encoders; counts[0] = disagreements on
// finite |x| < 480, counts[1] = disagreements elsewhere (NaN, inf, overflow).
__global__ __launch_bounds__(256) void e4m3_selfcheck_kernel(unsigned long long* __restrict__ counts) {
  unsigned long long in_range = 0, outside = 0;
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t p = (uint64_t)blockIdx.x * 256 + threadIdx.x; p < (1ull << 31); p += stride) {
    const float x0 = __uint_as_float((uint32_t)(2 * p)), x1 = __uint_as_float((uint32_t)(2 * p + 1));
    const uint32_t hw = e4m3_encode2_hw(x0, x1);
    const bool ok0 = (hw & 0xFFu) == e4m3_encode(x0), ok1 = (hw >> 8) == e4m3_encode(x1);
    const bool dom0 = fabsf(x0) < 480.0f, dom1 = fabsf(x1) < 480.0f;  // false for NaN
    in_range += (dom0 && !ok0) + (dom1 && !ok1);
    outside += (!dom0 && !ok0) + (!dom1 && !ok1);
  }
  if (in_range) atomicAdd(&counts[0], in_range);
  if (outside) atomicAdd(&counts[1], outside);
}

// Every fp32 bit pattern through both bf16 roundings; counts[0] =
// disagreements on non-NaN inputs, counts[1] = on NaN inputs.
__global__ __launch_bounds__(256) void bf16_selfcheck_kernel(unsigned long long* __restrict__ counts) {
  unsigned long long num = 0, nan = 0;
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t p = (uint64_t)blockIdx.x * 256 + threadIdx.x; p < (1ull << 32); p += stride) {
    const float x = __uint_as_float((uint32_t)p);
    const bool bad = f32_to_bf16_bits(x) != f32_to_bf16_bits_sw(x);
    if (x == x) num += bad;
    else nan += bad;
  }
  if (num) atomicAdd(&counts[0], num);
  if (nan) atomicAdd(&counts[1], nan);
}

// Register-resident row width: the smallest V in {1, 2, 4, 8} with n <= 8192 V.
inline int row_vectors(int n) { return n <= 8192 ? 1 : n <= 16384 ? 2 : n <= 32768 ? 4 : 8; }
constexpr int kRowMaxN = 8 * kRowThreads * 8;

bool act_dtype_ok(int dt) { return dt == TI_DTYPE_F16 || dt == TI_DTYPE_BF16; }

}  // namespace
}  // namespace fp8
}  // namespace ti

using namespace ti;
using namespace ti::fp8;

extern "C" int ti_fp8_e4m3_selfcheck(unsigned long long* counts, hipStream_t stream) {
  TI_CHECK_ARG(counts, "ti_fp8_e4m3_selfcheck: null pointer");
  hipLaunchKernelGGL(e4m3_selfcheck_kernel, dim3(8192), dim3(256), 0, stream, counts);
  TI_CHECK_LAUNCH("ti_fp8_e4m3_selfcheck");
  return TI_OK;
}

extern "C" int ti_bf16_round_selfcheck(unsigned long long* counts, hipStream_t stream) {
  TI_CHECK_ARG(counts, "ti_bf16_round_selfcheck: null pointer");
  hipLaunchKernelGGL(bf16_selfcheck_kernel, dim3(8192), dim3(256), 0, stream, counts);
  TI_CHECK_LAUNCH("ti_bf16_round_selfcheck");
  return TI_OK;
}

static int quant_rows(const char* who, bool recip, const void* x, int x_dtype, int M, int K, float eps,
                      uint8_t* xq, float* xs, hipStream_t stream) {
  TI_CHECK_ARG(x && xq && xs, "%s: null pointer", who);
  TI_CHECK_ARG(act_dtype_ok(x_dtype), "%s: input must be fp16 or bf16", who);
  TI_CHECK_SHAPE(M >= 0 && K > 0 && K % 8 == 0, "%s: need K %% 8 == 0 (K=%d)", who, K);
  TI_CHECK_ARG(((uintptr_t)x & 15) == 0 && ((uintptr_t)xq & 7) == 0,
               "%s: input must be 16-byte and output 8-byte aligned", who);
  if (M == 0) return TI_OK;
  // column chunks: about 2048 workgroups in all, each at least 2048 elements
  // (measured: 512x28672 15.5 us on 4 chunks vs 19 us on one register-resident
  // workgroup per row; from 2048 rows one workgroup per row is fastest)
  const int chunks = std::max(1, std::min((2047 + M) / M, K / 2048));
  if (chunks == 1 && K <= 16 * 2048) {
    // one workgroup per row, the row in registers (NI loads of 8 per thread)
    const int ni = (K + 2047) / 2048;
#define TI_QRR(DT, R, NI)                                                                                      \
  hipLaunchKernelGGL((quant_per_token_reg_kernel<DT, R, NI>), dim3(M), dim3(256), 0, stream, (const uint16_t*)x, \
                     K, xq, xs, eps)
#define TI_QRN(DT, R)                                  \
  do {                                                 \
    if (ni <= 1) TI_QRR(DT, R, 1);                     \
    else if (ni <= 2) TI_QRR(DT, R, 2);                \
    else if (ni <= 4) TI_QRR(DT, R, 4);                \
    else if (ni <= 8) TI_QRR(DT, R, 8);                \
    else if (ni <= 12) TI_QRR(DT, R, 12);              \
    else TI_QRR(DT, R, 16);                            \
  } while (0)
    if (x_dtype == TI_DTYPE_F16) {
      if (recip) TI_QRN(TI_DTYPE_F16, true); else TI_QRN(TI_DTYPE_F16, false);
    } else {
      if (recip) TI_QRN(TI_DTYPE_BF16, true); else TI_QRN(TI_DTYPE_BF16, false);
    }
#undef TI_QRN
#undef TI_QRR
    TI_CHECK_LAUNCH(who);
    return TI_OK;
  }
#define TI_QR(DT, R)                                                                                             \
  hipLaunchKernelGGL((quant_per_token_kernel<DT, R>), dim3(M, chunks), dim3(256), 0, stream, (const uint16_t*)x, K, \
                     xq, xs, eps)
  if (x_dtype == TI_DTYPE_F16) {
    if (recip) TI_QR(TI_DTYPE_F16, true); else TI_QR(TI_DTYPE_F16, false);
  } else {
    if (recip) TI_QR(TI_DTYPE_BF16, true); else TI_QR(TI_DTYPE_BF16, false);
  }
#undef TI_QR
  TI_CHECK_LAUNCH(who);
  return TI_OK;
}

extern "C" int ti_fp8_quant_per_token(const void* x, int x_dtype, int M, int K, float eps,
                                      uint8_t* xq, float* xs, hipStream_t stream) {
  return quant_rows("ti_fp8_quant_per_token", false, x, x_dtype, M, K, eps, xq, xs, stream);
}

extern "C" int ti_fp8_quant_weight_per_channel(const void* w, int w_dtype, int N, int K, uint8_t* wq,
                                               float* ws, hipStream_t stream) {
  return quant_rows("ti_fp8_quant_weight_per_channel", true, w, w_dtype, N, K, 1e-10f, wq, ws, stream);
}

extern "C" int ti_fp8_quant_block(const void* x, int x_dtype, int M, int K, int block_size,
                                  int round_scale, uint8_t* xq, float* xs, int scale_layout,
                                  hipStream_t stream) {
  TI_CHECK_ARG(x && xq && xs, "ti_fp8_quant_block: null pointer");
  TI_CHECK_ARG(act_dtype_ok(x_dtype), "ti_fp8_quant_block: x must be fp16 or bf16");
  TI_CHECK_SHAPE(block_size == 128, "ti_fp8_quant_block: block_size must be 128 (got %d)", block_size);
  TI_CHECK_ARG(scale_layout == 0 || scale_layout == 1, "ti_fp8_quant_block: scale_layout must be 0 or 1");
  TI_CHECK_SHAPE(M >= 0 && K > 0 && K % 128 == 0, "ti_fp8_quant_block: need K %% 128 == 0 (K=%d)", K);
  TI_CHECK_ARG(((uintptr_t)x & 3) == 0 && ((uintptr_t)xq & 1) == 0,
               "ti_fp8_quant_block: x must be 4-byte and xq 2-byte aligned");
  if (M == 0) return TI_OK;
  const long blocks = (long)M * (K / 128);
  const bool wide = ((uintptr_t)x & 15) == 0 && ((uintptr_t)xq & 7) == 0;
  const long items = wide ? (long)M * ((K / 128 + 3) / 4) : blocks;
  dim3 grid((unsigned)((items + 3) / 4));
#define TI_QB(DT, P2)                                                                                     \
  do {                                                                                                    \
    if (wide)                                                                                             \
      hipLaunchKernelGGL((quant_block_wide_kernel<DT, P2>), grid, dim3(256), 0, stream, (const uint16_t*)x, \
                         M, K, xq, xs, scale_layout);                                                     \
    else                                                                                                  \
      hipLaunchKernelGGL((quant_block_kernel<DT, P2>), grid, dim3(256), 0, stream, (const uint16_t*)x,       \
                         M, K, xq, xs, scale_layout);                                                     \
  } while (0)
  if (x_dtype == TI_DTYPE_F16) {
    if (round_scale) TI_QB(TI_DTYPE_F16, true); else TI_QB(TI_DTYPE_F16, false);
  } else {
    if (round_scale) TI_QB(TI_DTYPE_BF16, true); else TI_QB(TI_DTYPE_BF16, false);
  }
#undef TI_QB
  TI_CHECK_LAUNCH("ti_fp8_quant_block");
  return TI_OK;
}

extern "C" int ti_fp8_quant_tensor(const void* x, int x_dtype, long n, const float* inv_scale,
                                   uint8_t* xq, hipStream_t stream) {
  TI_CHECK_ARG(x && xq && inv_scale, "ti_fp8_quant_tensor: null pointer");
  TI_CHECK_ARG(act_dtype_ok(x_dtype), "ti_fp8_quant_tensor: x must be fp16 or bf16");
  TI_CHECK_SHAPE(n >= 0 && n % 8 == 0, "ti_fp8_quant_tensor: need n %% 8 == 0 (n=%ld)", n);
  TI_CHECK_ARG(((uintptr_t)x & 15) == 0 && ((uintptr_t)xq & 7) == 0,
               "ti_fp8_quant_tensor: x must be 16-byte and xq 8-byte aligned");
  if (n == 0) return TI_OK;
  long blocks = (n / 8 + 255) / 256;
  dim3 grid((unsigned)(blocks < 4096 ? blocks : 4096));
  if (x_dtype == TI_DTYPE_F16)
    hipLaunchKernelGGL(quant_tensor_kernel<TI_DTYPE_F16>, grid, dim3(256), 0, stream,
                       (const uint16_t*)x, n, inv_scale, xq);
  else
    hipLaunchKernelGGL(quant_tensor_kernel<TI_DTYPE_BF16>, grid, dim3(256), 0, stream,
                       (const uint16_t*)x, n, inv_scale, xq);
  TI_CHECK_LAUNCH("ti_fp8_quant_tensor");
  return TI_OK;
}

extern "C" int ti_fp8_rmsnorm_quant_per_token(const void* x, const void* residual, const void* weight, int dtype,
                                              int rows, int n, float eps, void* hidden_out, uint8_t* xq, float* xs,
                                              hipStream_t stream) {
  using namespace ti::fp8;
  TI_CHECK_ARG(x && weight && xq && xs && (!residual || hidden_out), "ti_fp8_rmsnorm_quant_per_token: null pointer");
  TI_CHECK_ARG(act_dtype_ok(dtype), "ti_fp8_rmsnorm_quant_per_token: dtype must be fp16 or bf16");
  TI_CHECK_SHAPE(rows >= 0 && n > 0 && n % 8 == 0 && n <= kRowMaxN,
                 "ti_fp8_rmsnorm_quant_per_token: need n %% 8 == 0 and n <= %d (n=%d)", kRowMaxN, n);
  TI_CHECK_ARG(((uintptr_t)x & 15) == 0 && ((uintptr_t)weight & 15) == 0 && ((uintptr_t)xq & 7) == 0 &&
                   (!residual || (((uintptr_t)residual & 15) == 0 && ((uintptr_t)hidden_out & 15) == 0)),
               "ti_fp8_rmsnorm_quant_per_token: misaligned pointer");
  if (rows == 0) return TI_OK;
  const int v = row_vectors(n);
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(rows), dim3(kRowThreads), 0, stream, (const uint16_t*)x, (const uint16_t*)residual,
                       (const uint16_t*)weight, n, eps, (uint16_t*)hidden_out, xq, xs);
  };
  auto by_v = [&](auto dt, auto add) {
    constexpr int DT = decltype(dt)::value;
    constexpr bool ADD = decltype(add)::value;
    if (v == 1) launch(rmsnorm_quant_kernel<DT, 1, ADD>);
    else if (v == 2) launch(rmsnorm_quant_kernel<DT, 2, ADD>);
    else if (v == 4) launch(rmsnorm_quant_kernel<DT, 4, ADD>);
    else launch(rmsnorm_quant_kernel<DT, 8, ADD>);
  };
  using F16 = std::integral_constant<int, TI_DTYPE_F16>;
  using BF16 = std::integral_constant<int, TI_DTYPE_BF16>;
  if (dtype == TI_DTYPE_F16) {
    if (residual) by_v(F16{}, std::true_type{}); else by_v(F16{}, std::false_type{});
  } else {
    if (residual) by_v(BF16{}, std::true_type{}); else by_v(BF16{}, std::false_type{});
  }
  TI_CHECK_LAUNCH("ti_fp8_rmsnorm_quant_per_token");
  return TI_OK;
}

extern "C" int ti_fp8_swiglu_quant_per_token(const void* gate, long gate_row_stride, const void* up,
                                             long up_row_stride, int dtype, int rows, int n, uint8_t* xq, float* xs,
                                             hipStream_t stream) {
  using namespace ti::fp8;
  TI_CHECK_ARG(gate && up && xq && xs, "ti_fp8_swiglu_quant_per_token: null pointer");
  TI_CHECK_ARG(act_dtype_ok(dtype), "ti_fp8_swiglu_quant_per_token: dtype must be fp16 or bf16");
  TI_CHECK_SHAPE(rows >= 0 && n > 0 && n % 8 == 0 && n <= kRowMaxN && gate_row_stride % 8 == 0 &&
                     up_row_stride % 8 == 0,
                 "ti_fp8_swiglu_quant_per_token: need n and row strides %% 8 == 0 and n <= %d (n=%d)", kRowMaxN, n);
  TI_CHECK_ARG(((uintptr_t)gate & 15) == 0 && ((uintptr_t)up & 15) == 0 && ((uintptr_t)xq & 7) == 0,
               "ti_fp8_swiglu_quant_per_token: misaligned pointer");
  if (rows == 0) return TI_OK;
  const int v = row_vectors(n);
  // bf16: at most two workgroups per CU, each building its exp table once.
  const int grid = dtype == TI_DTYPE_BF16 ? (rows < 512 ? rows : 512) : rows;
  auto launch = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kRowThreads), 0, stream, (const uint16_t*)gate, gate_row_stride,
                       (const uint16_t*)up, up_row_stride, n, (long)rows, xq, xs);
  };
  auto by_v = [&](auto dt) {
    constexpr int DT = decltype(dt)::value;
    if (v == 1) launch(swiglu_quant_kernel<DT, 1>);
    else if (v == 2) launch(swiglu_quant_kernel<DT, 2>);
    else if (v == 4) launch(swiglu_quant_kernel<DT, 4>);
    else launch(swiglu_quant_kernel<DT, 8>);
  };
  if (dtype == TI_DTYPE_F16) by_v(std::integral_constant<int, TI_DTYPE_F16>{});
  else by_v(std::integral_constant<int, TI_DTYPE_BF16>{});
  TI_CHECK_LAUNCH("ti_fp8_swiglu_quant_per_token");
  return TI_OK;
}
