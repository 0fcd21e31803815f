// int4 W4A16 group-128 dequant-GEMM for gfx950 (CDNA4).
//
// Replaces Marlin's marlin_gemm as used by the reference's marlin_int4_mm
// (src/torchinferno/kernels/marlin.py:142-171): out[M,N] = a[M,K] @ W[K,N],
// W[k,n] = (q[k,n] - 8) * s[k/128, n], fp32 accumulation.
//
// Kernel weight layout ("tile-group" layout).  The weight is cut into tiles of
// 16 output columns x 128 rows of K (one quantization group).  A tile is 1 KiB
// and is stored contiguously so that one wave reads it with one 16-byte load
// per lane: lane l = 16*kq + c holds column c, and its dword j holds the 8
// codes at k = 128*g + 32*j + 8*kq + e (e = 0..7).  Those 8 codes are exactly
// the B operand lane l feeds to step j of v_mfma_f32_16x16x32_{f16,bf16}; the
// A operand uses the same (j, kq, e) -> k map, so the MFMA computes the true
// dot product whatever order the hardware assigns to the 32 K slots.
// Inside a dword, nibble p holds element e = 2p (p < 4) or e = 2(p-4)+1, so
// (w >> 4p) & 0x000F000F puts elements (2p, 2p+1) in the low/high halves.
//
// Unpack: OR-ing a nibble into the mantissa of a magic constant gives an exact
// biased value (fp16: 0x6400|q = 1024+q, bf16: 0x4300|q = 128+q) -- one
// v_and_or per two weights plus a shift.  The bias is removed exactly in fp32
// by starting each group's accumulator at -(bias+8) * rowsum(a), itself one
// MFMA against a constant operand per step that all column tiles share.  The
// group's scale is then applied in fp32: acc += s * group_sum.  Weights thus
// enter the MFMA as exact integers (no fp16 rounding of (q-8)*s).
//
// Work split: a workgroup of W waves owns NT column tiles (16*NT columns) and a
// range of groups; its waves split that range; a grid-level split-K (splits)
// fills the 256 CUs when N is small.  Wave partials are reduced through LDS;
// split partials go to an fp32 workspace and the last workgroup to arrive
// (atomic ticket) sums them in split order, so results are deterministic.
// The ticket counter is reset by that last workgroup, never by a memset.
#include "ti_common.h"

namespace ti {
namespace int4 {

constexpr int kGroup = 128;
constexpr int kWaves = 4;    // waves per workgroup
constexpr int kNT = 4;       // 16-column tiles per workgroup
constexpr int kMaxMT = 4;    // 16-row tiles per workgroup (M chunk = 64 rows)

__device__ __forceinline__ uint32_t interleave_nibbles(uint32_t w) {
  uint32_t r = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    int p = (e & 1) ? 4 + (e >> 1) : (e >> 1);
    r |= ((w >> (4 * e)) & 0xFu) << (4 * p);
  }
  return r;
}

// Canonical [K/8, N] -> tile-group layout; one thread per output dword.
__global__ void repack_weight_kernel(const uint32_t* __restrict__ q, uint32_t* __restrict__ out,
                                     int N, int NG, long total) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  int j = idx & 3;
  int lane = (idx >> 2) & 63;
  long tg = idx >> 8;
  int g = (int)(tg % NG);
  int t = (int)(tg / NG);
  int c = lane & 15, kq = lane >> 4;
  int n = t * 16 + c;
  long krow = (long)g * 16 + j * 4 + kq;  // canonical word row: k/8
  out[idx] = interleave_nibbles(q[krow * N + n]);
}

// scales [NG, N] -> [N/16][NG][16].
__global__ void repack_scale_kernel(const uint16_t* __restrict__ s, uint16_t* __restrict__ out,
                                    int N, int NG, long total) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  int c = idx & 15;
  long tg = idx >> 4;
  int g = (int)(tg % NG);
  int t = (int)(tg / NG);
  out[idx] = s[(long)g * N + t * 16 + c];
}

template <int DT>
struct Magic;
template <>
struct Magic<TI_DTYPE_F16> {
  static constexpr uint32_t kOr = 0x64006400u;   // 1024 + q
  static constexpr float kBias = 1032.0f;        // 1024 + zero point 8
  static constexpr uint32_t kNegBiasPair = 0xE408E408u;  // fp16 -1032 x2
};
template <>
struct Magic<TI_DTYPE_BF16> {
  static constexpr uint32_t kOr = 0x43004300u;   // 128 + q
  static constexpr float kBias = 136.0f;         // 128 + zero point 8
  static constexpr uint32_t kNegBiasPair = 0xC308C308u;  // bf16 -136 x2
};

template <int DT>
__device__ __forceinline__ i32x4 unpack8(uint32_t w) {
  i32x4 r;
  r[0] = (int)((w & 0x000F000Fu) | Magic<DT>::kOr);
  r[1] = (int)(((w >> 4) & 0x000F000Fu) | Magic<DT>::kOr);
  r[2] = (int)(((w >> 8) & 0x000F000Fu) | Magic<DT>::kOr);
  r[3] = (int)(((w >> 12) & 0x000F000Fu) | Magic<DT>::kOr);
  return r;
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

// Exact dequant of the tile-group layout, through the same unpack8.
template <int DT>
__global__ void dequant_kernel(const i32x4* __restrict__ wp, const uint16_t* __restrict__ sp,
                               float* __restrict__ out, int N, int NG) {
  // one wave per (tile, group); lane layout as in the GEMM
  const int lane = threadIdx.x & 63;
  const long tg = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (tg >= (long)(N / 16) * NG) return;
  const int g = (int)(tg % NG), t = (int)(tg / NG);
  const int c = lane & 15, kq = lane >> 4;
  const float s = load_act<DT>(sp + tg * 16 + c);
  const i32x4 w = wp[tg * 64 + lane];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    i32x4 b = unpack8<DT>((uint32_t)w[j]);
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      uint16_t bits = (uint16_t)(((uint32_t)b[h >> 1]) >> (16 * (h & 1)));
      float biased = (DT == TI_DTYPE_F16) ? f16_bits_to_f32(bits) : bf16_bits_to_f32(bits);
      float q = biased - Magic<DT>::kBias;  // q - 8, exact
      long k = (long)g * kGroup + j * 32 + kq * 8 + h;
      out[k * N + t * 16 + c] = q * s;
    }
  }
}

template <int DT, int MT>
__global__ __launch_bounds__(64 * kWaves) void w4a16_gemm_kernel(
    const uint16_t* __restrict__ A, const i32x4* __restrict__ Wp, const uint16_t* __restrict__ Sp,
    uint16_t* __restrict__ out, float* __restrict__ partial, int* __restrict__ tickets,
    int M, int N, int K, int splits) {
  __shared__ float red[(kWaves - 1) * kNT * MT * 4 * 64];
  __shared__ int last_flag;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nb = blockIdx.x;
  const int split = blockIdx.y;
  const int mchunk = blockIdx.z;
  const int NG = K / kGroup;
  const int c = lane & 15, kq = lane >> 4;
  const int m0 = mchunk * MT * 16;

  const int per_split = cdiv(NG, splits);
  const int g0 = split * per_split;
  const int g1 = min(NG, g0 + per_split);
  const int per_wave = cdiv(max(g1 - g0, 0), kWaves);
  const int wg0 = g0 + wave * per_wave;
  const int wg1 = min(g1, wg0 + per_wave);

  f32x4 acc[kNT][MT];
#pragma unroll
  for (int t = 0; t < kNT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const i32x4 negbias = {(int)Magic<DT>::kNegBiasPair, (int)Magic<DT>::kNegBiasPair,
                         (int)Magic<DT>::kNegBiasPair, (int)Magic<DT>::kNegBiasPair};

  // A row pointers (rows past M read nothing and feed zeros).
  const uint16_t* arow[MT];
  bool avalid[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    int row = m0 + mt * 16 + c;
    avalid[mt] = row < M;
    arow[mt] = A + (long)(avalid[mt] ? row : 0) * K + kq * 8;
  }
  const long tile0 = (long)nb * kNT;

  for (int g = wg0; g < wg1; ++g) {
    i32x4 wv[kNT];
    float s[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      long tg = (tile0 + t) * NG + g;
      wv[t] = __builtin_nontemporal_load(&Wp[tg * 64 + lane]);
      s[t] = load_act<DT>(Sp + tg * 16 + c);
    }
    i32x4 a[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        a[mt][j] = avalid[mt] ? *(const i32x4*)(arow[mt] + g * kGroup + j * 32)
                              : i32x4{0, 0, 0, 0};
    f32x4 nbias[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      nbias[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) nbias[mt] = mfma16x16x32<DT>(a[mt][j], negbias, nbias[mt]);
    }
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
      i32x4 b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = unpack8<DT>((uint32_t)wv[t][j]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f32x4 cc = nbias[mt];
#pragma unroll
        for (int j = 0; j < 4; ++j) cc = mfma16x16x32<DT>(a[mt][j], b[j], cc);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][mt][i] = __builtin_fmaf(s[t], cc[i], acc[t][mt][i]);
      }
    }
  }

  // ---- reduce the waves' partial sums through LDS: wave 0 adds waves 1..W-1
  // in order (deterministic) ----
  constexpr int kElems = kNT * MT * 4;  // per lane
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < kNT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          red[(((wave - 1) * kNT + t) * MT + mt) * 4 * 64 + i * 64 + lane] = acc[t][mt][i];
  }
  __syncthreads();

  const int nthreads = 64 * kWaves;
  const int col_base = nb * kNT * 16;
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < kNT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = acc[t][mt][i];
#pragma unroll
          for (int w = 1; w < kWaves; ++w)
            v += red[(((w - 1) * kNT + t) * MT + mt) * 4 * 64 + i * 64 + lane];
          const int row = m0 + mt * 16 + (lane >> 4) * 4 + i;
          const int col = col_base + t * 16 + (lane & 15);
          if (row < M) {
            if (splits == 1) out[(long)row * N + col] = to_bits<DT>(v);
            else partial[((long)split * M + row) * N + col] = v;
          }
        }
  }
  if (splits == 1) return;

  // ---- split-K: the last workgroup of this tile sums the splits in order ----
  __threadfence();
  __syncthreads();
  int* ticket = tickets + mchunk * gridDim.x + nb;
  if (threadIdx.x == 0) last_flag = (atomicAdd(ticket, 1) == splits - 1);
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
  const int rows = min(MT * 16, M - m0);
  for (int e = threadIdx.x; e < rows * kNT * 16; e += nthreads) {
    const int r = e / (kNT * 16);
    const int col = col_base + e % (kNT * 16);
    const long off = (long)(m0 + r) * N + col;
    float v = 0.f;
    for (int sp = 0; sp < splits; ++sp) v += __builtin_nontemporal_load(&partial[(long)sp * M * N + off]);
    out[off] = to_bits<DT>(v);
  }
  if (threadIdx.x == 0) atomicExch(ticket, 0);
}

struct Plan {
  int mt;       // 16-row tiles per M chunk
  int mchunks;  // grid z
  int nblocks;  // grid x
  int splits;   // grid y
};

static Plan make_plan(int M, int N, int K) {
  Plan p;
  p.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.mchunks = cdiv(M, p.mt * 16);
  p.nblocks = N / (kNT * 16);
  const int NG = K / kGroup;
  const int wgs = p.nblocks * p.mchunks;
  // Aim for >= 512 workgroups (2 per CU) while keeping >= 2 groups per wave.
  int s = cdiv(512, wgs);
  int smax = max(1, NG / (2 * kWaves));
  p.splits = max(1, min(s, smax));
  return p;
}

static size_t workspace_bytes(const Plan& p, int M, int N) {
  if (p.splits <= 1) return 0;
  size_t tickets = (size_t)p.nblocks * p.mchunks * sizeof(int);
  tickets = (tickets + 255) & ~(size_t)255;
  return tickets + (size_t)p.splits * M * N * sizeof(float);
}

}  // namespace int4
}  // namespace ti

using namespace ti;
using namespace ti::int4;

extern "C" size_t ti_int4_packed_weight_bytes(int K, int N) {
  if (K <= 0 || N <= 0) return 0;
  return (size_t)K * N / 2;
}

extern "C" size_t ti_int4_packed_scale_bytes(int K, int N, int group_size) {
  if (K <= 0 || N <= 0 || group_size <= 0) return 0;
  return (size_t)(K / group_size) * N * 2;
}

extern "C" int ti_int4_repack(const int32_t* qweight, const void* scales, int scale_dtype, int K,
                              int N, int group_size, int32_t* packed_weight, void* packed_scales,
                              hipStream_t stream) {
  TI_CHECK_ARG(qweight && scales && packed_weight && packed_scales, "ti_int4_repack: null pointer");
  TI_CHECK_ARG(scale_dtype == TI_DTYPE_F16 || scale_dtype == TI_DTYPE_BF16,
               "ti_int4_repack: scale dtype must be fp16 or bf16");
  TI_CHECK_SHAPE(group_size == kGroup, "ti_int4_repack: group_size must be 128 (got %d)", group_size);
  TI_CHECK_SHAPE(K > 0 && N > 0 && K % kGroup == 0 && N % 16 == 0,
                 "ti_int4_repack: need K %% 128 == 0 and N %% 16 == 0 (K=%d N=%d)", K, N);
  const int NG = K / kGroup;
  long wtotal = (long)(N / 16) * NG * 256;
  hipLaunchKernelGGL(repack_weight_kernel, dim3((unsigned)cdiv((int)((wtotal + 255) / 256), 1)),
                     dim3(256), 0, stream, (const uint32_t*)qweight, (uint32_t*)packed_weight, N,
                     NG, wtotal);
  TI_CHECK_LAUNCH("ti_int4_repack");
  long stotal = (long)(N / 16) * NG * 16;
  hipLaunchKernelGGL(repack_scale_kernel, dim3((unsigned)((stotal + 255) / 256)), dim3(256), 0,
                     stream, (const uint16_t*)scales, (uint16_t*)packed_scales, N, NG, stotal);
  TI_CHECK_LAUNCH("ti_int4_repack");
  return TI_OK;
}

extern "C" int ti_int4_dequant(const int32_t* packed_weight, const void* packed_scales,
                               int scale_dtype, int K, int N, int group_size, float* out,
                               hipStream_t stream) {
  TI_CHECK_ARG(packed_weight && packed_scales && out, "ti_int4_dequant: null pointer");
  TI_CHECK_ARG(scale_dtype == TI_DTYPE_F16 || scale_dtype == TI_DTYPE_BF16,
               "ti_int4_dequant: scale dtype must be fp16 or bf16");
  TI_CHECK_SHAPE(group_size == kGroup, "ti_int4_dequant: group_size must be 128");
  TI_CHECK_SHAPE(K > 0 && N > 0 && K % kGroup == 0 && N % 16 == 0,
                 "ti_int4_dequant: need K %% 128 == 0 and N %% 16 == 0");
  const long tiles = (long)(N / 16) * (K / kGroup);
  const int waves_per_block = 4;
  dim3 grid((unsigned)((tiles + waves_per_block - 1) / waves_per_block));
  if (scale_dtype == TI_DTYPE_F16)
    hipLaunchKernelGGL(dequant_kernel<TI_DTYPE_F16>, grid, dim3(64 * waves_per_block), 0, stream,
                       (const i32x4*)packed_weight, (const uint16_t*)packed_scales, out, N,
                       K / kGroup);
  else
    hipLaunchKernelGGL(dequant_kernel<TI_DTYPE_BF16>, grid, dim3(64 * waves_per_block), 0, stream,
                       (const i32x4*)packed_weight, (const uint16_t*)packed_scales, out, N,
                       K / kGroup);
  TI_CHECK_LAUNCH("ti_int4_dequant");
  return TI_OK;
}

extern "C" size_t ti_w4a16_workspace_bytes(int M, int N, int K, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size != kGroup || N % (kNT * 16) || K % kGroup) return 0;
  Plan p = make_plan(M, N, K);
  return workspace_bytes(p, M, N);
}

template <int DT, int MT>
static void launch_w4a16(const Plan& p, const void* a, const int32_t* w, const void* s, void* out,
                         float* partial, int* tickets, int M, int N, int K, hipStream_t stream) {
  hipLaunchKernelGGL((w4a16_gemm_kernel<DT, MT>), dim3(p.nblocks, p.splits, p.mchunks),
                     dim3(64 * kWaves), 0, stream, (const uint16_t*)a, (const i32x4*)w,
                     (const uint16_t*)s, (uint16_t*)out, partial, tickets, M, N, K, p.splits);
}

extern "C" int ti_w4a16_gemm(const void* a, int dtype, const int32_t* packed_weight,
                             const void* packed_scales, void* out, int M, int N, int K,
                             int group_size, void* workspace, size_t workspace_bytes_,
                             hipStream_t stream) {
  TI_CHECK_ARG(a && packed_weight && packed_scales && out, "ti_w4a16_gemm: null pointer");
  TI_CHECK_ARG(dtype == TI_DTYPE_F16 || dtype == TI_DTYPE_BF16,
               "ti_w4a16_gemm: dtype must be fp16 or bf16");
  TI_CHECK_SHAPE(group_size == kGroup, "ti_w4a16_gemm: group_size must be 128 (got %d)", group_size);
  TI_CHECK_SHAPE(M >= 1 && N > 0 && K > 0 && K % kGroup == 0 && N % (kNT * 16) == 0,
                 "ti_w4a16_gemm: need M >= 1, K %% 128 == 0, N %% 64 == 0 (M=%d N=%d K=%d)", M, N, K);
  TI_CHECK_ARG(((uintptr_t)a & 15) == 0 && ((uintptr_t)packed_weight & 15) == 0,
               "ti_w4a16_gemm: a and packed_weight must be 16-byte aligned");
  Plan p = make_plan(M, N, K);
  size_t need = workspace_bytes(p, M, N);
  float* partial = nullptr;
  int* tickets = nullptr;
  if (need) {
    if (!workspace || workspace_bytes_ < need) {
      set_error("ti_w4a16_gemm: workspace of %zu bytes required (got %zu)", need, workspace_bytes_);
      return TI_ERR_WORKSPACE;
    }
    size_t tb = ((size_t)p.nblocks * p.mchunks * sizeof(int) + 255) & ~(size_t)255;
    tickets = (int*)workspace;
    partial = (float*)((char*)workspace + tb);
  }
  if (dtype == TI_DTYPE_F16) {
    if (p.mt == 1) launch_w4a16<TI_DTYPE_F16, 1>(p, a, packed_weight, packed_scales, out, partial, tickets, M, N, K, stream);
    else if (p.mt == 2) launch_w4a16<TI_DTYPE_F16, 2>(p, a, packed_weight, packed_scales, out, partial, tickets, M, N, K, stream);
    else launch_w4a16<TI_DTYPE_F16, 4>(p, a, packed_weight, packed_scales, out, partial, tickets, M, N, K, stream);
  } else {
    if (p.mt == 1) launch_w4a16<TI_DTYPE_BF16, 1>(p, a, packed_weight, packed_scales, out, partial, tickets, M, N, K, stream);
    else if (p.mt == 2) launch_w4a16<TI_DTYPE_BF16, 2>(p, a, packed_weight, packed_scales, out, partial, tickets, M, N, K, stream);
    else launch_w4a16<TI_DTYPE_BF16, 4>(p, a, packed_weight, packed_scales, out, partial, tickets, M, N, K, stream);
  }
  TI_CHECK_LAUNCH("ti_w4a16_gemm");
  return TI_OK;
}
