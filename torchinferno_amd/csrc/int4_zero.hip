// Asymmetric zero points for the int4 W4A16 GEMM (GPTQ / AWQ checkpoints).
//
// With a per-(group, column) zero point z the weight is (q - z) * s.  Split as
// (q - 8) * s + (8 - z) * s: the first term is the symmetric weight every int4
// kernel computes; the second is a per-(group, column) offset zb[g, n], exact in
// fp32 (a small integer times a 16-bit scale).  Its contribution to the product
// is out[m, n] += sum_g rowsum_g(a[m]) * zb[g, n], where rowsum_g sums the 128
// activations of group g.  This kernel adds it to the symmetric GEMM's output
// (in fp32, then rounds once more to the output dtype).
#include "ti_common.h"

namespace ti {
namespace int4 {
namespace {

constexpr int kZpThreads = 256;
constexpr int kZpCols = kZpThreads * 4;  // columns per workgroup
constexpr int kZpMaxGroups = 1024;      // K <= 131072

// Workgroup (m, column chunk): the row's group sums into LDS (fp32, in K
// order within each group), then four columns per thread.
template <int DT>
__global__ __launch_bounds__(kZpThreads) void zero_point_kernel(const uint16_t* __restrict__ a,
                                                                const float* __restrict__ zb,
                                                                uint16_t* __restrict__ out, int N, int K) {
  __shared__ float rs[kZpMaxGroups];
  const int m = blockIdx.y;
  const int NG = K / 128;
  const uint16_t* ar = a + (long)m * K;
  // one wave per group: 64 lanes x 2 values, then a fixed-order tree
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int g = wave; g < NG; g += kZpThreads / 64) {
    const uint32_t w = *(const uint32_t*)(ar + g * 128 + lane * 2);
    float v = load_act<DT>((const uint16_t*)&w) + load_act<DT>((const uint16_t*)&w + 1);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if (lane == 0) rs[g] = v;
  }
  __syncthreads();
  const int n0 = blockIdx.x * kZpCols + threadIdx.x * 4;
  if (n0 >= N) return;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < NG; ++g) {
    const float4 z = *(const float4*)(zb + (long)g * N + n0);
    acc[0] = __builtin_fmaf(rs[g], z.x, acc[0]);
    acc[1] = __builtin_fmaf(rs[g], z.y, acc[1]);
    acc[2] = __builtin_fmaf(rs[g], z.z, acc[2]);
    acc[3] = __builtin_fmaf(rs[g], z.w, acc[3]);
  }
  uint16_t* o = out + (long)m * N + n0;
  const uint2 cur = *(const uint2*)o;
  const uint16_t h[4] = {(uint16_t)(cur.x & 0xFFFFu), (uint16_t)(cur.x >> 16), (uint16_t)(cur.y & 0xFFFFu),
                         (uint16_t)(cur.y >> 16)};
  uint16_t r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = to_bits<DT>(load_act<DT>(&h[i]) + acc[i]);
  *(uint2*)o = make_uint2(r[0] | ((uint32_t)r[1] << 16), r[2] | ((uint32_t)r[3] << 16));
}

}  // namespace
}  // namespace int4
}  // namespace ti

using namespace ti;
using namespace ti::int4;

extern "C" int ti_w4a16_zero_point_add(const void* a, int dtype, const float* zero_offset, void* out, int M,
                                       int N, int K, hipStream_t stream) {
  TI_CHECK_ARG(a && zero_offset && out, "ti_w4a16_zero_point_add: null pointer");
  TI_CHECK_ARG(dtype == TI_DTYPE_F16 || dtype == TI_DTYPE_BF16, "ti_w4a16_zero_point_add: dtype must be fp16 or bf16");
  TI_CHECK_SHAPE(M >= 0 && N > 0 && N % 4 == 0 && K > 0 && K % 128 == 0 && K / 128 <= kZpMaxGroups,
                 "ti_w4a16_zero_point_add: need N %% 4 == 0, K %% 128 == 0, K <= 131072 (N=%d K=%d)", N, K);
  TI_CHECK_ARG(((uintptr_t)a & 3) == 0 && ((uintptr_t)zero_offset & 15) == 0 && ((uintptr_t)out & 7) == 0,
               "ti_w4a16_zero_point_add: a must be 4-byte, zero_offset 16-byte and out 8-byte aligned");
  if (M == 0) return TI_OK;
  dim3 grid((unsigned)((N + kZpCols - 1) / kZpCols), (unsigned)M);
  if (dtype == TI_DTYPE_F16)
    hipLaunchKernelGGL(zero_point_kernel<TI_DTYPE_F16>, grid, dim3(kZpThreads), 0, stream, (const uint16_t*)a,
                       zero_offset, (uint16_t*)out, N, K);
  else
    hipLaunchKernelGGL(zero_point_kernel<TI_DTYPE_BF16>, grid, dim3(kZpThreads), 0, stream, (const uint16_t*)a,
                       zero_offset, (uint16_t*)out, N, K);
  TI_CHECK_LAUNCH("ti_w4a16_zero_point_add");
  return TI_OK;
}
