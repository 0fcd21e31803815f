// Internal interface of the FP8 GEMM kernel (fp8_gemm.hip).
#pragma once

#include "ti_common.h"

namespace ti {
namespace fp8 {

constexpr int kNumKinds = 7;

struct GemmArgs {
  const uint8_t* a;   // [M, K] e4m3
  const uint8_t* b;   // [N, K] e4m3
  const float* sa;    // row scales (SMODE 0, stride sa_stride) or [M, K/128] (SMODE 1)
  const float* sb;    // column scales (SMODE 0, stride sb_stride) or [ceil(N/128), K/128]
  int sa_stride, sb_stride;
  uint16_t* out;      // [M, N] bf16 / fp16
  float* partial;     // split-K fp32 partials [splits][M][N]
  int* tickets;       // one per tile, zero between calls
  int M, N, K;
  int splits, tiles_m, tiles_n;
};

struct GemmPlan {
  int kind;     // tile configuration (fp8_gemm.hip)
  int tiles_m, tiles_n;
  int splits;
};

GemmPlan make_gemm_plan(int M, int N, int K, int smode);
size_t gemm_workspace_bytes(const GemmPlan& p, int M, int N);
size_t gemm_ticket_bytes(const GemmPlan& p);
void launch_gemm(const GemmPlan& p, int smode, int odt, const GemmArgs& x, hipStream_t stream);

}  // namespace fp8
}  // namespace ti
