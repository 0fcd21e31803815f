// Internal interface of the FP8 GEMM kernel (fp8_gemm.hip).
#pragma once

#include "ti_common.h"

namespace ti {
namespace fp8 {

constexpr int kNumKinds = 24;

struct GemmArgs {
  const uint8_t* a;   // [M, K] e4m3
  const uint8_t* b;   // [N, K] e4m3
  const float* sa;    // row scales (SMODE 0, stride sa_stride) or [M, K/128] (SMODE 1)
  const float* sb;    // column scales (SMODE 0, stride sb_stride), [ceil(N/128), K/128] (SMODE 1),
                      // or e8m0 bytes [N, K/32] (SMODE 2)
  int sa_stride, sb_stride;
  uint16_t* out;      // [M, N] bf16 / fp16
  float* partial;     // split-K fp32 partials [splits][M][N]
  int* tickets;       // one per tile, zero between calls
  int M, N, K;
  int splits, tiles_m, tiles_n;
  int group_m;        // tile rows per raster group
  // Gather / grouped (MoE) mode:
  const int* row_index;     // A (and block-mode sa) row of output row p; nullptr = p
  int grouped;              // 1: m-tiles come from the device tables below
  const int* tile_expert;   // [max m-tiles] expert of each m-tile
  const int* tile_row0;     // first output row of each m-tile
  const int* tile_rows;     // rows of each m-tile (<= BM)
  const int* num_mtiles;    // device scalar: m-tiles in use
  long b_expert_stride;     // bytes between experts' [N, K] weights
  long sb_expert_stride;    // 4-byte units between experts' weight-scale grids
  int sb_layout;            // SMODE 2: 0 = e8m0 [N, K/32]; 1 = step-major [K/128][N][4]
  int sa_layout;            // SMODE 1/2: 0 = [M, K/128]; 1 = step-major [K/128][M]
  int b_tiled;              // 1: B in tiles of 128 rows x 128 K, [N/128][K/128][128][128] (e4m3)
};

struct GemmPlan {
  int kind;     // tile configuration (fp8_gemm.hip)
  int tiles_m, tiles_n;
  int splits;
  int group_m;
};

GemmPlan make_gemm_plan(int M, int N, int K, int smode);
size_t gemm_workspace_bytes(const GemmPlan& p, int M, int N);
size_t gemm_ticket_bytes(const GemmPlan& p);
void launch_gemm(const GemmPlan& p, int smode, int odt, const GemmArgs& x, hipStream_t stream);

// Grouped block-scaled GEMM (bf16 out) over a device m-tile table; kind is one
// of 2-5, 9-13, 15-20, and 14 with power-of-two block scales
// (the tile configurations of fp8_gemm.hip).
int grouped_bm(int kind);
int grouped_bn(int kind);
void launch_gemm_grouped(int kind, int smode, const GemmArgs& x, int max_mtiles, hipStream_t stream);

}  // namespace fp8
}  // namespace ti
