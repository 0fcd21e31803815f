// Internal interface of the int4 W4A16 decode kernel (int4_decode.hip), used by
// the ti_w4a16_gemm dispatcher in int4_gemm.hip.
#pragma once

#include "int4_common.h"

namespace ti {
namespace int4 {

constexpr int kDecodeLdsMax = 160 * 1024 - 256;  // gfx950 LDS per workgroup, less static LDS

struct DecodePlan {
  int mr;       // activation rows staged per K range and stage (4, 16, 32, 64, 128)
  int nt;       // 16-column tiles per wave
  int wk;       // waves splitting K inside the workgroup
  int waves;    // waves per workgroup (4, or 8 for tall tiles: two per SIMD)
  int ring;     // LDS ring stages
  int splits;   // K splits across workgroups
  int mchunks;  // row chunks (grid z)
  int nblocks;  // column blocks (grid x)
  int lds;      // dynamic LDS bytes
};

struct DecodeArgs {
  const uint16_t* a;
  const i32x4* w;
  const uint16_t* s;
  uint16_t* out;
  float* partial;
  int* tickets;
  int M, N, K;
};

DecodePlan make_decode_plan(int M, int N, int K);
// The plan names an instantiated kernel whose workgroups tile N exactly.
bool decode_plan_valid(const DecodePlan& p, int N);
size_t decode_ticket_bytes(const DecodePlan& p);
size_t decode_partial_bytes(const DecodePlan& p, int M, int N);
void launch_decode(const DecodePlan& p, int dtype, const DecodeArgs& x, hipStream_t stream);

}  // namespace int4
}  // namespace ti
