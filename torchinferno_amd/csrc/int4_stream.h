// Internal interface of the skinny-M int4 W4A16 streaming kernel
// (int4_stream.hip), used by the ti_w4a16_gemm dispatcher in int4_gemm.hip.
#pragma once

#include "int4_common.h"

namespace ti {
namespace int4 {

struct StreamPlan {
  int mt;       // 16-row MFMA tiles per row chunk (1 or 2)
  int nt;       // 16-column tiles per workgroup
  int waves;    // waves per workgroup (they split the workgroup's K range)
  int depth;    // groups each wave keeps in flight (register ring stages)
  int splits;   // K ranges across workgroups
  int mchunks;  // row chunks (grid z)
  int nblocks;  // column chunks (grid x)
  int lds;      // dynamic LDS bytes
};

struct StreamArgs {
  const uint16_t* a;
  const i32x4* w;
  const uint16_t* s;
  uint16_t* out;
  float* partial;
  int* tickets;
  int M, N, K;
};

// A plan for this problem, or false when the streaming kernel does not take it
// (then the other int4 kernels do).
bool make_stream_plan(int M, int N, int K, StreamPlan& p);
size_t stream_partial_bytes(const StreamPlan& p, int M, int N);
size_t stream_ticket_bytes(const StreamPlan& p);
void launch_stream(const StreamPlan& p, int dtype, const StreamArgs& x, hipStream_t stream);

}  // namespace int4
}  // namespace ti
