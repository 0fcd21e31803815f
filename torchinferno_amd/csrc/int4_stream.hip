// int4 W4A16 streaming kernel for skinny M (decode, M <= 32) on gfx950.
//
// Same arithmetic and weight layout as int4_gemm.hip (1 KiB blocks of 16
// columns x one 128-row group, in-register magic-number unpack, MFMA sums of
// exact biased integers corrected by a per-group activation row sum, group
// scale applied in fp32), organised for HBM streaming at small M:
//
//   * Balance.  A workgroup owns NT column tiles and one of `splits` K ranges;
//     the host picks NT and splits so that the grid is a multiple of the 256
//     CUs and every workgroup streams the same number of bytes (gate_up
//     N=28672: 7 tiles, no split; N=4096: 1 tile x all K or 4 tiles x K/4),
//     and the dynamic LDS size keeps one workgroup per CU.
//   * Bytes in flight.  Weights and activation fragments travel in a ring of
//     D register stages per wave (global loads straight to VGPRs, no LDS), so
//     a CU keeps W * D * NT KiB of weights in flight -- far more than an LDS
//     ring of the same depth could hold.  Loads are unconditional (group index
//     clamped, a group past the wave's range contributes with scale 0), which
//     keeps the compiler's in-order vmcnt accounting exact across the loop.
//   * Scales travel in the ring too (one dword per lane per group, handed to
//     the lanes that need them by a cross-lane shuffle), so no wave waits on
//     a prologue: each starts computing when its own first stage lands.
//   * Wave w of a workgroup takes groups g0 + w, g0 + w + W, ...: at any moment
//     the workgroup reads W adjacent groups of its tiles.
//   * Epilogue: every wave's fp32 partial goes to LDS; each output fragment is
//     summed over the waves in wave order by one wave.  Split partials are
//     summed in split order by the last-arriving workgroup of a column chunk
//     (agent-scope stores/loads and a ticket, as int4_gemm.hip).  Results are
//     deterministic.
#include "int4_stream.h"

// Timeline hook for profiling builds (per-wave timestamps); empty in the library.
#ifndef TI_STREAM_MARK
#define TI_STREAM_MARK(k)
#endif

namespace ti {
namespace int4 {
namespace {

template <int MT, int NT>
struct SStage {
  i32x4 w[NT];
  i32x4 a[MT][4];
  uint32_t s;  // scales of columns col0 + 2*lane, +1 of the stage's group
};

// One ring stage: the wave's NT weight blocks of group g, its activation
// fragments, and the group's NT*16 scales (one dword per lane, lanes past the
// workgroup's columns re-read the last dword).
template <int MT, int NT>
__device__ __forceinline__ void load_sstage(SStage<MT, NT>& st, const i32x4* __restrict__ Wp,
                                            const uint16_t* const (&arow)[MT], const uint32_t* __restrict__ srow,
                                            long tile0, long T, int N, int g, int lane) {
#pragma unroll
  for (int t = 0; t < NT; ++t) st.w[t] = __builtin_nontemporal_load(&Wp[((long)g * T + tile0 + t) * 64 + lane]);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) st.a[mt][j] = *(const i32x4*)(arow[mt] + (long)g * kGroup + j * 32);
  st.s = srow[(long)g * (N / 2) + min(lane, NT * 8 - 1)];
}

template <int DT, int MT, int NT, int W, int D, int SPLIT>
__global__ __launch_bounds__(64 * W) void w4a16_stream_kernel(
    const uint16_t* __restrict__ A, const i32x4* __restrict__ Wp, const uint16_t* __restrict__ Sg,
    uint16_t* __restrict__ out, float* __restrict__ partial, int* __restrict__ tickets, int M, int N, int K,
    int splits) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int last_flag;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nb = blockIdx.x, split = blockIdx.y, mchunk = blockIdx.z;
  const int NG = K / kGroup;
  const long T = N / 16;
  const int c = lane & 15;
  const int m0 = mchunk * MT * 16;
  const int rows = min(MT * 16, M - m0);
  const long tile0 = (long)nb * NT;
  const int col0 = nb * NT * 16;

  const int per_split = cdiv(NG, splits);
  const int g0 = split * per_split;
  const int ngr = max(min(NG, g0 + per_split) - g0, 0);
  const int mine = ngr > wave ? cdiv(ngr - wave, W) : 0;  // groups of this wave
  const int nit = cdiv(mine, D);
  TI_STREAM_MARK(0);

  // Rows past M re-read the last row: MFMA rows are independent and those
  // output rows are never stored.
  const uint16_t* arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    arow[mt] = A + (long)(m0 + min(mt * 16 + c, rows - 1)) * K + (lane >> 4) * 8;

  const uint32_t* srow = (const uint32_t*)(Sg + col0);  // scale dwords of the workgroup's columns

  // Ring prologue: the wave's first D groups.
  auto gidx = [&](int i) {  // global group of the wave's i-th group, clamped into range
    const int li = min(wave + i * W, max(ngr - 1, 0));
    return g0 + li;
  };
  SStage<MT, NT> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d) load_sstage<MT, NT>(ring[d], Wp, arow, srow, tile0, T, N, gidx(d), lane);
  TI_STREAM_MARK(1);

  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](int it, bool reload) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = it * D + d;
      const bool valid = i < mine;
      float sc[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {  // column t*16 + c sits in lane t*8 + c/2, half c&1
        const uint32_t pair = (uint32_t)__shfl((int)ring[d].s, t * 8 + (c >> 1), 64);
        const float v = scale_to_f32<DT>((c & 1) ? pair >> 16 : pair & 0xFFFFu);
        sc[t] = valid ? v : 0.f;
      }
      compute_group<DT, MT, NT>(ring[d].w, ring[d].a, sc, acc);
      if (reload) load_sstage<MT, NT>(ring[d], Wp, arow, srow, tile0, T, N, gidx(i + D), lane);
      // Keep the stages in order: without this the scheduler hoists later
      // stages' MFMAs (e.g. their bias sums) into this one, and the vmcnt wait
      // they need drains the whole ring.
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int it = 0; it + 1 < nit; ++it) step(it, true);
  if (nit > 0) step(nit - 1, false);
  TI_STREAM_MARK(2);

  // ---- wave partials -> LDS; fragment f = (t, mt) summed over waves in order ----
  float* red = (float*)smem;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[((wave * NT + t) * MT + mt) * 256 + i * 64 + lane] = acc[t][mt][i];
  __syncthreads();
  for (int f = wave; f < NT * MT; f += W) {
    const int t = f / MT, mt = f % MT;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) v += red[((w * NT + t) * MT + mt) * 256 + i * 64 + lane];
      const int row = m0 + mt * 16 + (lane >> 4) * 4 + i;
      const int col = col0 + t * 16 + c;
      if (row < M) {
        if (SPLIT == 0) out[(long)row * N + col] = to_bits<DT>(v);
        else __hip_atomic_store(&partial[((long)split * M + row) * N + col], v, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  TI_STREAM_MARK(3);
  if (SPLIT == 0) return;

  // Partials are written through once vmcnt drains; then the ticket.  The last
  // workgroup of the column chunk sums the splits in order and resets it.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* ticket = tickets + mchunk * gridDim.x + nb;
  if (threadIdx.x == 0)
    last_flag = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
  __syncthreads();
  if (!last_flag) return;
  for (int e = threadIdx.x; e < rows * NT * 16; e += 64 * W) {
    const int r = e / (NT * 16);
    const long off = (long)(m0 + r) * N + col0 + e % (NT * 16);
    float v = 0.f;
    for (int sp = 0; sp < splits; ++sp)
      v += __hip_atomic_load(&partial[(long)sp * M * N + off], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out[off] = to_bits<DT>(v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Instantiated configurations (MT, NT, W, D).
#define TI_STREAM_CONFIGS(X) \
  X(1, 7, 8, 2)              \
  X(2, 7, 8, 2)              \
  X(1, 7, 16, 1)             \
  X(1, 2, 8, 4)              \
  X(1, 4, 8, 2)              \
  X(2, 4, 16, 1)             \
  X(1, 1, 8, 4)              \
  X(1, 1, 16, 2)             \
  X(2, 2, 16, 1)

bool config_instantiated(int mt, int nt, int w, int d) {
#define TI_X(MT, NT, W, D) \
  if (mt == MT && nt == NT && w == W && d == D) return true;
  TI_STREAM_CONFIGS(TI_X)
#undef TI_X
  return false;
}

int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return (e && *e) ? atoi(e) : dflt;
}

}  // namespace

// Plans measured on MI355X (Llama-3-8B MLP gate_up/down and q/o-proj shapes,
// HIP-event timed over rotating weight copies); where the register-ring or
// LDS-DMA kernel of int4_gemm.hip / int4_decode.hip measured faster, this
// returns false and they run.
bool make_stream_plan(int M, int N, int K, StreamPlan& p) {
  if (env_int("TI_ROCM_W4A16_STREAM_OFF", 0)) return false;
  if (M < 1 || M > 32 || N % 16 || K % kGroup) return false;
  const int T = N / 16, NG = K / kGroup;
  p.mt = M <= 16 ? 1 : 2;
  p.mchunks = 1;
  p.waves = 8;
  p.depth = 2;
  p.splits = 1;
  const bool forced = getenv("TI_ROCM_W4A16_STREAM") && *getenv("TI_ROCM_W4A16_STREAM");
  if (T % 7 == 0 && T / 7 >= 192) {          // wide N: 7 tiles per workgroup, no split
    if (M < 8 && !forced) return false;
    p.nt = 7;
  } else if (T == 256 && NG >= 64) {         // narrow N, deep K: split K over 4-tile chunks
    if (M <= 4 && !forced) return false;
    if (M <= 8) { p.nt = 2; p.depth = 4; p.splits = 2; }
    else if (M <= 16) { p.nt = 4; p.splits = 4; }
    else { p.nt = 4; p.waves = 16; p.depth = 1; p.splits = 4; }
  } else if (T == 256) {                     // narrow N, short K: one tile per workgroup
    p.nt = 1;
    if (M == 1) { p.waves = 16; p.depth = 2; }
    else if (M <= 16) { p.depth = 4; }
    else { p.nt = 2; p.waves = 16; p.depth = 1; p.splits = 2; }
  } else if (!forced) {
    return false;
  } else {
    p.nt = 1;
  }
  const char* e = getenv("TI_ROCM_W4A16_STREAM");
  if (e && *e) {
    int nt, w, d, s;
    if (sscanf(e, "%d:%d:%d:%d", &nt, &w, &d, &s) == 4) {
      p.nt = nt; p.waves = w; p.depth = d; p.splits = s;
    }
  }
  if (!config_instantiated(p.mt, p.nt, p.waves, p.depth) || T % p.nt) return false;
  p.splits = max(1, min(p.splits, NG));
  const int per = cdiv(NG, p.splits);
  p.splits = cdiv(NG, per);  // no empty K range
  p.nblocks = T / p.nt;
  const int ngr = per;
  (void)ngr;
  const int red = p.waves * p.nt * p.mt * 1024;
  // At least 81 KiB keeps one workgroup per CU (two would not fit in 160 KiB).
  p.lds = max(red, env_int("TI_ROCM_W4A16_STREAM_LDS", 81 * 1024));
  return true;
}

size_t stream_partial_bytes(const StreamPlan& p, int M, int N) {
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

size_t stream_ticket_bytes(const StreamPlan& p) {
  return ((size_t)p.nblocks * p.mchunks * sizeof(int) + 255) & ~(size_t)255;
}

template <int DT, int MT, int NT, int W, int D>
static void launch_cfg(const StreamPlan& p, const StreamArgs& x, hipStream_t stream) {
  dim3 grid(p.nblocks, p.splits, p.mchunks);
  if (p.splits == 1)
    hipLaunchKernelGGL((w4a16_stream_kernel<DT, MT, NT, W, D, 0>), grid, dim3(64 * W), p.lds, stream, x.a, x.w,
                       x.s, x.out, x.partial, x.tickets, x.M, x.N, x.K, 1);
  else
    hipLaunchKernelGGL((w4a16_stream_kernel<DT, MT, NT, W, D, 2>), grid, dim3(64 * W), p.lds, stream, x.a, x.w,
                       x.s, x.out, x.partial, x.tickets, x.M, x.N, x.K, p.splits);
}

void launch_stream(const StreamPlan& p, int dtype, const StreamArgs& x, hipStream_t stream) {
#define TI_X(MT, NT, W, D)                                                              \
  if (p.mt == MT && p.nt == NT && p.waves == W && p.depth == D) {                       \
    if (dtype == TI_DTYPE_F16) launch_cfg<TI_DTYPE_F16, MT, NT, W, D>(p, x, stream);    \
    else launch_cfg<TI_DTYPE_BF16, MT, NT, W, D>(p, x, stream);                         \
    return;                                                                             \
  }
  TI_STREAM_CONFIGS(TI_X)
#undef TI_X
}

}  // namespace int4
}  // namespace ti
