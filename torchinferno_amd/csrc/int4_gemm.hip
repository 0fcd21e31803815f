// int4 W4A16 group-128 dequant-GEMM for gfx950 (CDNA4).
//
// Replaces Marlin's marlin_gemm as used by the reference's marlin_int4_mm
// (src/torchinferno/kernels/marlin.py:142-171): out[M,N] = a[M,K] @ W[K,N],
// W[k,n] = (q[k,n] - 8) * s[k/128, n], fp32 accumulation.
//
// Kernel weight layout.  The weight is cut into blocks of 16 output columns
// (a "tile") x 128 rows of K (one quantization group).  A block is 1 KiB and
// one wave reads it with one 16-byte load per lane: lane l = 16*kq + c holds
// column c, and its dword j holds the 8 codes at k = 128*g + 32*j + 8*kq + e
// (e = 0..7) -- exactly the B operand lane l feeds to step j of
// v_mfma_f32_16x16x32_{f16,bf16}.  The A operand uses the same (j, kq, e) -> k
// map, so the MFMA computes the true dot product whatever order the hardware
// assigns to the 32 K slots.  Inside a dword, nibble p holds element e = 2p
// (p < 4) or e = 2(p-4)+1, so (w >> 4p) & 0x000F000F puts elements (2p, 2p+1)
// in the low/high halves.  Blocks are stored group-major (block (g, t) at
// g*N/16 + t): at any moment the waves of the grid stream one contiguous
// region of HBM, which keeps DRAM pages open.  Scales stay [K/128, N].
//
// Unpack: OR-ing a nibble into the mantissa of a magic constant gives an exact
// biased value (fp16: 0x6400|q = 1024+q, bf16: 0x4300|q = 128+q) -- one
// v_and_or_b32 per two weights plus a shift.  The bias is removed exactly in
// fp32 by starting each group's accumulator at -(bias+8) * rowsum(a), itself
// one MFMA against a constant operand per step that all column tiles share.
// The group's scale is then applied in fp32: acc += s * group_sum.  Weights
// enter the MFMA as exact integers (no fp16 rounding of (q-8)*s).
//
// Work split: a workgroup of W waves owns NT column tiles (16*NT columns) and
// a range of groups (the whole K, or one of `splits` K ranges); its waves split
// that range.  A prologue stages the workgroup's A rows and scales in LDS, so
// the main loop issues only weight loads on the (in-order) vmcnt counter; each
// wave keeps a ring of D groups of them in flight and reads A and scales with
// ds_reads.  When the A slice does not fit in LDS, A fragments travel in the
// same ring instead.  Wave partials are reduced through LDS in a fixed order;
// split partials are summed in split order by the last workgroup of the tile
// (or by a second kernel), so results are deterministic and nothing is memset.
#include "int4_decode.h"
#include "int4_stream.h"

namespace ti {
namespace int4 {

constexpr int kLdsBudget = 48 * 1024;  // A + scales staged per workgroup

__device__ __forceinline__ uint32_t interleave_nibbles(uint32_t w) {
  uint32_t r = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    int p = (e & 1) ? 4 + (e >> 1) : (e >> 1);
    r |= ((w >> (4 * e)) & 0xFu) << (4 * p);
  }
  return r;
}

// Canonical [K/8, N] -> group-major block layout; one thread per output dword.
__global__ void repack_weight_kernel(const uint32_t* __restrict__ q, uint32_t* __restrict__ out,
                                     int N, long total) {
  long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int T = N / 16;
  int j = idx & 3;
  int lane = (idx >> 2) & 63;
  long blk = idx >> 8;
  int t = (int)(blk % T);
  long g = blk / T;
  int c = lane & 15, kq = lane >> 4;
  long krow = g * 16 + j * 4 + kq;  // canonical word row: k/8
  out[idx] = interleave_nibbles(q[krow * N + t * 16 + c]);
}

// Symmetric RTN int4 quantization of a [K, N] weight into the canonical
// layout: the quantizer of src/torchinferno/kernels/marlin.py:117-128.  Per
// (128-row group, column): w is first rounded to fp16 (as the reference casts
// the weight), s = max(|max/7|, |min/-8|) clamped >= 1e-8 in fp32 (IEEE
// division), q = clamp(rint(w / s), -8, 7) + 8 (round half to even), scales
// stored RNE in the scale dtype.  One thread per (group, column).
template <int WDT, int SDT>
__global__ void quantize_rtn_kernel(const uint16_t* __restrict__ w, int K, int N,
                                    uint32_t* __restrict__ q, uint16_t* __restrict__ s) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int NG = K / kGroup;
  if (idx >= (long)NG * N) return;
  const int n = (int)(idx % N);
  const int g = (int)(idx / N);
  const uint16_t* col = w + (long)g * kGroup * N + n;
  float v[kGroup];
  float mx = -INFINITY, mn = INFINITY;
#pragma unroll 8
  for (int i = 0; i < kGroup; ++i) {
    const float f = WDT == TI_DTYPE_F16 ? f16_bits_to_f32(col[(long)i * N]) : bf16_bits_to_f32(col[(long)i * N]);
    v[i] = (float)(_Float16)f;  // round to fp16 (subnormals kept)
    mx = fmaxf(mx, v[i]);
    mn = fminf(mn, v[i]);
  }
  float sc = fmaxf(fabsf(mx / 7.0f), fabsf(mn / -8.0f));
  sc = fmaxf(sc, 1e-8f);
#pragma unroll
  for (int r = 0; r < kGroup / 8; ++r) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float c = __builtin_rintf(v[r * 8 + e] / sc);
      c = fminf(fmaxf(c, -8.0f), 7.0f);
      word |= (uint32_t)((int)c + 8) << (4 * e);
    }
    q[((long)g * (kGroup / 8) + r) * N + n] = word;
  }
  s[(long)g * N + n] = SDT == TI_DTYPE_F16 ? f32_to_f16_bits(sc) : f32_to_bf16_bits(sc);
}

// Exact dequant of the block layout, through the same unpack8: one wave per block.
template <int DT>
__global__ void dequant_kernel(const i32x4* __restrict__ wp, const uint16_t* __restrict__ sp,
                               float* __restrict__ out, int N, int NG) {
  const int lane = threadIdx.x & 63;
  const int T = N / 16;
  const long blk = (long)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (blk >= (long)T * NG) return;
  const int t = (int)(blk % T);
  const long g = blk / T;
  const int c = lane & 15, kq = lane >> 4;
  const float s = scale_to_f32<DT>(sp[g * N + t * 16 + c]);
  const i32x4 w = wp[blk * 64 + lane];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    i32x4 b = unpack8<DT>((uint32_t)w[j], 0x000F000Fu, Magic<DT>::kOr);
#pragma unroll
    for (int h = 0; h < 8; ++h) {
      uint16_t bits = (uint16_t)(((uint32_t)b[h >> 1]) >> (16 * (h & 1)));
      float q = scale_to_f32<DT>(bits) - Magic<DT>::kBias;  // q - 8, exact
      long k = g * kGroup + j * 32 + kq * 8 + h;
      out[k * N + t * 16 + c] = q * s;
    }
  }
}

// One ring stage: the wave's weight blocks for one group (16 B per lane per
// tile), plus the A fragments when A is not staged in LDS.
template <int MT, int NT, bool ALDS>
struct Stage {
  i32x4 w[NT];
  i32x4 a[ALDS ? 1 : MT][4];
};

template <int MT, int NT, bool ALDS>
__device__ __forceinline__ void load_stage(Stage<MT, NT, ALDS>& st, const i32x4* __restrict__ Wp,
                                           const uint16_t* const (&arow)[MT], long tile0, long T,
                                           int g, int lane) {
#pragma unroll
  for (int t = 0; t < NT; ++t) st.w[t] = __builtin_nontemporal_load(&Wp[((long)g * T + tile0 + t) * 64 + lane]);
  if constexpr (!ALDS) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) st.a[mt][j] = *(const i32x4*)(arow[mt] + g * kGroup + j * 32);
  }
}

// LDS layout of one workgroup (dynamic shared memory):
//   [A rows: rows x astride halves][scales: groups x 16*NT halves]  (main loop)
//   [W-1 wave partials]                                              (epilogue)
__host__ __device__ inline int a_stride(int groups) { return groups * kGroup + 8; }  // +16 B: bank skew

// SPLIT: 0 = the workgroup owns all of K and writes `out`;
//        1 = writes its fp32 partial; w4a16_reduce_kernel then sums the splits;
//        2 = writes its partial with agent-scope (L2 write-through) stores, waits
//            for them, takes a ticket; the last workgroup of the tile reads the
//            partials with agent-scope loads, sums them in split order, writes
//            `out` and resets the ticket.  One kernel, deterministic, and no
//            L2 writeback: the per-XCD L2s are bypassed for exactly the partials.
//            (A __threadfence()-based fix-up costs ~100 us per call on MI355X,
//            since an agent-scope release writes back each XCD's whole L2.)
// D = depth of the register ring of group loads each wave keeps in flight.
// ALDS = A staged in LDS (else A fragments ride in the ring).
template <int DT, int MT, int NT, int W, int D, int SPLIT, bool ALDS>
__global__ __launch_bounds__(64 * W) void w4a16_gemm_kernel(
    const uint16_t* __restrict__ A, const i32x4* __restrict__ Wp, const uint16_t* __restrict__ Sg,
    uint16_t* __restrict__ out, float* __restrict__ partial, int* __restrict__ tickets, int M, int N,
    int K, int splits) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int last_flag;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar
  const int nb = blockIdx.x;
  const int split = blockIdx.y;
  const int mchunk = blockIdx.z;
  const int NG = K / kGroup;
  const long T = N / 16;
  const int c = lane & 15, kq = lane >> 4;
  const int m0 = mchunk * MT * 16;
  const int rows = min(MT * 16, M - m0);
  const long tile0 = (long)nb * NT;
  const int col_base = nb * NT * 16;

  const int per_split = cdiv(NG, splits);
  const int g0 = split * per_split;
  const int g1 = min(NG, g0 + per_split);
  const int ngr = max(g1 - g0, 0);
  const int per_wave = cdiv(ngr, W);
  const int wg0 = g0 + wave * per_wave;
  const int wg1 = min(g1, wg0 + per_wave);

  const int astride = a_stride(ngr);
  uint16_t* sA = (uint16_t*)smem;
  uint16_t* sS = sA + (ALDS ? rows * astride : 0);

  // A sources.  Rows past M re-read the last row: MFMA rows are independent and
  // those output rows are never stored, so no masking is needed.
  const uint16_t* arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = min(mt * 16 + c, rows - 1);
    arow[mt] = ALDS ? sA + r * astride + kq * 8 : A + (long)(m0 + r) * K + kq * 8;
  }

  // The first D groups of weights go out before the LDS staging, so the
  // staging's latency overlaps theirs.
  // Every wave runs nit = ceil(n / D) iterations of D groups with
  // unconditional loads (group index clamped into [0, NG)); a group past wg1
  // contributes with scale 0.  Unconditional loads keep the in-order vmcnt
  // bookkeeping exact across the loop back-edge, so the compiler waits for one
  // ring stage at a time instead of draining the ring every group.
  const int nwg = max(wg1 - wg0, 0);
  const int nit = cdiv(nwg, D);
  const int gclamp = max(min(wg1, NG) - 1, 0);
  Stage<MT, NT, ALDS> ring[D];
#pragma unroll
  for (int d = 0; d < D; ++d)
    load_stage<MT, NT, ALDS>(ring[d], Wp, arow, tile0, T, min(wg0 + d, gclamp), lane);

  // ---- stage A rows [m0, m0+rows) x groups [g0, g1) and the scales in LDS ----
  {
    const int sq = NT * 2;  // 16-byte chunks per group row of scales (16*NT halves)
    for (int i = threadIdx.x; i < ngr * sq; i += 64 * W) {
      const int gi = i / sq, q = i % sq;
      *(i32x4*)(sS + gi * NT * 16 + q * 8) = *(const i32x4*)(Sg + (long)(g0 + gi) * N + col_base + q * 8);
    }
    if constexpr (ALDS) {
      const int aq = ngr * (kGroup / 8);  // 16-byte chunks per A row
      for (int i = threadIdx.x; i < rows * aq; i += 64 * W) {
        const int r = i / aq, q = i % aq;
        *(i32x4*)(sA + r * astride + q * 8) =
            *(const i32x4*)(A + (long)(m0 + r) * K + (long)g0 * kGroup + q * 8);
      }
    }
  }
  __syncthreads();

  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](int it, bool reload) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int g = wg0 + it * D + d;
      const int gs = min(g, gclamp) - g0;  // staged-scale / A row index (clamped)
      float sc[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const float v = scale_to_f32<DT>(sS[max(gs, 0) * NT * 16 + t * 16 + c]);
        sc[t] = g < wg1 ? v : 0.f;
      }
      if constexpr (ALDS) {
        i32x4 a[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < 4; ++j) a[mt][j] = *(const i32x4*)(arow[mt] + max(gs, 0) * kGroup + j * 32);
        compute_group<DT, MT, NT>(ring[d].w, a, sc, acc);
      } else {
        compute_group<DT, MT, NT>(ring[d].w, ring[d].a, sc, acc);
      }
      if (reload) load_stage<MT, NT, ALDS>(ring[d], Wp, arow, tile0, T, min(g + D, gclamp), lane);
    }
  };
  for (int it = 0; it + 1 < nit; ++it) step(it, true);
  if (nit > 0) step(nit - 1, false);

  // ---- reduce the waves' partial sums through LDS: wave 0 adds waves 1..W-1
  // in order (deterministic).  The staging area is reused. ----
  float* red = (float*)smem;
  if (W > 1) {
    __syncthreads();
    if (wave > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            red[(((wave - 1) * NT + t) * MT + mt) * 4 * 64 + i * 64 + lane] = acc[t][mt][i];
    }
    __syncthreads();
  }

  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = acc[t][mt][i];
#pragma unroll
          for (int w = 1; w < W; ++w)
            v += red[(((w - 1) * NT + t) * MT + mt) * 4 * 64 + i * 64 + lane];
          const int row = m0 + mt * 16 + (lane >> 4) * 4 + i;
          const int col = col_base + t * 16 + (lane & 15);
          if (row < M) {
            if (SPLIT == 0) out[(long)row * N + col] = to_bits<DT>(v);
            else if (SPLIT == 1) partial[((long)split * M + row) * N + col] = v;
            else __hip_atomic_store(&partial[((long)split * M + row) * N + col], v,
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
  }
  if (SPLIT != 2) return;

  // Partials are written through to memory once vmcnt drains; then the ticket.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* ticket = tickets + mchunk * gridDim.x + nb;
  if (threadIdx.x == 0)
    last_flag = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                splits - 1;
  __syncthreads();
  if (!last_flag) return;
  for (int e = threadIdx.x; e < rows * NT * 16; e += 64 * W) {
    const int r = e / (NT * 16);
    const int col = col_base + e % (NT * 16);
    const long off = (long)(m0 + r) * N + col;
    float v = 0.f;
    for (int sp = 0; sp < splits; ++sp)
      v += __hip_atomic_load(&partial[(long)sp * M * N + off], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out[off] = to_bits<DT>(v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sums `splits` fp32 partials [splits][M][N] in split order -> out (4 columns per thread).
template <int DT>
__global__ void w4a16_reduce_kernel(const float* __restrict__ partial, uint16_t* __restrict__ out,
                                    long mn, int splits) {
  const long i4 = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i4 >= mn) return;
  f32x4 v = *(const f32x4*)(partial + i4);
  for (int sp = 1; sp < splits; ++sp) {
    f32x4 p = *(const f32x4*)(partial + (long)sp * mn + i4);
    v += p;
  }
  uint32_t lo = (uint32_t)to_bits<DT>(v[0]) | ((uint32_t)to_bits<DT>(v[1]) << 16);
  uint32_t hi = (uint32_t)to_bits<DT>(v[2]) | ((uint32_t)to_bits<DT>(v[3]) << 16);
  *(uint2*)(out + i4) = make_uint2(lo, hi);
}

struct Plan {
  int mt;       // 16-row tiles per M chunk (template)
  int nt;       // 16-column tiles per workgroup (template)
  int waves;    // waves per workgroup (template)
  int depth;    // ring depth per wave (template)
  int splits;   // K splits across workgroups (grid y)
  int mode;     // split reduction: 1 = reduce kernel, 2 = in-kernel ticket (SPLIT template)
  int alds;     // A staged in LDS (template)
  int mchunks;  // grid z
  int nblocks;  // grid x
  int lds;      // dynamic LDS bytes
};

// TI_ROCM_W4A16_PLAN="nt:waves:depth:splits[:mode[:alds]]" overrides the heuristic (tuning).
static bool env_plan(Plan& p) {
  const char* e = getenv("TI_ROCM_W4A16_PLAN");
  if (!e || !*e) return false;
  int nt, w, d, s, mode = 2, alds = -1;
  if (sscanf(e, "%d:%d:%d:%d:%d:%d", &nt, &w, &d, &s, &mode, &alds) < 4) return false;
  p.nt = nt; p.waves = w; p.depth = d; p.splits = s; p.mode = mode; p.alds = alds;
  return true;
}

static Plan make_plan(int M, int N, int K) {
  Plan p;
  p.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.mchunks = cdiv(M, p.mt * 16);
  const int NG = K / kGroup;
  if (!env_plan(p)) {
    // Measured on MI355X for the Llama-3-8B MLP shapes (K=4096/N=28672 and
    // K=14336/N=4096): wide N streams best with 4 tiles x 4 waves per
    // workgroup and no split; narrow N needs split-K to cover 256 CUs, with
    // fewer tiles per workgroup the smaller M is.
    const int T = N / 16;
    p.depth = 2;
    p.mode = 2;
    p.alds = 0;
    if (T / 4 >= 256) {
      p.nt = 4; p.waves = 4; p.splits = 1;
    } else if (M == 1) {
      p.nt = 1; p.waves = 8; p.depth = 4; p.alds = -1;
      p.splits = cdiv(256, T);
    } else if (M <= 16) {
      p.nt = 2; p.waves = 8; p.splits = cdiv(256, T / 2);
    } else if (M <= 32) {
      p.nt = 4; p.waves = 8; p.splits = cdiv(256, T / 4);
    } else {
      p.nt = 4; p.waves = 4; p.splits = cdiv(256, (T / 4) * p.mchunks);
    }
    p.splits = max(1, min(p.splits, NG / (2 * p.waves)));
  }
  if (p.nt != 1 && p.nt != 2 && p.nt != 4) p.nt = 4;
  if (p.waves != 4 && p.waves != 8) p.waves = 4;
  if (p.depth != 2 && p.depth != 4 && p.depth != 8) p.depth = 2;
  if (p.depth == 8 && (p.mt != 1 || p.nt > 2)) p.depth = 4;  // depth 8: single-row-tile, narrow plans only
  if (N % (p.nt * 16)) p.nt = 1;
  p.nblocks = N / (p.nt * 16);
  p.splits = max(1, min(p.splits, NG));
  if (p.mode != 1) p.mode = 2;
  const int ngr = cdiv(NG, p.splits);
  const int rows = min(p.mt * 16, M);
  const int a_bytes = rows * a_stride(ngr) * 2;
  const int s_bytes = ngr * p.nt * 16 * 2;
  if (p.alds < 0) p.alds = (a_bytes + s_bytes <= kLdsBudget) ? 1 : 0;
  const int stage = (p.alds ? a_bytes : 0) + s_bytes;
  const int red = (p.waves - 1) * p.nt * p.mt * 4 * 64 * 4;
  p.lds = stage > red ? stage : red;
  return p;
}

// Workspace: fp32 partials [splits][M][N] from the start; the ticket ints sit
// at the 256-aligned end of the caller's buffer.  A buffer of at least
// max(partial bytes) + max(ticket bytes) + 256 over every problem it serves
// (ti_w4a16_workspace_bytes_max) therefore never lets one call's partials
// overlap another call's tickets, which must stay zero between calls.
static size_t ticket_bytes(const Plan& p) {
  return ((size_t)p.nblocks * p.mchunks * sizeof(int) + 255) & ~(size_t)255;
}

static size_t partial_bytes(const Plan& p, int M, int N) {
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

static size_t workspace_bytes(const Plan& p, int M, int N) {
  if (p.splits <= 1) return 0;
  return partial_bytes(p, M, N) + ticket_bytes(p) + 256;
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
  const long wtotal = (long)(N / 16) * (K / kGroup) * 256;
  hipLaunchKernelGGL(repack_weight_kernel, dim3((unsigned)((wtotal + 255) / 256)), dim3(256), 0,
                     stream, (const uint32_t*)qweight, (uint32_t*)packed_weight, N, wtotal);
  TI_CHECK_LAUNCH("ti_int4_repack");
  // The kernel reads scales in their [K/128, N] order.
  hipError_t e = hipMemcpyAsync(packed_scales, scales, (size_t)(K / kGroup) * N * 2,
                                hipMemcpyDeviceToDevice, stream);
  if (e != hipSuccess) {
    set_error("ti_int4_repack: scale copy failed: %s", hipGetErrorString(e));
    return TI_ERR_HIP;
  }
  return TI_OK;
}

extern "C" int ti_int4_quantize_rtn(const void* weight_kn, int weight_dtype, int K, int N, int group_size,
                                    int scale_dtype, int32_t* qweight, void* scales, hipStream_t stream) {
  TI_CHECK_ARG(weight_kn && qweight && scales, "ti_int4_quantize_rtn: null pointer");
  TI_CHECK_ARG((weight_dtype == TI_DTYPE_F16 || weight_dtype == TI_DTYPE_BF16) &&
                   (scale_dtype == TI_DTYPE_F16 || scale_dtype == TI_DTYPE_BF16),
               "ti_int4_quantize_rtn: weight and scale dtypes must be fp16 or bf16");
  TI_CHECK_SHAPE(group_size == kGroup, "ti_int4_quantize_rtn: group_size must be 128 (got %d)", group_size);
  TI_CHECK_SHAPE(K > 0 && N > 0 && K % kGroup == 0, "ti_int4_quantize_rtn: need K %% 128 == 0 (K=%d)", K);
  const long total = (long)(K / kGroup) * N;
  dim3 grid((unsigned)((total + 255) / 256));
#define TI_QR(W, S)                                                                                       \
  hipLaunchKernelGGL((quantize_rtn_kernel<W, S>), grid, dim3(256), 0, stream, (const uint16_t*)weight_kn, K, N, \
                     (uint32_t*)qweight, (uint16_t*)scales)
  if (weight_dtype == TI_DTYPE_F16) {
    if (scale_dtype == TI_DTYPE_F16) TI_QR(TI_DTYPE_F16, TI_DTYPE_F16); else TI_QR(TI_DTYPE_F16, TI_DTYPE_BF16);
  } else {
    if (scale_dtype == TI_DTYPE_F16) TI_QR(TI_DTYPE_BF16, TI_DTYPE_F16); else TI_QR(TI_DTYPE_BF16, TI_DTYPE_BF16);
  }
#undef TI_QR
  TI_CHECK_LAUNCH("ti_int4_quantize_rtn");
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
  const long blocks = (long)(N / 16) * (K / kGroup);
  const int waves_per_block = 4;
  dim3 grid((unsigned)((blocks + waves_per_block - 1) / waves_per_block));
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

// Kernel choice by M (measured on MI355X at the Llama-3-8B MLP shapes): the
// register-ring kernel of this file streams best for M <= 8; the LDS-DMA
// decode kernel (int4_decode.hip) for 9 <= M <= 128; above, this file's kernel
// again.  TI_ROCM_W4A16_DECODE_MIN_M / _MAX_M override the range (tuning).
static int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return (e && *e) ? atoi(e) : dflt;
}

// The decode kernel addresses activations with 32-bit byte offsets (M*K*2 < 2^31).
static bool use_decode(int M, int K) {
  return M >= env_int("TI_ROCM_W4A16_DECODE_MIN_M", 9) && M <= env_int("TI_ROCM_W4A16_DECODE_MAX_M", 128) &&
         (long)M * K * 2 < (1L << 31);
}

// Workspace of one call: fp32 partials [splits][M][N] from the start, ticket
// ints at the 256-aligned end of the caller's buffer.  A buffer of at least
// max(partial bytes) + max(ticket bytes) + 256 over every problem it serves
// (ti_w4a16_workspace_bytes_max) never lets one call's partials overlap another
// call's tickets, which must stay zero between calls.
struct WsNeed {
  size_t partial, tickets;
};

static WsNeed ws_need(int M, int N, int K) {
  StreamPlan sp;
  if (make_stream_plan(M, N, K, sp)) {
    if (sp.splits <= 1) return {0, 0};
    return {stream_partial_bytes(sp, M, N), stream_ticket_bytes(sp)};
  }
  if (use_decode(M, K)) {
    DecodePlan d = make_decode_plan(M, N, K);
    if (d.splits <= 1) return {0, 0};
    return {decode_partial_bytes(d, M, N), decode_ticket_bytes(d)};
  }
  Plan p = make_plan(M, N, K);
  if (p.splits <= 1) return {0, 0};
  return {partial_bytes(p, M, N), ticket_bytes(p)};
}

extern "C" int ti_w4a16_plan_name(int M, int N, int K, int group_size, char* buf, size_t len) {
  TI_CHECK_ARG(buf && len > 0, "ti_w4a16_plan_name: null buffer");
  TI_CHECK_SHAPE(group_size == kGroup && M >= 1 && N > 0 && K > 0 && K % kGroup == 0 && N % 64 == 0,
                 "ti_w4a16_plan_name: need M >= 1, K %% 128 == 0, N %% 64 == 0");
  StreamPlan sp;
  if (make_stream_plan(M, N, K, sp)) {
    snprintf(buf, len, "w4a16_stream_kernel mt=%d nt=%d waves=%d depth=%d splits=%d lds=%d", sp.mt, sp.nt,
             sp.waves, sp.depth, sp.splits, sp.lds);
  } else if (use_decode(M, K)) {
    DecodePlan d = make_decode_plan(M, N, K);
    snprintf(buf, len, "w4a16_decode_kernel mr=%d nt=%d wk=%d waves=%d ring=%d splits=%d mchunks=%d lds=%d", d.mr,
             d.nt, d.wk, d.waves, d.ring, d.splits, d.mchunks, d.lds);
    TI_CHECK_SHAPE(d.lds <= kDecodeLdsMax && decode_plan_valid(d, N), "ti_w4a16_plan_name: invalid plan (%s)", buf);
  } else {
    Plan p = make_plan(M, N, K);
    snprintf(buf, len, "w4a16_gemm_kernel mt=%d nt=%d waves=%d depth=%d splits=%d mode=%d alds=%d lds=%d", p.mt, p.nt,
             p.waves, p.depth, p.splits, p.mode, p.alds, p.lds);
    TI_CHECK_SHAPE(p.lds <= 160 * 1024, "ti_w4a16_plan_name: invalid plan (%s)", buf);
  }
  return TI_OK;
}

extern "C" size_t ti_w4a16_workspace_bytes(int M, int N, int K, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size != kGroup || N % 64 || K % kGroup) return 0;
  WsNeed w = ws_need(M, N, K);
  return w.partial ? w.partial + w.tickets + 256 : 0;
}

extern "C" size_t ti_w4a16_workspace_bytes_max(int max_m, int N, int K, int group_size) {
  if (max_m <= 0 || N <= 0 || K <= 0 || group_size != kGroup || N % 64 || K % kGroup) return 0;
  size_t pmax = 0, tmax = 0;
  for (int m = 1; m <= max_m; ++m) {
    WsNeed w = ws_need(m, N, K);
    pmax = w.partial > pmax ? w.partial : pmax;
    tmax = w.tickets > tmax ? w.tickets : tmax;
  }
  return pmax ? pmax + tmax + 256 : 0;
}

struct LaunchArgs {
  const uint16_t* a;
  const i32x4* w;
  const uint16_t* s;
  uint16_t* out;
  float* partial;
  int* tickets;
  int M, N, K;
};

template <int DT, int MT, int NT, int W, int D, bool AL>
static void launch_split(const Plan& p, const LaunchArgs& x, hipStream_t stream) {
  dim3 grid(p.nblocks, p.splits, p.mchunks);
  if (p.splits == 1) {
    hipLaunchKernelGGL((w4a16_gemm_kernel<DT, MT, NT, W, D, 0, AL>), grid, dim3(64 * W), p.lds, stream,
                       x.a, x.w, x.s, x.out, x.partial, x.tickets, x.M, x.N, x.K, 1);
  } else if (p.mode == 2) {
    hipLaunchKernelGGL((w4a16_gemm_kernel<DT, MT, NT, W, D, 2, AL>), grid, dim3(64 * W), p.lds, stream,
                       x.a, x.w, x.s, x.out, x.partial, x.tickets, x.M, x.N, x.K, p.splits);
  } else {
    hipLaunchKernelGGL((w4a16_gemm_kernel<DT, MT, NT, W, D, 1, AL>), grid, dim3(64 * W), p.lds, stream,
                       x.a, x.w, x.s, x.out, x.partial, x.tickets, x.M, x.N, x.K, p.splits);
    const long mn = (long)x.M * x.N;
    hipLaunchKernelGGL(w4a16_reduce_kernel<DT>, dim3((unsigned)((mn / 4 + 255) / 256)), dim3(256), 0,
                       stream, x.partial, x.out, mn, p.splits);
  }
}

template <int DT, int MT, int NT, int W, int D>
static void launch_al(const Plan& p, const LaunchArgs& x, hipStream_t stream) {
  if (p.alds) launch_split<DT, MT, NT, W, D, true>(p, x, stream);
  else launch_split<DT, MT, NT, W, D, false>(p, x, stream);
}

template <int DT, int MT, int NT, int W>
static void launch_d(const Plan& p, const LaunchArgs& x, hipStream_t stream) {
  if constexpr (MT == 1 && NT <= 2) {
    if (p.depth == 8) {
      launch_al<DT, MT, NT, W, 8>(p, x, stream);
      return;
    }
  }
  if (p.depth >= 4) launch_al<DT, MT, NT, W, 4>(p, x, stream);
  else launch_al<DT, MT, NT, W, 2>(p, x, stream);
}

template <int DT, int MT, int NT>
static void launch_w(const Plan& p, const LaunchArgs& x, hipStream_t stream) {
  if (p.waves == 8) launch_d<DT, MT, NT, 8>(p, x, stream);
  else launch_d<DT, MT, NT, 4>(p, x, stream);
}

template <int DT, int MT>
static void launch_nt(const Plan& p, const LaunchArgs& x, hipStream_t stream) {
  if (p.nt == 1) launch_w<DT, MT, 1>(p, x, stream);
  else if (p.nt == 2) launch_w<DT, MT, 2>(p, x, stream);
  else launch_w<DT, MT, 4>(p, x, stream);
}

template <int DT>
static void launch_mt(const Plan& p, const LaunchArgs& x, hipStream_t stream) {
  if (p.mt == 1) launch_nt<DT, 1>(p, x, stream);
  else if (p.mt == 2) launch_nt<DT, 2>(p, x, stream);
  else launch_nt<DT, 4>(p, x, stream);
}

extern "C" int ti_w4a16_gemm(const void* a, int dtype, const int32_t* packed_weight,
                             const void* packed_scales, void* out, int M, int N, int K,
                             int group_size, void* workspace, size_t workspace_bytes_,
                             hipStream_t stream) {
  TI_CHECK_ARG(a && packed_weight && packed_scales && out, "ti_w4a16_gemm: null pointer");
  TI_CHECK_ARG(dtype == TI_DTYPE_F16 || dtype == TI_DTYPE_BF16,
               "ti_w4a16_gemm: dtype must be fp16 or bf16");
  TI_CHECK_SHAPE(group_size == kGroup, "ti_w4a16_gemm: group_size must be 128 (got %d)", group_size);
  TI_CHECK_SHAPE(M >= 1 && N > 0 && K > 0 && K % kGroup == 0 && N % 64 == 0,
                 "ti_w4a16_gemm: need M >= 1, K %% 128 == 0, N %% 64 == 0 (M=%d N=%d K=%d)", M, N, K);
  TI_CHECK_ARG(((uintptr_t)a & 15) == 0 && ((uintptr_t)packed_weight & 15) == 0 &&
               ((uintptr_t)packed_scales & 15) == 0,
               "ti_w4a16_gemm: a, packed_weight and packed_scales must be 16-byte aligned");
  TI_CHECK_ARG(((uintptr_t)out & 7) == 0, "ti_w4a16_gemm: out must be 8-byte aligned");
  StreamPlan sp;
  if (make_stream_plan(M, N, K, sp)) {
    StreamArgs x{(const uint16_t*)a, (const i32x4*)packed_weight, (const uint16_t*)packed_scales,
                 (uint16_t*)out, nullptr, nullptr, M, N, K};
    if (sp.splits > 1) {
      const size_t need = stream_partial_bytes(sp, M, N) + stream_ticket_bytes(sp) + 256;
      if (!workspace || workspace_bytes_ < need) {
        set_error("ti_w4a16_gemm: workspace of %zu bytes required (got %zu)", need, workspace_bytes_);
        return TI_ERR_WORKSPACE;
      }
      TI_CHECK_ARG(((uintptr_t)workspace & 15) == 0, "ti_w4a16_gemm: workspace must be 16-byte aligned");
      x.partial = (float*)workspace;
      const uintptr_t end = ((uintptr_t)workspace + workspace_bytes_) & ~(uintptr_t)255;
      x.tickets = (int*)(end - stream_ticket_bytes(sp));
    }
    launch_stream(sp, dtype, x, stream);
    TI_CHECK_LAUNCH("ti_w4a16_gemm");
    return TI_OK;
  }
  if (use_decode(M, K)) {
    DecodePlan d = make_decode_plan(M, N, K);
    TI_CHECK_SHAPE(d.lds <= kDecodeLdsMax, "ti_w4a16_gemm: decode plan needs %d bytes of LDS", d.lds);
    TI_CHECK_SHAPE(decode_plan_valid(d, N), "ti_w4a16_gemm: no decode kernel for plan nt=%d wk=%d ring=%d mr=%d at N=%d",
                   d.nt, d.wk, d.ring, d.mr, N);
    DecodeArgs x{(const uint16_t*)a, (const i32x4*)packed_weight, (const uint16_t*)packed_scales,
                 (uint16_t*)out, nullptr, nullptr, M, N, K};
    if (d.splits > 1) {
      const size_t need = decode_partial_bytes(d, M, N) + decode_ticket_bytes(d) + 256;
      if (!workspace || workspace_bytes_ < need) {
        set_error("ti_w4a16_gemm: workspace of %zu bytes required (got %zu)", need, workspace_bytes_);
        return TI_ERR_WORKSPACE;
      }
      TI_CHECK_ARG(((uintptr_t)workspace & 15) == 0, "ti_w4a16_gemm: workspace must be 16-byte aligned");
      x.partial = (float*)workspace;
      const uintptr_t end = ((uintptr_t)workspace + workspace_bytes_) & ~(uintptr_t)255;
      x.tickets = (int*)(end - decode_ticket_bytes(d));
    }
    launch_decode(d, dtype, x, stream);
    TI_CHECK_LAUNCH("ti_w4a16_gemm");
    return TI_OK;
  }
  Plan p = make_plan(M, N, K);
  TI_CHECK_SHAPE(p.lds <= 160 * 1024, "ti_w4a16_gemm: plan needs %d bytes of LDS", p.lds);
  size_t need = workspace_bytes(p, M, N);
  LaunchArgs x{(const uint16_t*)a, (const i32x4*)packed_weight, (const uint16_t*)packed_scales,
               (uint16_t*)out, nullptr, nullptr, M, N, K};
  if (need) {
    if (!workspace || workspace_bytes_ < need) {
      set_error("ti_w4a16_gemm: workspace of %zu bytes required (got %zu)", need, workspace_bytes_);
      return TI_ERR_WORKSPACE;
    }
    TI_CHECK_ARG(((uintptr_t)workspace & 15) == 0, "ti_w4a16_gemm: workspace must be 16-byte aligned");
    x.partial = (float*)workspace;
    const uintptr_t end = ((uintptr_t)workspace + workspace_bytes_) & ~(uintptr_t)255;
    x.tickets = (int*)(end - ticket_bytes(p));
  }
  if (dtype == TI_DTYPE_F16) launch_mt<TI_DTYPE_F16>(p, x, stream);
  else launch_mt<TI_DTYPE_BF16>(p, x, stream);
  TI_CHECK_LAUNCH("ti_w4a16_gemm");
  return TI_OK;
}
