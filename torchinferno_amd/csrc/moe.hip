// Routed FP8 block-scaled MoE for gfx950 (DeepSeek-V3/V4 expert shapes).
//
// Replaces the reference's grouped expert path -- fused_mxfp4_moe with its
// moe_align_block_size / grouped Marlin GEMMs
// (src/torchinferno/kernels/deepseek_v4_marlin.py:267-411) -- and computes the
// per-expert loop it stands for (src/torchinferno/models/deepseek_v4/
// tensor_parallel.py:792-802,882-914): for every routed expert e of token t,
//   g, u = w1 x, w3 x   (block-FP8 Linear: 1x128 act quant + 128x128 GEMM, bf16)
//   h    = bf16(w[t,e] * silu(g) * u)          (fp32 math, optional clamp)
//   y[t] += w2 h                               (block-FP8 Linear, bf16 out)
// with y accumulated in fp32 over the token's experts in expert-index order.
// Router (ti_moe_route_topk): softmax over fp32 logits, top-k, gather the
// chosen probabilities, renormalise, scale -- tensor_parallel.py:760-780 and
// src/torchinferno/models/deepseek_v32/model.py:692-722.
//
// Pipeline (one stream, no host synchronisation, graph-capturable):
//   1. act_quant of the T hidden rows (1x128, shared by all k routes of a row);
//   2. align: routes counted per expert, prefix-summed, every route assigned a
//      row in expert-sorted order, and the grouped GEMM's m-tile table
//      (expert, first row, rows) written -- rows inside an expert are placed by
//      atomics, which changes no value because every output row of the GEMMs
//      depends only on its own input row;
//   3. grouped GEMM w13 (gathering hidden rows by token) -> [R, 2I] bf16;
//   4. SwiGLU x route weight -> bf16 -> 1x128 quant, per sorted row;
//   5. grouped GEMM w2 -> [R, H] bf16;
//   6. combine: per token, its routes' rows summed in fp32 in expert order.
#include "fp8_common.h"
#include "fp8_gemm.h"

namespace ti {
namespace moe {
namespace {

using fp8::e4m3_encode;
using fp8::kE4M3Max;

constexpr int kAlignThreads = 1024;
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopk = 16;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One wave per token; E <= 1024 logits, k <= 16.
__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits, int T, int E, int k,
                                                    int renorm, float route_scale, float* __restrict__ w_out,
                                                    int* __restrict__ id_out) {
  const int lane = threadIdx.x & 63;
  const long t = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* z = logits + t * E;
  constexpr int PER = kMaxExperts / 64;
  float v[PER];
  float zmax = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? z[e] : -INFINITY;
    zmax = fmaxf(zmax, v[i]);
  }
  zmax = wave_max(zmax);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    if (lane + 64 * i < E) sum += expf(v[i] - zmax);
  sum = wave_sum(sum);
  // Top-k on the logits (softmax is monotonic, so this is the probabilities'
  // order); ties go to the lower expert index.
  float sel_w[kMaxTopk];
  int sel_id[kMaxTopk];
  float wsum = 0.f;
  for (int j = 0; j < k; ++j) {
    float best = -INFINITY;
    int bid = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = lane + 64 * i;
      if (e < E && (v[i] > best || (v[i] == best && e < bid))) { best = v[i]; bid = e; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ob = __shfl_xor(best, off, 64);
      const int oi = __shfl_xor(bid, off, 64);
      if (ob > best || (ob == best && oi < bid)) { best = ob; bid = oi; }
    }
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (lane + 64 * i == bid) v[i] = -INFINITY;
    const float p = expf(best - zmax) / sum;
    sel_w[j] = p;
    sel_id[j] = bid;
    wsum += p;
  }
  if (lane == 0) {
    const float den = fmaxf(wsum, 1e-20f);
    for (int j = 0; j < k; ++j) {
      const float w = renorm ? sel_w[j] / den : sel_w[j];
      w_out[t * k + j] = w * route_scale;
      id_out[t * k + j] = sel_id[j];
    }
  }
}

struct Plan {
  int kind;        // grouped GEMM tile kind
  int bm;          // its m-tile rows
  int max_tiles;   // m-tile table capacity
  int kind2;       // second tier (-1: none): 256-row m-tiles for experts with more than bm rows
  int bm2;         // its m-tile rows (0: no second tier)
  int max_tiles2;  // second-tier table capacity
};

Plan make_plan(int T, int k, int E, int smode) {
  const long R = (long)T * k;
  const long avg = (R + E - 1) / E;
  Plan p;
  // Measured at the config-4 shapes: 16-row tiles for few rows per expert
  // (T=64: avg 2; the 8-wave 16x256 tile, 1-2% over 16x128), 32-row tiles at
  // T=512 (avg 16: the 4-wave 32x256 tile, 6-8% over the 8-wave 32x128 one for
  // FP8 experts; MXFP4 with fp32 activation scales keeps 32x128, 3% faster
  // there), 8-wave 128x256 at avg 128
  // (T=4096: one m-tile per expert and half the activation re-reads of
  // 128x128; -20% FP8, -4% MXFP4), 8-wave 128x128 between.  At avg 128 the
  // 16x16x128 form of the 128x256 tile (kind 20; 4-register partial sums)
  // folds the block scales 1-2% faster than the 32x32x64 form (kind 17).
  p.kind = avg <= 8 ? 10 : (avg <= 48 ? (smode == 2 ? 12 : 4) : (avg <= 96 ? 15 : 20));
  const char* env = getenv("TI_ROCM_MOE_KIND");
  if (env && *env) {
    const int kk = atoi(env);
    if (kk == 2 || kk == 3 || kk == 4 || kk == 5 || kk == 6 || kk == 9 || kk == 10 || kk == 11 || kk == 12 || kk == 13 ||
        kk == 15 || kk == 16 ||
        kk == 17 || kk == 20)
      p.kind = kk;
  }
  p.bm = fp8::grouped_bm(p.kind);
  p.max_tiles = (int)(R / p.bm + E + 1);
  // Two tiers with the 128-row tile: an expert's rows go to 192-row tiles,
  // and a remainder of at most 128 rows to one 128-row tile.  An expert with
  // 129-192 rows then streams its weights once (one 192-row tile) instead of
  // once per 128-row tile.  At T=4096 the rows per expert cluster around 128
  // (sd ~11), so the second tier is mostly 129-160 rows: 192-row tiles
  // (kind 19, 16x16x128 MFMAs) waste a third of the MFMA work of 256-row ones
  // (kind 16) and measured 4-8% faster over the whole MoE.
  p.kind2 = -1;
  p.bm2 = 0;
  p.max_tiles2 = 0;
  if (p.kind == 17 || p.kind == 20) {
    const char* e2 = getenv("TI_ROCM_MOE_KIND2");
    p.kind2 = (e2 && *e2) ? atoi(e2) : 19;
    if (p.kind2 != 9 && p.kind2 != 16 && p.kind2 != 18 && p.kind2 != 19 && !(p.kind2 == 14 && smode == 3))
      p.kind2 = -1;
  }
  if (p.kind2 >= 0) {
    p.bm2 = fp8::grouped_bm(p.kind2);
    p.max_tiles = E + 1;
    p.max_tiles2 = (int)(R / p.bm2 + E + 1);
  }
  return p;
}

// Workspace carve-up (256-byte aligned pieces).
struct Ws {
  uint8_t* xq; float* xs;                  // act_quant of the hidden rows
  int* pos_of_route;                       // [R] sorted row of route r (-1: dropped)
  int* tok_of_pos;                         // [R] token of sorted row p
  int* route_of_pos;                       // [R] route of sorted row p
  int* tile_expert; int* tile_row0; int* tile_rows; int* num_tiles;
  int* tile2_expert; int* tile2_row0; int* tile2_rows; int* num_tiles2;  // second tier
  int* num_rows;                           // device scalar: sorted rows in use
  int* cnt;                                // [2E]: routes per expert, then the placement cursors
  int* row0;                               // [E] first sorted row of each expert
  uint16_t* out1;                          // [R, 2I] bf16
  uint8_t* hq; float* hs;                  // [R, I] e4m3, [R, I/128]
  uint16_t* out2;                          // [R, H] bf16
  size_t bytes;
};

Ws carve(uint8_t* base, int T, int k, int E, int H, int I, const Plan& p) {
  const size_t R = (size_t)T * k;
  size_t off = 0;
  auto take = [&](size_t n) {
    uint8_t* q = base ? base + off : nullptr;
    off += (n + 255) & ~(size_t)255;
    return q;
  };
  Ws w;
  w.xq = take((size_t)T * H);
  w.xs = (float*)take((size_t)T * (H / 128) * 4);
  w.pos_of_route = (int*)take(R * 4);
  w.tok_of_pos = (int*)take(R * 4);
  w.route_of_pos = (int*)take(R * 4);
  w.tile_expert = (int*)take((size_t)p.max_tiles * 4);
  w.tile_row0 = (int*)take((size_t)p.max_tiles * 4);
  w.tile_rows = (int*)take((size_t)p.max_tiles * 4);
  w.num_tiles = (int*)take(4);
  w.tile2_expert = (int*)take((size_t)p.max_tiles2 * 4);
  w.tile2_row0 = (int*)take((size_t)p.max_tiles2 * 4);
  w.tile2_rows = (int*)take((size_t)p.max_tiles2 * 4);
  w.num_tiles2 = (int*)take(4);
  w.num_rows = (int*)take(4);
  w.cnt = (int*)take((size_t)2 * E * 4);
  w.row0 = (int*)take((size_t)E * 4);
  w.out1 = (uint16_t*)take(R * 2 * I * 2);
  w.hq = take(R * I);
  w.hs = (float*)take(R * (I / 128) * 4);
  w.out2 = (uint16_t*)take(R * H * 2);
  w.bytes = off;
  return w;
}

// Routes -> expert-sorted rows and the m-tile table, in three launches over
// the R = T*k routes (no single-workgroup pass over them):
//   align_count: per-workgroup LDS histogram of expert ids, added to cnt[E];
//   align_scan:  one workgroup: prefix sums of cnt -> first row and first
//                m-tile of every expert, the m-tile table, and the cursors;
//   align_place: every route takes the next row of its expert (a global
//                atomic on the expert's cursor) and records the row <-> route
//                maps.
// Rows inside an expert are placed in arrival order, which changes no value:
// every output row of the grouped GEMMs depends only on its own input row, and
// the combine sums a token's routes in expert order.  cnt and cursors start at
// zero: align_zero clears them (a kernel, not a memset, so graph replays clear
// them too).
constexpr int kAlignBlock = 256;

__global__ __launch_bounds__(kAlignBlock) void align_zero_kernel(int* __restrict__ cnt, int E) {
  for (int e = blockIdx.x * kAlignBlock + threadIdx.x; e < 2 * E; e += gridDim.x * kAlignBlock) cnt[e] = 0;
}

__global__ __launch_bounds__(kAlignBlock) void align_count_kernel(const int* __restrict__ ids, int R, int E,
                                                                  int* __restrict__ cnt) {
  __shared__ int h[kMaxExperts];
  for (int e = threadIdx.x; e < E; e += kAlignBlock) h[e] = 0;
  __syncthreads();
  const int r = blockIdx.x * kAlignBlock + threadIdx.x;
  if (r < R) {
    const int e = ids[r];
    if (e >= 0 && e < E) atomicAdd(&h[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += kAlignBlock)
    if (h[e]) atomicAdd(&cnt[e], h[e]);
}

// One workgroup of kAlignThreads: exclusive scans of rows and m-tiles over
// E <= 1024.  With a second tier (bm2 > 0) an expert of n rows takes n / bm2
// tiles of bm2 rows, the remainder r a further bm2 tile when r > bm and one
// bm tile when 0 < r <= bm.
__global__ __launch_bounds__(kAlignThreads) void align_scan_kernel(const int* __restrict__ cnt, int E, int bm,
                                                                   int bm2, int* __restrict__ row0,
                                                                   int* __restrict__ tile_expert,
                                                                   int* __restrict__ tile_row0,
                                                                   int* __restrict__ tile_rows,
                                                                   int* __restrict__ num_tiles,
                                                                   int* __restrict__ tile2_expert,
                                                                   int* __restrict__ tile2_row0,
                                                                   int* __restrict__ tile2_rows,
                                                                   int* __restrict__ num_tiles2,
                                                                   int* __restrict__ num_rows) {
  __shared__ int srow[kMaxExperts], stile[kMaxExperts], stile2[kMaxExperts];
  const int e = threadIdx.x;
  const int n = e < E ? cnt[e] : 0;
  int n2 = 0, n1;  // second-tier and first-tier tiles of this expert
  if (bm2 > 0) {
    n2 = n / bm2;
    const int r = n - n2 * bm2;
    if (r > bm) ++n2;
    n1 = (r > 0 && r <= bm) ? 1 : 0;
  } else {
    n1 = (n + bm - 1) / bm;
  }
  srow[e] = n;
  stile[e] = n1;
  stile2[e] = n2;
  __syncthreads();
  // Hillis-Steele inclusive scan over the 1024 slots
  for (int off = 1; off < kMaxExperts; off <<= 1) {
    const int a = e >= off ? srow[e - off] : 0, b = e >= off ? stile[e - off] : 0,
              c = e >= off ? stile2[e - off] : 0;
    __syncthreads();
    srow[e] += a;
    stile[e] += b;
    stile2[e] += c;
    __syncthreads();
  }
  if (e < E) {
    const int first = srow[e] - n, t0 = stile[e] - n1, u0 = stile2[e] - n2;
    row0[e] = first;
    for (int j = 0; j < n2; ++j) {
      tile2_expert[u0 + j] = e;
      tile2_row0[u0 + j] = first + j * bm2;
      tile2_rows[u0 + j] = min(bm2, n - j * bm2);
    }
    const int done = min(n, n2 * bm2);
    for (int j = 0; j < n1; ++j) {
      tile_expert[t0 + j] = e;
      tile_row0[t0 + j] = first + done + j * bm;
      tile_rows[t0 + j] = min(bm, n - done - j * bm);
    }
  }
  if (e == kMaxExperts - 1) {
    *num_tiles = stile[e];
    *num_tiles2 = stile2[e];
    *num_rows = srow[e];
  }
}

__global__ __launch_bounds__(kAlignBlock) void align_place_kernel(const int* __restrict__ ids, int R, int E, int k,
                                                                  const int* __restrict__ row0,
                                                                  int* __restrict__ cursor,
                                                                  int* __restrict__ pos_of_route,
                                                                  int* __restrict__ tok_of_pos,
                                                                  int* __restrict__ route_of_pos) {
  const int r = blockIdx.x * kAlignBlock + threadIdx.x;
  if (r >= R) return;
  const int e = ids[r];
  if (e < 0 || e >= E) {
    pos_of_route[r] = -1;
    return;
  }
  const int p = row0[e] + atomicAdd(&cursor[e], 1);
  pos_of_route[r] = p;
  tok_of_pos[p] = r / k;
  route_of_pos[p] = r;
}

// h = bf16(w * silu(g) * u) over one sorted row's 128-wide block, then 1x128
// e4m3 quant (act_quant; power-of-two scales when round_scale).  An item is
// (row, four blocks): one wave, a 16-lane group per block, 8 elements (16-byte
// loads) per lane; the launch has a wave per item (a grid-stride loop with a
// capped grid measured slower: 155 vs 135 us at T=4096).
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const uint16_t* __restrict__ gu, int I,
                                                           const float* __restrict__ route_w,
                                                           const int* __restrict__ route_of_pos,
                                                           const int* __restrict__ num_rows, long R,
                                                           float clamp_limit, int round_scale,
                                                           uint8_t* __restrict__ hq, float* __restrict__ hs) {
  const int lane = threadIdx.x & 63;
  const int IB = I / 128;
  const int QB = (IB + 3) / 4;
  const long items = (long)*num_rows * QB;  // rows in use
  const long stride = (long)gridDim.x * 4;
#pragma unroll 2
  for (long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6); item < items; item += stride) {
    const long p = item / QB;
    const int blk = (int)(item % QB) * 4 + (lane >> 4);
    const bool on = blk < IB;
    const float w = route_w[route_of_pos[p]];
    const uint16_t* row = gu + p * 2 * I;
    const int c = min(blk, IB - 1) * 128 + (lane & 15) * 8;
    const uint4 gw = *(const uint4*)(row + c);
    const uint4 uw = *(const uint4*)(row + I + c);
    const uint32_t gv[4] = {gw.x, gw.y, gw.z, gw.w}, uv[4] = {uw.x, uw.y, uw.z, uw.w};
    float h[8];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float g = bf16_bits_to_f32((uint16_t)(gv[i >> 1] >> (16 * (i & 1))));
      float u = bf16_bits_to_f32((uint16_t)(uv[i >> 1] >> (16 * (i & 1))));
      if (clamp_limit > 0.f) {
        u = fminf(fmaxf(u, -clamp_limit), clamp_limit);
        g = fminf(g, clamp_limit);
      }
      const float act = g / (1.0f + expf(-g)) * u;
      h[i] = bf16_bits_to_f32(f32_to_bf16_bits(w * act));
      amax = fmaxf(amax, fabsf(h[i]));
    }
    // block max over the 16 lanes of the group
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
    amax = fmaxf(amax, 1e-4f);
    float sc = amax * (1.0f / kE4M3Max);
    if (round_scale) {  // 2^ceil(log2(amax / 448)), the ue8m0 scale format
      const uint32_t bits = __float_as_uint(sc);
      const int e = (int)((bits >> 23) & 0xFF) - 127 + ((bits & 0x7FFFFFu) != 0 ? 1 : 0);
      sc = __uint_as_float((uint32_t)(e + 127) << 23);
    }
    // x / sc: exact as a product for power-of-two scales, else quot_for_e4m3
    const float r = 1.0f / sc;
    float y[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      y[i] = fminf(fmaxf(round_scale ? h[i] * r : fp8::quot_for_e4m3(h[i], sc, r), -kE4M3Max), kE4M3Max);
    if (on) {
      *(uint2*)(hq + p * I + c) = fp8::e4m3_pack8_hw(y);
      if ((lane & 15) == 0) hs[p * IB + blk] = sc;
    }
  }
}

// y[t] = bf16(sum over t's routes, in expert order, of fp32(out2[row])).
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ out2, int H,
                                                      const int* __restrict__ ids,
                                                      const int* __restrict__ pos_of_route, int k,
                                                      uint16_t* __restrict__ y) {
  const long t = blockIdx.x;
  // The token's rows sorted by expert id (stable: slot order for equal ids),
  // by one thread into LDS.
  __shared__ int spos[kMaxTopk], eid[kMaxTopk];
  __shared__ int sn;
  if (threadIdx.x == 0) {
    int n = 0;
    for (int s = 0; s < k; ++s) {
      const int p = pos_of_route[t * k + s];
      if (p < 0) continue;
      const int e = ids[t * k + s];
      int j = n++;
      while (j > 0 && eid[j - 1] > e) { eid[j] = eid[j - 1]; spos[j] = spos[j - 1]; --j; }
      eid[j] = e;
      spos[j] = p;
    }
    sn = n;
  }
  __syncthreads();
  const int n = sn;
  int pos[kMaxTopk];
#pragma unroll
  for (int j = 0; j < kMaxTopk; ++j) pos[j] = j < n ? spos[j] : 0;
  for (int c = threadIdx.x * 8; c < H; c += 256 * 8) {
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // all of the token's rows in flight before the in-order sum
    // (absent rows read as +0, which leaves a sum that starts at +0 unchanged)
    uint4 v[kMaxTopk];
#pragma unroll
    for (int j = 0; j < kMaxTopk; ++j)
      v[j] = j < n ? *(const uint4*)(out2 + (long)pos[j] * H + c) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int j = 0; j < kMaxTopk; ++j) {
      const uint32_t vv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] += bf16_bits_to_f32((uint16_t)(vv[i >> 1] >> (16 * (i & 1))));
    }
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = (uint32_t)f32_to_bf16_bits(a[2 * i]) | ((uint32_t)f32_to_bf16_bits(a[2 * i + 1]) << 16);
    uint16_t* yc = y + t * H + c;
    if (((uintptr_t)y & 15) == 0) {
      *(uint4*)yc = make_uint4(o[0], o[1], o[2], o[3]);
    } else {  // `out` need only be 4-byte aligned
#pragma unroll
      for (int i = 0; i < 4; ++i) ((uint32_t*)yc)[i] = o[i];
    }
  }
}

}  // namespace
}  // namespace moe
}  // namespace ti

using namespace ti;
using namespace ti::moe;

extern "C" int ti_moe_route_topk(const float* logits, int T, int E, int k, int renormalize, float route_scale,
                                 float* topk_weights, int32_t* topk_ids, hipStream_t stream) {
  TI_CHECK_ARG(logits && topk_weights && topk_ids, "ti_moe_route_topk: null pointer");
  TI_CHECK_SHAPE(T >= 0 && E >= 1 && E <= kMaxExperts && k >= 1 && k <= kMaxTopk && k <= E,
                 "ti_moe_route_topk: need 1 <= k <= min(16, E), E <= 1024 (E=%d k=%d)", E, k);
  if (T == 0) return TI_OK;
  hipLaunchKernelGGL(route_kernel, dim3((unsigned)((T + 3) / 4)), dim3(256), 0, stream, logits, T, E, k,
                     renormalize, route_scale, topk_weights, topk_ids);
  TI_CHECK_LAUNCH("ti_moe_route_topk");
  return TI_OK;
}

static bool moe_shape_ok(int T, int k, int E, int H, int I) {
  return T >= 0 && k >= 1 && k <= kMaxTopk && E >= 1 && E <= kMaxExperts && H > 0 && I > 0 && H % 128 == 0 &&
         I % 128 == 0 && (long)T * k <= (1L << 26);
}

extern "C" size_t ti_fp8_moe_workspace_bytes(int T, int k, int E, int H, int I) {
  if (!moe_shape_ok(T, k, E, H, I) || T == 0) return 0;
  // One size serves every weight and scale format (their plans may pick different tiles).
  size_t b = 0;
  for (int smode = 1; smode <= 4; ++smode) {
    const size_t bs = carve(nullptr, T, k, E, H, I, make_plan(T, k, E, smode)).bytes;
    b = bs > b ? bs : b;
  }
  return b;
}

// Routed experts, shared by the block-FP8 (smode 1: e4m3 weights, 128x128
// fp32 scales) and MXFP4 (smode 2: e2m1 weights two per byte, e8m0 scale per
// 32 K) weight formats; activations are 1x128 block FP8 in both.  With
// round_scale 2 every scale is a power of two and the grouped GEMMs apply
// them inside the MFMA (smode 3 / 4).
static int moe_run(const char* name, int smode, int sb_layout, const void* hidden, const float* topk_weights,
                   const int32_t* topk_ids, int T, int k, const uint8_t* w13, const void* s13, const uint8_t* w2,
                   const void* s2, int E, int H, int I, float clamp_limit, int round_scale, void* out,
                   void* workspace, size_t workspace_bytes, hipStream_t stream) {
  TI_CHECK_ARG(hidden && topk_weights && topk_ids && w13 && s13 && w2 && s2 && out, "%s: null pointer", name);
  TI_CHECK_SHAPE(moe_shape_ok(T, k, E, H, I),
                 "%s: need H %% 128 == 0, I %% 128 == 0, 1 <= k <= 16, E <= 1024 (T=%d k=%d E=%d H=%d I=%d)",
                 name, T, k, E, H, I);
  TI_CHECK_ARG(((uintptr_t)hidden & 15) == 0 && ((uintptr_t)w13 & 15) == 0 && ((uintptr_t)w2 & 15) == 0 &&
                   ((uintptr_t)out & 3) == 0 && ((uintptr_t)s13 & 3) == 0 && ((uintptr_t)s2 & 3) == 0,
               "%s: hidden, w13, w2 must be 16-byte and out, scales 4-byte aligned", name);
  TI_CHECK_ARG(round_scale >= 0 && round_scale <= 2, "%s: round_scale must be 0, 1 or 2", name);
  if (T == 0) return TI_OK;
  if (round_scale == 2) smode += 2;
  Plan p = make_plan(T, k, E, smode);
  Ws w = carve(nullptr, T, k, E, H, I, p);
  if (!workspace || workspace_bytes < w.bytes) {
    set_error("%s: workspace of %zu bytes required (got %zu)", name, w.bytes, workspace_bytes);
    return TI_ERR_WORKSPACE;
  }
  TI_CHECK_ARG(((uintptr_t)workspace & 255) == 0, "%s: workspace must be 256-byte aligned", name);
  w = carve((uint8_t*)workspace, T, k, E, H, I, p);
  const long R = (long)T * k;
  const bool f4 = smode == 2 || smode == 4;

  // 1. hidden -> e4m3 1x128
  int st = ti_fp8_quant_block(hidden, TI_DTYPE_BF16, T, H, 128, round_scale ? 1 : 0, w.xq, w.xs, 0, stream);
  if (st != TI_OK) return st;
  // 2. align
  const unsigned rblocks = (unsigned)((R + kAlignBlock - 1) / kAlignBlock);
  hipLaunchKernelGGL(align_zero_kernel, dim3((unsigned)((2 * E + kAlignBlock - 1) / kAlignBlock)), dim3(kAlignBlock),
                     0, stream, w.cnt, E);
  hipLaunchKernelGGL(align_count_kernel, dim3(rblocks), dim3(kAlignBlock), 0, stream, (const int*)topk_ids, (int)R,
                     E, w.cnt);
  hipLaunchKernelGGL(align_scan_kernel, dim3(1), dim3(kAlignThreads), 0, stream, (const int*)w.cnt, E, p.bm, p.bm2,
                     w.row0, w.tile_expert, w.tile_row0, w.tile_rows, w.num_tiles, w.tile2_expert, w.tile2_row0,
                     w.tile2_rows, w.num_tiles2, w.num_rows);
  hipLaunchKernelGGL(align_place_kernel, dim3(rblocks), dim3(kAlignBlock), 0, stream, (const int*)topk_ids, (int)R,
                     E, k, (const int*)w.row0, w.cnt + E, w.pos_of_route, w.tok_of_pos, w.route_of_pos);
  TI_CHECK_LAUNCH("moe(align)");
  // 3. grouped w13: [R, 2I] = xq[tok] . w13[e]^T
  fp8::GemmArgs g{};
  g.a = w.xq; g.sa = w.xs; g.b = w13; g.sb = (const float*)s13;
  g.sb_layout = sb_layout;
  g.row_index = w.tok_of_pos;
  g.out = w.out1;
  g.M = (int)R; g.N = 2 * I; g.K = H;
  g.splits = 1; g.tiles_m = 0; g.tiles_n = cdiv(2 * I, fp8::grouped_bn(p.kind)); g.group_m = 1;
  g.grouped = 1; g.tile_expert = w.tile_expert; g.tile_row0 = w.tile_row0; g.tile_rows = w.tile_rows;
  g.num_mtiles = w.num_tiles;
  g.b_expert_stride = f4 ? (long)I * H : (long)2 * I * H;
  g.sb_expert_stride = f4 ? (long)2 * I * H / 128 : (long)cdiv(2 * I, 128) * (H / 128);
  fp8::launch_gemm_grouped(p.kind, smode, g, p.max_tiles, stream);
  if (p.kind2 >= 0) {
    fp8::GemmArgs gb = g;
    gb.tiles_n = cdiv(2 * I, fp8::grouped_bn(p.kind2));
    gb.tile_expert = w.tile2_expert; gb.tile_row0 = w.tile2_row0; gb.tile_rows = w.tile2_rows;
    gb.num_mtiles = w.num_tiles2;
    fp8::launch_gemm_grouped(p.kind2, smode, gb, p.max_tiles2, stream);
  }
  TI_CHECK_LAUNCH("moe(w13)");
  // 4. swiglu x route weight -> 1x128 quant
  const long items = R * ((I / 128 + 3) / 4);
  const long sw_blocks = (items + 3) / 4;
  hipLaunchKernelGGL(swiglu_quant_kernel, dim3((unsigned)sw_blocks), dim3(256), 0, stream,
                     w.out1, I,
                     topk_weights, w.route_of_pos, w.num_rows, R, clamp_limit,
                     round_scale, w.hq, w.hs);
  TI_CHECK_LAUNCH("moe(swiglu)");
  // 5. grouped w2: [R, H] = hq . w2[e]^T
  fp8::GemmArgs g2 = g;
  g2.a = w.hq; g2.sa = w.hs; g2.b = w2; g2.sb = (const float*)s2;
  g2.row_index = nullptr;
  g2.out = w.out2;
  g2.N = H; g2.K = I;
  g2.tiles_n = cdiv(H, fp8::grouped_bn(p.kind));
  g2.b_expert_stride = f4 ? (long)H * I / 2 : (long)H * I;
  g2.sb_expert_stride = f4 ? (long)H * I / 128 : (long)cdiv(H, 128) * (I / 128);
  fp8::launch_gemm_grouped(p.kind, smode, g2, p.max_tiles, stream);
  if (p.kind2 >= 0) {
    fp8::GemmArgs gb = g2;
    gb.tiles_n = cdiv(H, fp8::grouped_bn(p.kind2));
    gb.tile_expert = w.tile2_expert; gb.tile_row0 = w.tile2_row0; gb.tile_rows = w.tile2_rows;
    gb.num_mtiles = w.num_tiles2;
    fp8::launch_gemm_grouped(p.kind2, smode, gb, p.max_tiles2, stream);
  }
  TI_CHECK_LAUNCH("moe(w2)");
  // 6. combine
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)T), dim3(256), 0, stream, w.out2, H, (const int*)topk_ids,
                     w.pos_of_route, k, (uint16_t*)out);
  TI_CHECK_LAUNCH("moe(combine)");
  return TI_OK;
}

extern "C" int ti_fp8_moe(const void* hidden, const float* topk_weights, const int32_t* topk_ids, int T, int k,
                          const uint8_t* w13, const float* s13, const uint8_t* w2, const float* s2, int E, int H,
                          int I, float clamp_limit, int round_scale, void* out, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
  return moe_run("ti_fp8_moe", 1, 0, hidden, topk_weights, topk_ids, T, k, w13, s13, w2, s2, E, H, I, clamp_limit,
                 round_scale, out, workspace, workspace_bytes, stream);
}

extern "C" int ti_fp4_moe(const void* hidden, const float* topk_weights, const int32_t* topk_ids, int T, int k,
                          const uint8_t* w13, const uint8_t* s13, const uint8_t* w2, const uint8_t* s2,
                          int scale_layout, int E, int H, int I, float clamp_limit, int round_scale, void* out,
                          void* workspace, size_t workspace_bytes, hipStream_t stream) {
  TI_CHECK_ARG(scale_layout == 0 || scale_layout == 1, "ti_fp4_moe: scale_layout must be 0 or 1");
  return moe_run("ti_fp4_moe", 2, scale_layout, hidden, topk_weights, topk_ids, T, k, w13, s13, w2, s2, E, H, I,
                 clamp_limit, round_scale, out, workspace, workspace_bytes, stream);
}
