// int4 W4A16 decode kernel for gfx950: the skinny-M (M <= 32 per row chunk)
// path of ti_w4a16_gemm.  Same arithmetic and weight layout as int4_gemm.hip
// (blocks of 16 columns x 128 rows, one 1 KiB block per wave-load, in-register
// magic-number unpack, bias-corrected MFMA sums scaled in fp32); what differs
// is how operands reach the waves.
//
// Every operand travels HBM/L2 -> LDS by direct LDS DMA
// (global_load_lds_dwordx4 / _dword), issued from inline asm so that this
// kernel, not the compiler, accounts the in-order vmcnt counter:
//   * weights: a wave's NT blocks of the next group, each a fully coalesced
//     1 KiB read that lands lane-linear in LDS (read back lane-linear);
//   * activations: the MP (16 or 32) rows x 128 K of the group, read with
//     coalesced 256 B row segments and stored XOR-swizzled (16-byte chunk q of
//     row r at slot r*16 + (q ^ (r & 15))), so the MFMA operand read -- lane
//     l takes row l%16, chunk l/16 + 4j -- is bank-conflict free;
//   * scales: the workgroup's [groups x columns] slab once, in the prologue.
// A ring of R LDS stages keeps R-1 groups in flight per wave without holding
// them in VGPRs.  One step: wait for the own DMAs of the current stage
// (s_waitcnt vmcnt(#later stages * per-stage count)), s_barrier (all waves'
// DMAs landed, and everyone finished the previous stage, whose buffer is the
// one refilled next), issue the DMAs of step i+R-1, compute step i.
//
// Workgroup = 4 waves = WK (K ranges) x WN (column sets).  Waves that share a
// K range share its activation stage; the WK partial sums are added through
// LDS in wk order at the end.  Across workgroups, `splits` K ranges are summed
// by the last-arriving workgroup of a column block in split order (agent-scope
// stores and loads of fp32 partials + a ticket), so results are deterministic.
#include "int4_decode.h"
#include "lds_dma.h"

namespace ti {
namespace int4 {

namespace {

constexpr int kWaves = 4;

template <int DT, int MR, int NT, int WK, int R, int SPLIT, int KW>
__global__ __launch_bounds__(64 * KW) void w4a16_decode_kernel(
    const uint16_t* __restrict__ A, const i32x4* __restrict__ Wp, const uint16_t* __restrict__ Sg,
    uint16_t* __restrict__ out, float* __restrict__ partial, int* __restrict__ tickets, int M, int N,
    int K, int splits) {
  constexpr int WN = KW / WK;
  constexpr int MT = MR > 16 ? MR / 16 : 1;      // 16-row MFMA tiles
  constexpr int MP = MT * 16;                    // rows of one row chunk
  constexpr int AI = WK * MR / 4;                // 1 KiB activation DMAs per stage (all waves)
  constexpr int AI_LO = AI / KW;             // ... per wave: AI_LO or AI_HI
  constexpr int AI_HI = (AI + KW - 1) / KW;
  constexpr int P = R - 1;                       // stages in flight ahead of compute
  constexpr int W_BYTES = KW * NT * 1024;    // weight blocks of one stage
  constexpr int A_BYTES = MR * 256;              // one K range's activations of one stage
  constexpr int STAGE = W_BYTES + WK * A_BYTES;
  constexpr int WC = WN * NT * 16;               // columns of the workgroup
  static_assert((NT + AI_HI) * P <= 63, "vmcnt holds at most 63 outstanding loads");

  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int last_flag;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar
  const int wk = wave / WN, wn = wave % WN;
  const int nb = blockIdx.x, split = blockIdx.y, mchunk = blockIdx.z;
  const int NG = K / kGroup;
  const long T = N / 16;
  const int m0 = mchunk * MP;
  // Activation DMAs of this wave: ids wave, wave + 4, ... below AI.
  const int a_cnt = (AI - wave + KW - 1) / KW;
  const int col_base = nb * WC;
  const long tile0 = (long)nb * (WN * NT) + wn * NT;

  // K range of the workgroup: groups [g0, g1); wave range wk: g0 + wk*nper + i.
  const int per_split = cdiv(NG, splits);
  const int g0 = split * per_split;
  const int g1 = min(NG, g0 + per_split);
  const int ngr = max(g1 - g0, 0);
  const int nper = cdiv(ngr, WK);
  const int gmax = max(g1 - 1, 0);  // clamp target: any valid group

  const uint32_t lds0 = lds_offset(smem);
  const uint32_t ring0 = lds0;
  const uint32_t sc0 = lds0 + R * STAGE;
  const uint16_t* sS = (const uint16_t*)(smem + R * STAGE);

  // ---- prologue: scales [ngr x WC] halves, dword DMA, 256 B per instruction ----
  {
    const int sbytes = ngr * WC * 2;
    const int nch = cdiv(sbytes, 256);
    for (int ch = wave; ch < nch; ch += KW) {
      const int o = ch * 256 + lane * 4;
      const uint16_t* src = Sg;
      if (o < sbytes) {
        const int gi = o / (WC * 2);
        const int cb = (o % (WC * 2)) / 2;
        src = Sg + (long)(g0 + gi) * N + col_base + cb;
      }
      dma4(src, sc0 + ch * 256);
    }
  }

  // Issue the DMAs of step `i` into ring buffer i % R.  Per-lane byte offsets
  // are fixed for the whole walk (computed here, once); per step only the
  // wave-uniform group base moves, in scalar registers.
  uint32_t woff[NT], aoff[AI_HI];
#pragma unroll
  for (int t = 0; t < NT; ++t) woff[t] = (uint32_t)(((tile0 + t) * 64 + lane) * 16);
#pragma unroll
  for (int u = 0; u < AI_HI; ++u) {
    const int id = min(wave + u * KW, AI - 1);
    const int k4 = id % (MR / 4);
    const int r = 4 * k4 + (lane >> 4);
    const int q = (lane & 15) ^ (r & 15);
    const int row = min(m0 + r, M - 1);
    aoff[u] = (uint32_t)(((long)row * K + q * 8) * 2);
  }
  auto issue = [&](int i) {
    const uint32_t base = ring0 + (uint32_t)((i % R) * STAGE);
    const int g = min(g0 + wk * nper + i, gmax);
    const char* wbase = (const char*)Wp + (long)g * T * 1024;
#pragma unroll
    for (int t = 0; t < NT; ++t) dma16_sv(wbase, woff[t], base + (uint32_t)((wave * NT + t) * 1024));
#pragma unroll
    for (int u = 0; u < AI_HI; ++u) {
      const int id = wave + u * KW;        // 0 .. AI - 1
      if (id >= AI) break;
      const int awk = id / (MR / 4), k4 = id % (MR / 4);
      const int ga = min(g0 + awk * nper + i, gmax);
      dma16_sv((const char*)A + (long)ga * kGroup * 2, aoff[u],
               base + (uint32_t)(W_BYTES + awk * A_BYTES + k4 * 1024));
    }
  };

#pragma unroll
  for (int s = 0; s < P; ++s)
    if (s < nper) issue(s);

  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int c = lane & 15, kq = lane >> 4;
  for (int i = 0; i < nper; ++i) {
    // Stages issued after stage i: min(P-1, nper-1-i).  Full-depth steps wait
    // for exactly one stage; the last P-1 steps drain.
    if (i + P - 1 < nper) {
      if (a_cnt > AI_LO) wait_vm_barrier<(P - 1) * (NT + AI_HI)>();
      else wait_vm_barrier<(P - 1) * (NT + AI_LO)>();
    } else {
      wait_vm_barrier<0>();
    }
    if (i + P < nper) issue(i + P);

    const uint8_t* st = smem + (i % R) * STAGE;
    const int g = g0 + wk * nper + i;
    const bool valid = g < g1;
    const int gl = valid ? g - g0 : 0;
    i32x4 w[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) w[t] = *(const i32x4*)(st + (wave * NT + t) * 1024 + lane * 16);
    const uint8_t* ab = st + W_BYTES + wk * A_BYTES;
    float sc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float v = scale_to_f32<DT>(sS[gl * WC + (wn * NT + t) * 16 + c]);
      sc[t] = valid ? v : 0.f;
    }
    // A operand of row tile mt, step j: row r = mt*16 + c (rows past the staged
    // MR repeat staged ones; their outputs are not stored), chunk 4j + kq.
    auto get_a = [&](int mt, int j) {
      const int r = (mt * 16 + c) % MR;
      const int q = 4 * j + kq;
      return *(const i32x4*)(ab + (r * 16 + (q ^ (r & 15))) * 16);
    };
    if constexpr (MT <= 2) {
      i32x4 a[MT][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) a[mt][j] = get_a(mt, j);
      compute_group<DT, MT, NT>(w, a, sc, acc);
    } else {
      compute_group_rows<DT, MT, NT>(w, get_a, sc, acc);
    }
  }
  // No DMA may still be writing LDS when it is reused or the workgroup ends.
  wait_vm_all();

  // ---- add the WK partial sums through LDS (fixed wk order) ----
  float* red = (float*)smem;
  if constexpr (WK > 1) {
    __syncthreads();
    if (wk > 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            red[((((wk - 1) * WN + wn) * NT + t) * MT + mt) * 256 + e * 64 + lane] = acc[t][mt][e];
    }
    __syncthreads();
  }

  const int rows = min(MP, M - m0);
  if (wk == 0) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float v = acc[t][mt][e];
#pragma unroll
          for (int w2 = 1; w2 < WK; ++w2) v += red[((((w2 - 1) * WN + wn) * NT + t) * MT + mt) * 256 + e * 64 + lane];
          const int row = mt * 16 + kq * 4 + e;
          const int col = col_base + (wn * NT + t) * 16 + c;
          if (row < rows) {
            const long off = (long)(m0 + row) * N + col;
            if constexpr (SPLIT == 0) out[off] = to_bits<DT>(v);
            else __hip_atomic_store(&partial[(long)split * M * N + off], v, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
          }
        }
  }
  if constexpr (SPLIT == 0) return;

  // Partials are written through to memory once vmcnt drains; then the ticket.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* ticket = tickets + mchunk * gridDim.x + nb;
  if (threadIdx.x == 0)
    last_flag = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
  __syncthreads();
  if (!last_flag) return;
  for (int e = threadIdx.x; e < rows * WC; e += 64 * KW) {
    const int r = e / WC;
    const long off = (long)(m0 + r) * N + col_base + e % WC;
    float v = 0.f;
    for (int sp = 0; sp < splits; ++sp)
      v += __hip_atomic_load(&partial[(long)sp * M * N + off], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out[off] = to_bits<DT>(v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT, int MR, int NT, int WK, int R, int KW = kWaves>
void launch_split(const DecodePlan& p, const DecodeArgs& x, hipStream_t stream) {
  dim3 grid(p.nblocks, p.splits, p.mchunks);
  if (p.splits == 1)
    hipLaunchKernelGGL((w4a16_decode_kernel<DT, MR, NT, WK, R, 0, KW>), grid, dim3(64 * KW), p.lds,
                       stream, x.a, x.w, x.s, x.out, x.partial, x.tickets, x.M, x.N, x.K, 1);
  else
    hipLaunchKernelGGL((w4a16_decode_kernel<DT, MR, NT, WK, R, 2, KW>), grid, dim3(64 * KW), p.lds,
                       stream, x.a, x.w, x.s, x.out, x.partial, x.tickets, x.M, x.N, x.K, p.splits);
}

template <int DT, int MR, int NT, int WK>
void launch_r(const DecodePlan& p, const DecodeArgs& x, hipStream_t stream) {
  if (p.ring <= 3) launch_split<DT, MR, NT, WK, 3>(p, x, stream);
  else if (p.ring == 4) launch_split<DT, MR, NT, WK, 4>(p, x, stream);
  else launch_split<DT, MR, NT, WK, 6>(p, x, stream);
}

template <int DT, int MR, int NT>
void launch_wk(const DecodePlan& p, const DecodeArgs& x, hipStream_t stream) {
  if (p.wk == 1) launch_r<DT, MR, NT, 1>(p, x, stream);
  else if (p.wk == 2) launch_r<DT, MR, NT, 2>(p, x, stream);
  else launch_r<DT, MR, NT, 4>(p, x, stream);
}

template <int DT, int MR>
void launch_nt(const DecodePlan& p, const DecodeArgs& x, hipStream_t stream) {
  if (p.nt == 1) launch_wk<DT, MR, 1>(p, x, stream);
  else if (p.nt == 2) launch_wk<DT, MR, 2>(p, x, stream);
  else launch_wk<DT, MR, 4>(p, x, stream);
}

// Tall tiles (64 / 128 staged rows) on 4 waves instantiate a curated set of
// (nt, wk, ring) configurations -- (2,2,2), (4,1,2|3), (2,1,2|3|4); the plan
// only produces these.
template <int DT, int MR>
void launch_tall(const DecodePlan& p, const DecodeArgs& x, hipStream_t stream) {
  if (p.wk == 2) launch_split<DT, MR, 2, 2, 2>(p, x, stream);
  else if (p.nt == 4) {
    if (p.ring == 2) launch_split<DT, MR, 4, 1, 2>(p, x, stream);
    else launch_split<DT, MR, 4, 1, 3>(p, x, stream);
  } else {
    if (p.ring == 4) launch_split<DT, MR, 2, 1, 4>(p, x, stream);
    else if (p.ring == 2) launch_split<DT, MR, 2, 1, 2>(p, x, stream);
    else launch_split<DT, MR, 2, 1, 3>(p, x, stream);
  }
}

// 8-wave workgroups (two waves per SIMD), the configurations of kEight.
template <int DT>
void launch_eight(const DecodePlan& p, const DecodeArgs& x, hipStream_t stream) {
  if (p.mr == 64) {
    if (p.nt == 4) launch_split<DT, 64, 4, 2, 2, 8>(p, x, stream);
    else if (p.ring == 2) launch_split<DT, 64, 2, 2, 2, 8>(p, x, stream);
    else launch_split<DT, 64, 2, 2, 3, 8>(p, x, stream);
  } else if (p.mr == 16) {
    if (p.nt == 4) launch_split<DT, 16, 4, 2, 3, 8>(p, x, stream);
    else if (p.nt == 1) launch_split<DT, 16, 1, 4, 6, 8>(p, x, stream);
    else if (p.wk == 2) launch_split<DT, 16, 2, 2, 4, 8>(p, x, stream);
    else launch_split<DT, 16, 2, 4, 4, 8>(p, x, stream);
  } else {
    if (p.nt == 4) launch_split<DT, 32, 4, 4, 2, 8>(p, x, stream);
    else if (p.nt == 1) launch_split<DT, 32, 1, 4, 3, 8>(p, x, stream);
    else if (p.wk == 2) launch_split<DT, 32, 2, 2, 3, 8>(p, x, stream);
    else launch_split<DT, 32, 2, 4, 3, 8>(p, x, stream);
  }
}

// 16-wave workgroups (four waves per SIMD), the configurations of kSixteen.
template <int DT>
void launch_sixteen(const DecodePlan& p, const DecodeArgs& x, hipStream_t stream) {
  if (p.mr == 64) launch_split<DT, 64, 2, 2, 2, 16>(p, x, stream);
  else if (p.mr == 32) {
    if (p.nt == 2) launch_split<DT, 32, 2, 4, 2, 16>(p, x, stream);
    else launch_split<DT, 32, 1, 4, 3, 16>(p, x, stream);
  } else {
    if (p.nt == 2) launch_split<DT, 16, 2, 4, 3, 16>(p, x, stream);
    else launch_split<DT, 16, 1, 4, 4, 16>(p, x, stream);
  }
}

template <int DT>
void launch_mr(const DecodePlan& p, const DecodeArgs& x, hipStream_t stream) {
  if (p.waves == 8) {
    launch_eight<DT>(p, x, stream);
    return;
  }
  if (p.waves == 16) {
    launch_sixteen<DT>(p, x, stream);
    return;
  }
  if (p.mr == 4) launch_nt<DT, 4>(p, x, stream);
  else if (p.mr == 16) launch_nt<DT, 16>(p, x, stream);
  else if (p.mr == 32) launch_nt<DT, 32>(p, x, stream);
  else if (p.mr == 64) launch_tall<DT, 64>(p, x, stream);
  else launch_tall<DT, 128>(p, x, stream);
}

int stage_bytes(int mr, int nt, int wk, int waves) { return waves * nt * 1024 + wk * mr * 256; }

// The instantiated 8-wave configurations (mr, nt, wk, ring): 64-row tiles with
// the K range halved, 32-row tiles with it halved or quartered.
struct EightCfg {
  int mr, nt, wk, ring;
};
constexpr EightCfg kEight[] = {{64, 4, 2, 2}, {64, 2, 2, 2}, {64, 2, 2, 3}, {32, 4, 4, 2},
                               {32, 2, 2, 3}, {32, 2, 4, 3}, {32, 1, 4, 3}, {16, 4, 2, 3},
                               {16, 2, 2, 4}, {16, 2, 4, 4}, {16, 1, 4, 6}};

// The instantiated 16-wave configurations.
constexpr EightCfg kSixteen[] = {{64, 2, 2, 2}, {32, 2, 4, 2}, {32, 1, 4, 3}, {16, 2, 4, 3}, {16, 1, 4, 4}};

bool eight_instantiated(const DecodePlan& p) {
  if (p.waves == 16) {
    for (const EightCfg& c : kSixteen)
      if (c.mr == p.mr && c.nt == p.nt && c.wk == p.wk && c.ring == p.ring) return true;
    return false;
  }
  for (const EightCfg& c : kEight)
    if (c.mr == p.mr && c.nt == p.nt && c.wk == p.wk && c.ring == p.ring) return true;
  return false;
}

bool env_plan_set() {
  const char* e = getenv("TI_ROCM_W4A16_DECODE_PLAN");
  return e && *e;
}

// TI_ROCM_W4A16_DECODE_PLAN="nt:wk:ring:splits" overrides the heuristic (tuning).
bool env_plan(DecodePlan& p) {
  const char* e = getenv("TI_ROCM_W4A16_DECODE_PLAN");
  if (!e || !*e) return false;
  int nt, wk, r, s;
  if (sscanf(e, "%d:%d:%d:%d", &nt, &wk, &r, &s) != 4) return false;
  p.nt = nt; p.wk = wk; p.ring = r; p.splits = s;
  return true;
}

// Completes a plan: snaps (nt, wk, ring) to an instantiated configuration,
// tiles N, caps splits and sizes the LDS (ring, staged scales, WK reduction).
DecodePlan finish_decode_plan(DecodePlan p, int N, int NG, bool tall) {
  if (p.waves == 8 || p.waves == 16) {
    // Snap to a table entry of this mr: the requested (nt, wk) if listed
    // (its ring), else the first whose columns tile N; none -> 4 waves.
    const EightCfg* tb = p.waves == 16 ? kSixteen : kEight;
    const int nc = p.waves == 16 ? (int)(sizeof(kSixteen) / sizeof(kSixteen[0]))
                                 : (int)(sizeof(kEight) / sizeof(kEight[0]));
    const int wv = p.waves;
    const EightCfg* pick = nullptr;
    for (int i = 0; i < nc; ++i) {
      const EightCfg& c = tb[i];
      if (c.mr == p.mr && c.nt == p.nt && c.wk == p.wk && N % (wv / c.wk * c.nt * 16) == 0 &&
          (!pick || c.ring == p.ring))
        pick = &c;
    }
    for (int i = 0; i < nc; ++i)
      if (!pick && tb[i].mr == p.mr && N % (wv / tb[i].wk * tb[i].nt * 16) == 0) pick = &tb[i];
    if (pick) {
      p.nt = pick->nt; p.wk = pick->wk; p.ring = pick->ring;
    } else {
      p.waves = kWaves;
      p.wk = 1;
    }
  }
  if (p.waves >= 8) {
    // fixed by the table entry
  } else if (tall) {
    // The instantiated tall configurations: (2,2,2), (4,1,2|3), (2,1,2|3|4); a
    // workgroup covers 256 / 128 / 64 columns, which must divide N.
    if (p.wk == 1 && p.nt >= 4 && N % 256) p.nt = 2;
    if (p.wk == 1 && p.nt < 4 && N % 128) p.wk = 2;
    if (p.wk != 1) { p.wk = 2; p.nt = 2; p.ring = 2; }
    else if (p.nt >= 4) { p.nt = 4; p.ring = p.ring <= 2 ? 2 : 3; }
    else { p.nt = 2; p.ring = p.ring >= 4 ? 4 : (p.ring <= 2 ? 2 : 3); }
  } else if (!tall) {
    if (p.nt != 1 && p.nt != 2 && p.nt != 4) p.nt = 2;
    if (p.wk != 1 && p.wk != 2 && p.wk != 4) p.wk = 1;
    if (p.ring != 3 && p.ring != 4 && p.ring != 6) p.ring = 4;
    while (p.nt > 1 && N % (kWaves / p.wk * p.nt * 16)) p.nt /= 2;
    while (p.wk < 4 && N % (kWaves / p.wk * p.nt * 16)) p.wk *= 2;
  }
  p.nblocks = N / (p.waves / p.wk * p.nt * 16);
  p.splits = max(1, min(p.splits, max(1, NG / (2 * p.wk))));
  const int ngr = cdiv(NG, p.splits);
  const int wc = p.waves / p.wk * p.nt * 16;
  const int sbytes = cdiv(ngr * wc * 2, 256) * 256;
  auto fits = [&](int r) { return r * stage_bytes(p.mr, p.nt, p.wk, p.waves) + sbytes <= kDecodeLdsMax; };
  if (p.waves >= 8) {
    // the table's ring; an oversized plan is stepped down by the caller
  } else if (tall) {
    while (p.ring > 2 && !fits(p.ring)) p.ring = p.ring == 4 ? 3 : 2;
  } else {
    while (p.ring > 3 && !fits(p.ring)) p.ring = p.ring == 6 ? 4 : 3;
  }
  const int stage = p.ring * stage_bytes(p.mr, p.nt, p.wk, p.waves) + sbytes;
  const int mt = p.mr >= 16 ? p.mr / 16 : 1;
  const int red = (p.wk - 1) * (p.waves / p.wk) * p.nt * mt * 256 * 4;
  p.lds = stage > red ? stage : red;
  return p;
}

}  // namespace

DecodePlan make_decode_plan(int M, int N, int K) {
  DecodePlan p;
  const int T = N / 16;
  const bool wide = T >= 1024;
  // Staged rows: M's own size up to 32; beyond, 32-row chunks for narrow N and
  // 64-row tiles (half the weight re-reads) for wide N.
  p.mr = M <= 4 ? 4 : (M <= 16 ? 16 : ((M <= 32 || !wide) ? 32 : 64));
  const char* emr = getenv("TI_ROCM_W4A16_DECODE_MR");
  if (emr && *emr) {
    const int v = atoi(emr);
    // 4-row tiles stage only 4 activation rows: valid for M <= 4 alone.
    if ((v == 4 && M <= 4) || v == 16 || v == 32 || v == 64 || v == 128) p.mr = v;
  }
  const bool tall = p.mr >= 64;
  p.mchunks = cdiv(M, p.mr > 16 ? p.mr : 16);
  // 32- and 64-row tiles run on 8 waves (two per SIMD, the K range split
  // between them): one wave per SIMD serializes its VALU unpack, MFMAs and LDS
  // waits.  Measured 7-19% faster than the best 4-wave plans at the
  // Llama-3-8B MLP shapes (M = 32..128); some 32-row plans take 16 (below).
  p.waves = ((p.mr == 64 && wide) || p.mr == 32 || p.mr == 16) ? 8 : kWaves;
  const int NG = K / kGroup;
  if (!env_plan(p)) {
    // Measured on MI355X at the Llama-3-8B MLP shapes, rows 9..128: wide N
    // (gate_up, N=28672) streams with whole-K workgroups; narrow N (down,
    // N=4096) puts all four waves on K (and a 2-way split at M <= 32).
    p.splits = 1;
    p.ring = 3;
    if (tall) {
      p.nt = (p.waves == 8 && M <= 64) ? 2 : 4; p.wk = p.waves == 8 ? 2 : 1; p.ring = 2;
      const int blocks = max(1, cdiv(T, kWaves * p.nt)) * p.mchunks;
      p.splits = blocks >= 192 ? 1 : cdiv(256, blocks);
    } else if (wide) {
      if (p.waves == 8) { p.nt = 2; p.wk = 2; p.ring = p.mr == 16 ? 4 : 3; }
      else if (M <= 32) { p.nt = 4; p.wk = 2; }
      else { p.nt = 2; p.wk = 1; p.ring = 4; }
    } else if (p.waves == 8) {
      // narrow N: K in quarters, 2-way split-K when K is deep (>= 64 groups:
      // the down projection; a 4096-deep K measured faster unsplit); wider
      // column sets as M grows
      p.wk = 4; p.splits = NG >= 64 ? 2 : 1;
      if (M <= 16) { p.nt = 1; p.ring = 6; }
      else if (M <= 32) { p.nt = 1; p.ring = 3; }
      else if (M <= 64) { p.nt = 2; p.ring = 3; }
      else { p.nt = 4; p.ring = 2; }
    } else {
      p.wk = 4;
      p.nt = M <= 64 ? 2 : 4;
      const int blocks = T / (p.nt * (kWaves / p.wk));
      p.splits = (M <= 32 && blocks * p.mchunks < 256) ? 2 : 1;
    }
  }
  // 32-row tiles at wide N, and at narrow N beyond 64 rows, measured 4-8%
  // faster on 16 waves (four per SIMD: 64 columns x a quarter of K each).
  if (!env_plan_set() && p.mr == 32 && (wide || M > 64)) {
    p.waves = 16; p.nt = 2; p.wk = 4; p.ring = 2;
  }
  const char* ew = getenv("TI_ROCM_W4A16_DECODE_WAVES");
  if (ew && *ew && (p.mr == 16 || p.mr == 32 || p.mr == 64)) {
    const int v = atoi(ew);
    p.waves = (v == 8 || v == 16) ? v : kWaves;
  }
  DecodePlan q = finish_decode_plan(p, N, NG, tall);
  // An 8-wave plan whose LDS (ring + the staged scale slab, which grows with
  // K) does not fit steps down to half the columns, then to the 4-wave table.
  if (q.waves >= 8 && q.lds > kDecodeLdsMax && q.nt >= 2) {
    p.nt = q.nt / 2;
    p.wk = q.wk;
    q = finish_decode_plan(p, N, NG, tall);
  }
  if (q.waves >= 8 && q.lds > kDecodeLdsMax) {
    p.waves = kWaves;
    p.wk = 1;
    q = finish_decode_plan(p, N, NG, tall);
  }
  return q;
}

bool decode_plan_valid(const DecodePlan& p, int N) {
  if (p.waves != 4 && p.waves != 8 && p.waves != 16) return false;
  if (N % (p.waves / p.wk * p.nt * 16) || p.nblocks * (p.waves / p.wk * p.nt * 16) != N) return false;
  if (p.lds > kDecodeLdsMax) return false;
  if (p.waves >= 8) return eight_instantiated(p);
  if (p.mr >= 64)
    return (p.nt == 2 && p.wk == 2 && p.ring == 2) || (p.nt == 4 && p.wk == 1 && (p.ring == 2 || p.ring == 3)) ||
           (p.nt == 2 && p.wk == 1 && (p.ring >= 2 && p.ring <= 4));
  return (p.nt == 1 || p.nt == 2 || p.nt == 4) && (p.wk == 1 || p.wk == 2 || p.wk == 4) &&
         (p.ring == 3 || p.ring == 4 || p.ring == 6) && (p.mr == 4 || p.mr == 16 || p.mr == 32);
}

size_t decode_ticket_bytes(const DecodePlan& p) {
  return ((size_t)p.nblocks * p.mchunks * sizeof(int) + 255) & ~(size_t)255;
}

size_t decode_partial_bytes(const DecodePlan& p, int M, int N) {
  return p.splits > 1 ? (size_t)p.splits * M * N * sizeof(float) : 0;
}

void launch_decode(const DecodePlan& p, int dtype, const DecodeArgs& x, hipStream_t stream) {
  if (dtype == TI_DTYPE_F16) launch_mr<TI_DTYPE_F16>(p, x, stream);
  else launch_mr<TI_DTYPE_BF16>(p, x, stream);
}

}  // namespace int4
}  // namespace ti
