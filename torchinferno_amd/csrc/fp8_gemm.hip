// FP8 e4m3 W8A8 GEMM for gfx950: C[M,N] = A[M,K] . B[N,K]^T with
//   * row/column scales  (SMODE 0): C = acc * sa[m] * sb[n]; sa/sb may also be
//     scalars -- the per-token x per-channel and tensorwise linears of
//     src/torchinferno/kernels/fp8.py:184-327 (torch._scaled_mm, sgl cutlass,
//     src/torchinferno/kernels/csrc/sgl_fp8_out.cpp:17-83);
//   * 128x128 block scales (SMODE 1): every 128-wide K block's partial sum is
//     scaled by sa[m, kb] * sb[n / 128, kb] and added into an fp32
//     accumulator -- DeepSeek fp8_gemm,
//     src/torchinferno/kernels/deepseek_v4_tilelang_definitions.py:436-485;
//   * MXFP4 weights (SMODE 2): B is e2m1, two per byte along K, with one E8M0
//     scale per 32 K of a row, applied by the MFMA itself (its per-lane block
//     scale operand); A keeps its 1x128 fp32 scales, folded per K step --
//     DeepSeek fp4_gemm, deepseek_v4_tilelang_definitions.py:674-769;
//   * power-of-two block scales (SMODE 3: block FP8; SMODE 4: MXFP4 with
//     power-of-two activation scales) -- DeepSeek-V4's ue8m0 format
//     (scale_dtype float8_e8m0fnu, deepseek_v4_tilelang.py:207-223): every
//     scale is an exponent, so the MFMA's per-lane E8M0 scale operands apply
//     both of them and the partial sums accumulate in the MFMA with no fold.
// A (and B outside SMODE 2) are K-contiguous e4m3 (OCP float8_e4m3fn,
// gfx950's native FP8).
//
// Structure.  A workgroup owns a BM x BN output tile and walks K in steps of
// 128 bytes.  Each step's A and B slabs (BM and BN rows of 128 B) reach LDS by
// direct DMA (global_load_lds_dwordx4, issued from inline asm with explicit
// vmcnt accounting) through a ring of R stages; block mode also DMAs the
// step's BM activation scales.  Rows are stored with their eight 16-byte
// chunks XOR-swizzled (chunk c of row r at position c ^ ((r >> 1) & 7)): the
// DMA side reads whole 128 B row segments (coalesced), and the MFMA operand
// reads -- 16 lanes on 16 consecutive rows, same chunk -- hit 16 distinct
// bank groups.  Waves form a WGM x WGN grid over the tile; each runs
// v_mfma_scale_f32_{32x32x64,16x16x128}_f8f6f4 with unit scales (e8m0 127).
// Both operands give lane l row (l % MF) and the same 32 K bytes, so every
// MFMA k-slot pairs A and B at one true k.
//
// Split-K (SPLIT 2, skinny M): `splits` workgroups share a tile; each writes
// an fp32 partial with agent-scope stores, takes a ticket, and the last one
// sums the partials in split order (deterministic) and stores C.
//
// Tile order: WG t is dispatched to XCD t % 8; t is remapped so that each XCD
// works through one contiguous run of a GM-row grouped raster, keeping the A
// and B slabs its L2 holds shared by the tiles in flight there.
#include "fp8_common.h"
#include "fp8_gemm.h"
#include "lds_dma.h"

namespace ti {
namespace fp8 {
namespace {

template <int MF>
struct Mfma;

template <>
struct Mfma<32> {
  typedef f32x16 acc_t;
  static constexpr int KS = 2;   // MFMAs per 128-byte K step
  static constexpr int NACC = 16;
  static __device__ __forceinline__ acc_t mma(i32x8 a, i32x8 b, acc_t c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
  }
  // e4m3 A x e2m1 B (blgp 4: the low four dwords of b), B block scale e8m0 eb.
  static __device__ __forceinline__ acc_t mma4(i32x8 a, i32x8 b, acc_t c, int eb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 4, 0, 127, 0, eb);
  }
  // E8M0 scales ea (A row of this lane) and eb (B row of this lane), each
  // covering the lane's 32 K values.
  static __device__ __forceinline__ acc_t mma_s(i32x8 a, i32x8 b, acc_t c, int ea, int eb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, ea, 0, eb);
  }
  static __device__ __forceinline__ acc_t mma4_s(i32x8 a, i32x8 b, acc_t c, int ea, int eb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 4, 0, ea, 0, eb);
  }
  // Row (within the 32x32 tile) of accumulator element e of this lane.
  static __device__ __forceinline__ int row(int e, int lane) { return 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3); }
  // First of the two 16-byte chunks (of the 128-byte K step) lane reads for MFMA ks.
  static __device__ __forceinline__ int chunk(int ks, int lane) { return ks * 4 + (lane >> 5) * 2; }
  // 16-byte chunk of a 64-byte e2m1 row (32 values) lane reads for MFMA ks;
  // it is also the row's 32-wide scale block within the K step.
  static __device__ __forceinline__ int chunk4(int ks, int lane) { return ks * 2 + (lane >> 5); }
  // Against an e2m1 B the 8-bit A operand must follow the MFMA's own K order:
  // lane group g's first 16 bytes are K [16g, 16g+16) of the 64-wide window,
  // its last 16 bytes K [32+16g, +16), while the e2m1 operand's 16 bytes are
  // K [32g, 32g+32).  (e4m3 x e4m3 loads both operands alike, so any order
  // works there.)  First A chunk; the second is CHUNK_A4_HI further.
  static __device__ __forceinline__ int chunk_a4(int ks, int lane) { return ks * 4 + (lane >> 5); }
  static constexpr int CHUNK_A4_HI = 2;
};

template <>
struct Mfma<16> {
  typedef f32x4 acc_t;
  static constexpr int KS = 1;
  static constexpr int NACC = 4;
  static __device__ __forceinline__ acc_t mma(i32x8 a, i32x8 b, acc_t c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
  }
  static __device__ __forceinline__ acc_t mma4(i32x8 a, i32x8 b, acc_t c, int eb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, 0, 127, 0, eb);
  }
  static __device__ __forceinline__ acc_t mma_s(i32x8 a, i32x8 b, acc_t c, int ea, int eb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, ea, 0, eb);
  }
  static __device__ __forceinline__ acc_t mma4_s(i32x8 a, i32x8 b, acc_t c, int ea, int eb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 4, 0, ea, 0, eb);
  }
  static __device__ __forceinline__ int row(int e, int lane) { return 4 * (lane >> 4) + e; }
  static __device__ __forceinline__ int chunk(int, int lane) { return (lane >> 4) * 2; }
  static __device__ __forceinline__ int chunk4(int, int lane) { return lane >> 4; }
  // 16x16x128: lane group q holds K [16q, +16) and [64+16q, +16) of an 8-bit
  // operand, K [32q, +32) of an e2m1 one.
  static __device__ __forceinline__ int chunk_a4(int, int lane) { return lane >> 4; }
  static constexpr int CHUNK_A4_HI = 4;
};

// Byte offset of 16-byte chunk c of row r in a swizzled [rows x BK bytes] slab:
// CPR = BK/16 chunks per row, RP = 256/BK rows per 256-byte bank period; chunk c
// sits at position c ^ ((r / RP) % CPR), so 16 consecutive rows reading one
// chunk cover all 64 banks.
template <int BK>
__device__ __forceinline__ int swz(int r, int c) {
  constexpr int CPR = BK / 16, RP = 256 / BK;  // BK: bytes per row
  return (r * CPR + (c ^ ((r / RP) % CPR))) * 16;
}

// E8M0 byte of a power-of-two fp32 scale: its exponent field (2^-127, the
// subnormal 0x00400000, gives 0 as well).
__device__ __forceinline__ int e8m0_of(float s) { return (int)((__float_as_uint(s) >> 23) & 0xFFu); }

template <int ODT>
__device__ __forceinline__ uint16_t out_bits(float v) {
  if constexpr (ODT == TI_DTYPE_F16) return f32_to_f16_bits(v);
  else return f32_to_bf16_bits(v);
}

template <int BM, int BN, int BK, int WGM, int WGN, int MF, int R, int SMODE, int SPLIT, int ODT>
__global__ __launch_bounds__(64 * WGM * WGN) void fp8_gemm_kernel(GemmArgs x) {
  using MM = Mfma<MF>;
  typedef typename MM::acc_t acc_t;
  constexpr int W = WGM * WGN;
  constexpr int TM = BM / WGM, TN = BN / WGN;
  constexpr int FM = TM / MF, FN = TN / MF;
  static_assert(FM >= 1 && FN >= 1 && TM % MF == 0 && TN % MF == 0, "wave tile must hold whole MFMA tiles");
  constexpr bool BLK = SMODE == 1 || SMODE == 3;  // 128x128 block weight scales
  constexpr bool F4 = SMODE == 2 || SMODE == 4;   // e2m1 B with E8M0 scales per 32 K
  constexpr bool PW2 = SMODE >= 3;                // all scales powers of two, applied by the MFMA
  static_assert(!BLK || 128 % TN == 0, "block scales need a wave's columns inside one 128 block");
  static_assert(BK == 128 || (BK == 64 && MF == 32), "16x16x128 MFMAs need 128-byte K steps");
  static_assert(!F4 || BK == 128, "e2m1 B takes 128-wide K steps (64-byte rows)");
  constexpr int BROW = F4 ? BK / 2 : BK;           // B bytes per row per K step
  constexpr int KS = BK / (MF == 32 ? 64 : 128);  // MFMAs per K step
  constexpr int CPR = BK / 16;                     // 16-byte chunks per row
  constexpr int RPI = 1024 / BK;                   // rows per 1 KiB DMA
  constexpr int A_BYTES = BM * BK, B_BYTES = BN * BROW;
  // Block and MXFP4 modes also stage the step's BM activation scales; block
  // mode then the weight scales of the tile's 128-column blocks (one 256-byte
  // DMA), MXFP4 mode the BN rows' four e8m0 bytes of the step (one dword each).
  constexpr int SA_ROWS = SMODE >= 1 ? ((BM * 4 + 255) / 256) * 256 : 0;
  constexpr int SB_BYTES = BLK ? 256 : (F4 ? ((BN * 4 + 255) / 256) * 256 : 0);
  constexpr int SA_BYTES = SA_ROWS + SB_BYTES;
  constexpr int STAGE = A_BYTES + B_BYTES + SA_BYTES;
  constexpr int NI_AB = (A_BYTES + B_BYTES) / 1024;
  constexpr int NI_SA = SA_ROWS / 256;
  constexpr int NI = NI_AB + NI_SA + SB_BYTES / 256;  // DMAs per stage, all waves
  constexpr int NI_LO = NI / W, NI_HI = (NI + W - 1) / W;
  constexpr int P = R - 1;
  static_assert(R >= 2, "ring needs two stages");
  static_assert(NI_HI * (P > 1 ? P - 1 : 1) <= 63, "vmcnt holds at most 63 outstanding loads");

  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ int last_flag;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WGN, wn = wave % WGN;
  const int M = x.M, N = x.N, K = x.K;
  const int KT = K / BK;      // K steps
  const int KB = K / 128;     // 128-wide scale blocks

  // ---- tile of this workgroup ----
  int m0, n0, Mlim;
  const uint8_t* bmat = x.b;
  const float* sbmat = x.sb;
  const int tiles_n = x.tiles_n;
  if (x.grouped) {
    // Grouped (MoE) launch: blockIdx.x = m-tile * tiles_n + n-tile over a device
    // table of (expert, first row, rows) m-tiles; surplus workgroups exit.
    const int mt = blockIdx.x / tiles_n;
    if (mt >= *x.num_mtiles) return;
    const int e = x.tile_expert[mt];
    m0 = x.tile_row0[mt];
    Mlim = m0 + x.tile_rows[mt];
    n0 = (blockIdx.x % tiles_n) * BN;
    bmat += (long)e * x.b_expert_stride;
    sbmat += (long)e * x.sb_expert_stride;
  } else {
    // XCD-contiguous runs of a grouped raster.
    int t = blockIdx.x;
    const int nt = gridDim.x;
    if ((nt & 7) == 0) t = (t & 7) * (nt >> 3) + (t >> 3);
    const int tiles_m = x.tiles_m;
    const int GM = x.group_m;
    const int group = t / (GM * tiles_n);
    const int first_m = group * GM;
    const int gsz = min(tiles_m - first_m, GM);
    const int tin = t - group * GM * tiles_n;
    m0 = (first_m + tin % gsz) * BM;
    n0 = (tin / gsz) * BN;
    Mlim = M;
  }

  const int split = blockIdx.y;
  const int per = cdiv(KT, x.splits);
  const int ks0 = split * per;
  const int nsteps = max(min(KT, ks0 + per) - ks0, 0);

  const uint32_t ring0 = lds_offset(smem);
  const int n_mine = (NI - wave + W - 1) / W;  // DMAs of this wave per stage

  // Source row pointer, per-step stride multiplier and LDS offset of each of
  // this wave's DMAs, fixed for the whole K walk (gather indices are read here,
  // once, so no ordinary load sits between the ring's DMAs).
  const uint8_t* dsrc[NI_HI];
  uint32_t dlds[NI_HI];
  bool dwide[NI_HI];
  int dstep[NI_HI];     // source bytes per K step, or per 128 K for the scale entries
  bool dper128[NI_HI];  // scale entry: advances every 128 K (a 64-wide step reads one twice)
#pragma unroll
  for (int u = 0; u < NI_HI; ++u) {
    const int id = min(wave + u * W, NI - 1);
    dstep[u] = BK;
    dper128[u] = false;
    if (id < NI_AB) {
      const bool is_a = id < A_BYTES / 1024;
      const int j = is_a ? id : id - A_BYTES / 1024;
      const int rowb = is_a ? BK : BROW;  // slab bytes per row
      const int cpr = rowb / 16;
      const int r = (1024 / rowb) * j + lane / cpr;
      const int c = (lane % cpr) ^ ((r / (256 / rowb)) % cpr);
      long row;
      if (is_a) {
        row = min(m0 + r, Mlim - 1);
        if (x.row_index) row = x.row_index[row];
      } else {
        row = min(n0 + r, N - 1);
      }
      dsrc[u] = is_a ? x.a + row * K + c * 16 : bmat + row * (F4 ? K / 2 : K) + c * 16;
      dstep[u] = rowb;
      if (SMODE == 0 && !is_a && x.b_tiled) {
        // tiled weights (per-token / tensorwise mode only): each K step of 128 rows is one contiguous 16 KiB run
        dsrc[u] = bmat + (row >> 7) * (128L * K) + (row & 127) * 128 + c * 16;
        dstep[u] = 128 * 128;
      }
      dlds[u] = (uint32_t)((is_a ? 0 : A_BYTES) + j * 1024);
      dwide[u] = true;
    } else if (id < NI_AB + NI_SA) {
      const int j = id - NI_AB;
      long row = min(m0 + min(j * 64 + lane, BM - 1), Mlim - 1);
      if (x.row_index) row = x.row_index[row];
      // [M, K/128]: one scattered dword per row; step-major [K/128][M]: the
      // tile's rows adjacent.
      dsrc[u] = (const uint8_t*)(x.sa + (x.sa_layout ? row : row * KB));
      dlds[u] = (uint32_t)(A_BYTES + B_BYTES + j * 256);
      dwide[u] = false;
      dstep[u] = x.sa_layout ? M * 4 : 4;
      dper128[u] = true;
    } else if constexpr (BLK) {
      // Only the column blocks the tile overlaps are read (a BN that is not a
      // multiple of 128 may start inside a block and overlap one more); the
      // other lanes repeat the last one (one cache line per step instead of 64).
      constexpr int NBLK = (BN + 127) / 128 + (BN % 128 != 0);
      const int nb = min(n0 / 128 + min(lane, NBLK - 1), (N + 127) / 128 - 1);
      dsrc[u] = (const uint8_t*)(sbmat + (long)nb * KB);
      dlds[u] = (uint32_t)(A_BYTES + B_BYTES + NI_SA * 256);
      dwide[u] = false;
      dstep[u] = 4;
      dper128[u] = true;
    } else {
      // e8m0 bytes, the row's dword of K step kk: [N, K/32] layout at byte
      // nrow * K/32 + 4*kk (one dword per row: scattered), step-major
      // [K/128][N][4] at byte (kk * N + nrow) * 4 (the tile's rows contiguous).
      const int j = id - NI_AB - NI_SA;
      const int nrow = min(n0 + j * 64 + lane, N - 1);
      dsrc[u] = (const uint8_t*)sbmat + (x.sb_layout ? (long)nrow * 4 : (long)nrow * (K / 32));
      dlds[u] = (uint32_t)(A_BYTES + B_BYTES + SA_ROWS + j * 256);
      dwide[u] = false;
      dstep[u] = x.sb_layout ? N * 4 : 4;
    }
  }

  auto issue = [&](int i) {
    const uint32_t base = ring0 + (uint32_t)((i % R) * STAGE);
    const long kk = ks0 + i;
#pragma unroll
    for (int u = 0; u < NI_HI; ++u) {
      if (wave + u * W >= NI) break;
      if (dwide[u]) dma16(dsrc[u] + kk * dstep[u], base + dlds[u]);
      else dma4(dsrc[u] + (dper128[u] ? (kk * BK / 128) * dstep[u] : kk * dstep[u]), base + dlds[u]);
    }
  };

#pragma unroll
  for (int s = 0; s < P; ++s)
    if (s < nsteps) issue(s);

  acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < MM::NACC; ++e) acc[i][j][e] = 0.f;
  // Scaled modes fold each step's partial sums into acc with a per-row scale.
  // Small wave tiles defer that fold by one step: the fold of step i-1 runs
  // while step i's MFMAs execute, instead of waiting on their result (with
  // one wave per SIMD nothing else hides that latency).  Same products and
  // association, so the same results.  pd/sd: the deferred partials and
  // scales (zero before the first step: acc + 0*0 = acc).
  constexpr bool DEFER = (SMODE == 1 || SMODE == 2) && FM * FN * MM::NACC <= 32;
  // Block mode with deferred folds forms the row-scale products once per
  // wave in LDS (the wave's TM products, one per lane) rather than once per
  // accumulator row in every lane.
  constexpr bool LDS_PROD = SMODE == 1 && DEFER && FM * MM::NACC >= 16;
  // Two buffers, alternated by the parity of the step (a compile-time index:
  // the K loop is unrolled by two), so no register copies carry them over.
  acc_t pd[DEFER ? 2 : 1][DEFER ? FM : 1][DEFER ? FN : 1];
  float sd[DEFER ? 2 : 1][DEFER ? FM : 1][MM::NACC];
#pragma unroll
  for (int q = 0; q < (DEFER ? 2 : 1); ++q)
#pragma unroll
    for (int i = 0; i < (DEFER ? FM : 1); ++i) {
#pragma unroll
      for (int e = 0; e < MM::NACC; ++e) sd[q][i][e] = 0.f;
#pragma unroll
      for (int j = 0; j < (DEFER ? FN : 1); ++j)
#pragma unroll
        for (int e = 0; e < MM::NACC; ++e) pd[q][i][j][e] = 0.f;
    }
  // Step parity Q: fold the other buffer (the previous step), keep this one.
  auto fold = [&](auto Q, int fm, int fn, const acc_t& p, const float (&srow)[MM::NACC]) {
    constexpr int q = decltype(Q)::value;
    if constexpr (DEFER) {
#pragma unroll
      for (int e = 0; e < MM::NACC; ++e)
        acc[fm][fn][e] = __builtin_fmaf(pd[1 - q][fm][fn][e], sd[1 - q][fm][e], acc[fm][fn][e]);
      pd[q][fm][fn] = p;
    } else {
#pragma unroll
      for (int e = 0; e < MM::NACC; ++e) acc[fm][fn][e] = __builtin_fmaf(p[e], srow[e], acc[fm][fn][e]);
    }
  };

  const int arow0 = wm * TM + (lane % MF);
  const int brow0 = wn * TN + (lane % MF);

  // Step i reads ring stage i % R, at byte offset soff (kept by the caller).
  auto step = [&](int i, int soff, auto Q) {
    constexpr int q = decltype(Q)::value;
    if (i + P - 1 < nsteps) {
      if constexpr (P > 1) {
        if (n_mine > NI_LO) wait_vm_barrier<(P - 1) * NI_HI>();
        else wait_vm_barrier<(P - 1) * NI_LO>();
      } else {
        wait_vm_barrier<0>();
      }
    } else {
      wait_vm_barrier<0>();
    }
    if (i + P < nsteps) issue(i + P);

    const uint8_t* st = smem + soff;
    const uint8_t* sA = st;
    const uint8_t* sB = st + A_BYTES;
    if constexpr (SMODE == 0 || SMODE == 3) {
      // Power-of-two block scales: this lane's A row exponent per M tile and
      // the wave's column block exponent (one 128 block per wave).
      int ea[FM], ebv = 127;
      if constexpr (SMODE == 3) {
        const float* sS = (const float*)(st + A_BYTES + B_BYTES);
        ebv = e8m0_of(sS[NI_SA * 64 + (n0 % 128 + wn * TN) / 128]);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) ea[fm] = e8m0_of(sS[wm * TM + fm * MF + lane % MF]);
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int c0 = MM::chunk(ks, lane);
        i32x8 af[FM], bf[FN];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          const int r = arow0 + fm * MF;
          const i32x4 lo = *(const i32x4*)(sA + swz<BK>(r, c0));
          const i32x4 hi = *(const i32x4*)(sA + swz<BK>(r, c0 + 1));
          af[fm] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int r = brow0 + fn * MF;
          const i32x4 lo = *(const i32x4*)(sB + swz<BK>(r, c0));
          const i32x4 hi = *(const i32x4*)(sB + swz<BK>(r, c0 + 1));
          bf[fn] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            if constexpr (SMODE == 3) acc[fm][fn] = MM::mma_s(af[fm], bf[fn], acc[fm][fn], ea[fm], ebv);
            else acc[fm][fn] = MM::mma(af[fm], bf[fn], acc[fm][fn]);
          }
      }
    } else if constexpr (F4) {
      const float* sS = (const float*)(st + A_BYTES + B_BYTES);
      const uint32_t* sE = (const uint32_t*)(st + A_BYTES + B_BYTES + SA_ROWS);
      // B fragments (16 bytes = 32 e2m1 values per lane) and their e8m0 block
      // scales for the whole step; A is read one M tile at a time.
      i32x8 bf[KS][FN];
      int eb[KS][FN];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int q = MM::chunk4(ks, lane);
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int r = brow0 + fn * MF;
          const i32x4 lo = *(const i32x4*)(sB + swz<BROW>(r, q));
          bf[ks][fn] = i32x8{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
          eb[ks][fn] = (int)((sE[r] >> (8 * q)) & 0xFFu);
        }
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        i32x8 af[KS];
        const int r = arow0 + fm * MF;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int c0 = MM::chunk_a4(ks, lane);
          const i32x4 lo = *(const i32x4*)(sA + swz<BK>(r, c0));
          const i32x4 hi = *(const i32x4*)(sA + swz<BK>(r, c0 + MM::CHUNK_A4_HI));
          af[ks] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        if constexpr (PW2) {
          // power-of-two activation scales: the MFMA applies both exponents
          const int ea = e8m0_of(sS[wm * TM + fm * MF + lane % MF]);
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) acc[fm][fn] = MM::mma4_s(af[ks], bf[ks][fn], acc[fm][fn], ea, eb[ks][fn]);
          continue;
        }
        float srow[MM::NACC];
#pragma unroll
        for (int e = 0; e < MM::NACC; ++e) srow[e] = sS[wm * TM + fm * MF + MM::row(e, lane)];
        // All FN partial sums first, then their folds: each fold then
        // waits only on its own MFMA chain, the later chains still running.
        acc_t pf[FN];
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
          for (int e = 0; e < MM::NACC; ++e) pf[fn][e] = 0.f;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) pf[fn] = MM::mma4(af[ks], bf[ks][fn], pf[fn], eb[ks][fn]);
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) fold(Q, fm, fn, pf[fn], srow);
        if constexpr (DEFER) {
#pragma unroll
          for (int e = 0; e < MM::NACC; ++e) sd[q][fm][e] = srow[e];
        }
      }
    } else {
      const float* sS = (const float*)(st + A_BYTES + B_BYTES);
      const float sbv = sS[NI_SA * 64 + (n0 % 128 + wn * TN) / 128];  // the wave's column block
      // LDS_PROD: the wave's TM row scales times its column block's scale,
      // one product per lane, through the wave's own LDS slot (a wave's LDS
      // accesses complete in order, so its reads below see its writes).
      float* wsc = (float*)(smem + R * STAGE) + wave * TM;
      if constexpr (LDS_PROD) {
#pragma unroll
        for (int j = 0; j < TM; j += 64)
          if (TM % 64 == 0 || j + lane < TM) wsc[j + lane] = sS[wm * TM + j + lane] * sbv;
        __builtin_amdgcn_wave_barrier();
      }
      // All B fragments of the step stay in registers; A is read one M tile
      // at a time (bounds register use with the per-tile partial sums).
      i32x8 bf[KS][FN];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int c0 = MM::chunk(ks, lane);
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int r = brow0 + fn * MF;
          const i32x4 lo = *(const i32x4*)(sB + swz<BK>(r, c0));
          const i32x4 hi = *(const i32x4*)(sB + swz<BK>(r, c0 + 1));
          bf[ks][fn] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        i32x8 af[KS];
        const int r = arow0 + fm * MF;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const int c0 = MM::chunk(ks, lane);
          const i32x4 lo = *(const i32x4*)(sA + swz<BK>(r, c0));
          const i32x4 hi = *(const i32x4*)(sA + swz<BK>(r, c0 + 1));
          af[ks] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        float srow[MM::NACC];
#pragma unroll
        for (int e = 0; e < MM::NACC; ++e)
          srow[e] = LDS_PROD ? wsc[fm * MF + MM::row(e, lane)] : sS[wm * TM + fm * MF + MM::row(e, lane)] * sbv;
        // All FN partial sums first, then their folds: each fold then
        // waits only on its own MFMA chain, the later chains still running.
        acc_t pf[FN];
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
          for (int e = 0; e < MM::NACC; ++e) pf[fn][e] = 0.f;
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) pf[fn] = MM::mma(af[ks], bf[ks][fn], pf[fn]);
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) fold(Q, fm, fn, pf[fn], srow);
        if constexpr (DEFER) {
#pragma unroll
          for (int e = 0; e < MM::NACC; ++e) sd[q][fm][e] = srow[e];
        }
      }
    }
  };
  auto next_stage = [](int soff) { return soff == (R - 1) * STAGE ? 0 : soff + STAGE; };
  using Q0 = std::integral_constant<int, 0>;
  using Q1 = std::integral_constant<int, 1>;
  if constexpr (DEFER) {
    // Unrolled by two so the deferred buffers alternate at compile time; the
    // last fold takes the buffer of the last step's parity.
    auto fold_last = [&](auto Q) {
      constexpr int q = decltype(Q)::value;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int e = 0; e < MM::NACC; ++e)
            acc[fm][fn][e] = __builtin_fmaf(pd[q][fm][fn][e], sd[q][fm][e], acc[fm][fn][e]);
    };
    int i = 0, soff = 0;
    for (; i + 1 < nsteps; i += 2) {
      step(i, soff, Q0{});
      soff = next_stage(soff);
      step(i + 1, soff, Q1{});
      soff = next_stage(soff);
    }
    if (i < nsteps) {
      step(i, soff, Q0{});
      fold_last(Q0{});
    } else {
      fold_last(Q1{});
    }
  } else {
    for (int i = 0; i < nsteps; ++i) step(i, (i % R) * STAGE, Q0{});
  }
  wait_vm_all();

  // ---- epilogue ----
  const int col_l = lane % MF;
  // Split-K: each split's fp32 partial of the tile goes to the tile's own
  // BM x BN region of the workspace with device-coherent stores, and the last
  // split of the tile to finish sums the splits in split order.  A tile whose
  // rows all lie below M stores in the register layout (float i of lane l of
  // wave w at (w * PER + i) * 64 + l: each store instruction writes 256
  // contiguous bytes) and is summed back into the registers, then stored like
  // an unsplit tile; a tile that overhangs M (small M) stores only its rows
  // below M, row-major, and the last split sums and stores element-wise.
  constexpr int PER = FM * FN * MM::NACC;  // accumulator floats per lane
  if constexpr (SPLIT != 0) {
    const int split = blockIdx.y;
    const bool full = m0 + BM <= M;  // uniform over the workgroup and its splits
    auto region = [&](int sp) { return x.partial + ((long)sp * gridDim.x + blockIdx.x) * ((long)BM * BN); };
    const long lane_base = (long)wave * PER * 64 + lane;
    if (full) {
      float* mine = region(split) + lane_base;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int e = 0; e < MM::NACC; ++e)
            __hip_atomic_store(mine + ((fm * FN + fn) * MM::NACC + e) * 64, acc[fm][fn][e], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    } else {
      float* mine = region(split);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          const int c = wn * TN + fn * MF + col_l;
#pragma unroll
          for (int e = 0; e < MM::NACC; ++e) {
            const int r = wm * TM + fm * MF + MM::row(e, lane);
            if (m0 + r < M)
              __hip_atomic_store(mine + r * BN + c, acc[fm][fn][e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    int* ticket = x.tickets + blockIdx.x;
    if (threadIdx.x == 0)
      last_flag = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == x.splits - 1;
    __syncthreads();
    if (!last_flag) return;
    if (!full) {
      const int rows = M - m0, cols = min(BN, N - n0);
      for (int e = threadIdx.x; e < rows * cols; e += 64 * W) {
        const int r = e / cols, c = e % cols;
        float v = 0.f;
        for (int sp = 0; sp < x.splits; ++sp)
          v += __hip_atomic_load(region(sp) + r * BN + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int row = m0 + r, col = n0 + c;
        if constexpr (SMODE == 0) v = v * x.sa[(long)row * x.sa_stride] * x.sb[(long)col * x.sb_stride];
        x.out[(long)row * N + col] = out_bits<ODT>(v);
      }
      if (threadIdx.x == 0) __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int e = 0; e < MM::NACC; ++e) acc[fm][fn][e] = 0.f;
    for (int sp = 0; sp < x.splits; ++sp) {
      const float* src = region(sp) + lane_base;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int e = 0; e < MM::NACC; ++e)
            acc[fm][fn][e] += __hip_atomic_load(src + ((fm * FN + fn) * MM::NACC + e) * 64, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    }
    if (threadIdx.x == 0) __hip_atomic_store(ticket, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // Row / column scales of this lane's outputs, loaded up front with clamped
  // indices (no load sits behind a bounds branch, so they are all in flight
  // together), then the stores, unconditional for a per-token tile inside M and
  // N (measured 2% faster at gate_up M=4096; the scaled modes keep the bounds
  // test, which measured faster there).
  float sarow[SMODE == 0 ? FM : 1][MM::NACC], sbcol[SMODE == 0 ? FN : 1];
  if constexpr (SMODE == 0) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int e = 0; e < MM::NACC; ++e) {
        const int row = min(m0 + wm * TM + fm * MF + MM::row(e, lane), Mlim - 1);
        sarow[fm][e] = x.sa[(long)row * x.sa_stride];
      }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) sbcol[fn] = x.sb[(long)min(n0 + wn * TN + fn * MF + col_l, N - 1) * x.sb_stride];
  }
  const bool inside = SMODE == 0 && m0 + BM <= Mlim && n0 + BN <= N;  // uniform over the workgroup
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int col = n0 + wn * TN + fn * MF + col_l;
#pragma unroll
      for (int e = 0; e < MM::NACC; ++e) {
        const int row = m0 + wm * TM + fm * MF + MM::row(e, lane);
        float v = acc[fm][fn][e];
        if constexpr (SMODE == 0) v = v * sarow[fm][e] * sbcol[fn];
        if (inside || (row < Mlim && col < N)) x.out[(long)row * N + col] = out_bits<ODT>(v);
      }
    }
}

// ---------------------------------------------------------------------------
// Tile configurations (kind):                                        K step  stages
//   0  BM=256 BN=256, 8 waves 2x4 (wave 128x64),  32x32 MFMA            64      4   -- prefill
//   1  BM=256 BN=256, 8 waves 2x4 (wave 128x64),  32x32 MFMA            128     2   -- prefill
//   2  BM=128 BN=128, 4 waves 2x2 (wave 64x64),   32x32 MFMA            128     3   -- mid M
//   3  BM=16  BN=256, 4 waves 1x4 (wave 16x64),   16x16 MFMA            128     4   -- decode
//   4  BM=32  BN=256, 4 waves 1x4 (wave 32x64),   16x16 MFMA            128     4   -- decode
//   5  BM=64  BN=128, 4 waves 1x4 (wave 64x32),   16x16 MFMA            128     4   -- small M
//   6  BM=16  BN=128, 4 waves 1x4 (wave 16x32),   16x16 MFMA            128     6   -- decode
//   7  BM=128 BN=128, 4 waves 2x2 (wave 64x64),   32x32 MFMA            64      6   -- mid M
//   8  BM=256 BN=128, 4 waves 2x2 (wave 128x64),  32x32 MFMA            64      6   -- prefill
//   9  BM=256 BN=128, 8 waves 4x2 (wave 64x64),   32x32 MFMA            128     3   -- prefill
//  10  BM=16  BN=256, 8 waves 1x8 (wave 16x32),   16x16 MFMA            128     4   -- decode (tuning)
//  11  BM=16  BN=128, 8 waves 1x8 (wave 16x16),   16x16 MFMA            128     6   -- decode
//  12  BM=32  BN=128, 8 waves 1x8 (wave 32x16),   16x16 MFMA            128     6   -- small M
//  13  BM=64  BN=128, 8 waves 2x4 (wave 32x32),   16x16 MFMA            128     4   -- small M
//  14  BM=256 BN=256, 16 waves 4x4 (wave 64x64),  32x32 MFMA            128     2   -- prefill (per-token)
//  15  BM=128 BN=128, 8 waves 2x4 (wave 64x32),   32x32 MFMA            128     3   -- mid M
//  16  BM=256 BN=256, 8 waves 2x4 (wave 128x64),  16x16 MFMA            128     2   -- prefill (scaled)
//  17  BM=128 BN=256, 8 waves 2x4 (wave 64x64),   32x32 MFMA            128     3   -- MoE, ~128 rows/expert
//  18  BM=192 BN=256, 8 waves 2x4 (wave 96x64),   32x32 MFMA            128     2   -- MoE, 129-192 rows/expert
//  19  BM=192 BN=256, 8 waves 2x4 (wave 96x64),   16x16 MFMA            128     2   -- MoE (block scales)
//  20  BM=128 BN=256, 8 waves 2x4 (wave 64x64),   16x16 MFMA            128     3   -- MoE (block scales)
//  21  BM=64  BN=224, 7 waves 1x7 (wave 64x32),   32x32 MFMA            128     4   -- small M, N = 7 * 2^k
//  22  BM=256 BN=96, 12 waves 4x3 (wave 64x32),   32x32 MFMA            128     3   -- mid M (per-token)
//  23  BM=16  BN=144, 9 waves 1x9 (wave 16x16),   16x16 MFMA            128     6   -- decode, N = 9 * 2^k
// The 8- and 16-wave kinds put two or four waves on each SIMD, which hides the
// per-step barrier -> LDS read -> MFMA -> fold latency of one wave.
// Block mode with deferred folds and the products in LDS (LDS_PROD in the
// kernel) adds, after the ring, each wave's TM scale products (WGN * BM floats
// in all).
template <int BM, int BN, int BK, int WGM, int WGN, int MF, int R, int SMODE>
constexpr int cfg_lds() {
  const int sa = SMODE >= 1 ? ((BM * 4 + 255) / 256) * 256 : 0;
  constexpr bool f4 = SMODE == 2 || SMODE == 4;
  const int sb = (SMODE == 1 || SMODE == 3) ? 256 : (f4 ? ((BN * 4 + 255) / 256) * 256 : 0);
  constexpr int fm = BM / WGM / MF, fn = BN / WGN / MF, nacc = MF == 32 ? 16 : 4;
  constexpr bool prod = SMODE == 1 && fm * fn * nacc <= 32 && fm * nacc >= 16;
  return R * (BM * BK + BN * (f4 ? BK / 2 : BK) + sa + sb) + (prod ? WGN * BM * 4 : 0);
}

template <int BM, int BN, int BK, int WGM, int WGN, int MF, int R, int SMODE, int ODT>
void launch_cfg(const GemmPlan& p, const GemmArgs& x, hipStream_t stream) {
  constexpr int lds = cfg_lds<BM, BN, BK, WGM, WGN, MF, R, SMODE>();
  static_assert(lds <= 160 * 1024 - 256, "tile configuration exceeds the 160 KiB LDS");
  dim3 grid(p.tiles_m * p.tiles_n, p.splits);
  if (p.splits > 1)
    hipLaunchKernelGGL((fp8_gemm_kernel<BM, BN, BK, WGM, WGN, MF, R, SMODE, 2, ODT>), grid, dim3(64 * WGM * WGN),
                       lds, stream, x);
  else
    hipLaunchKernelGGL((fp8_gemm_kernel<BM, BN, BK, WGM, WGN, MF, R, SMODE, 0, ODT>), grid, dim3(64 * WGM * WGN),
                       lds, stream, x);
}

template <int BM, int BN, int BK, int WGM, int WGN, int MF, int R, int SMODE>
void launch_grouped_cfg(const GemmArgs& x, int max_mtiles, hipStream_t stream) {
  constexpr int lds = cfg_lds<BM, BN, BK, WGM, WGN, MF, R, SMODE>();
  static_assert(lds <= 160 * 1024 - 256, "tile configuration exceeds the 160 KiB LDS");
  dim3 grid((unsigned)(max_mtiles * x.tiles_n), 1);
  hipLaunchKernelGGL((fp8_gemm_kernel<BM, BN, BK, WGM, WGN, MF, R, SMODE, 0, TI_DTYPE_BF16>), grid,
                     dim3(64 * WGM * WGN), lds, stream, x);
}

template <int SMODE, int ODT>
void launch_kind(const GemmPlan& p, const GemmArgs& x, hipStream_t stream) {
  if constexpr (SMODE == 2 || SMODE == 4) {
    // MXFP4 B: the 128-wide K step kinds (the e2m1 slab is half as large, so
    // 256x256 takes three stages).
    switch (p.kind) {
      case 2: launch_cfg<128, 128, 128, 2, 2, 32, 3, SMODE, ODT>(p, x, stream); break;
      case 3: launch_cfg<16, 256, 128, 1, 4, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 5: launch_cfg<64, 128, 128, 1, 4, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 6: launch_cfg<16, 128, 128, 1, 4, 16, 6, SMODE, ODT>(p, x, stream); break;
      case 9: launch_cfg<256, 128, 128, 4, 2, 32, 3, SMODE, ODT>(p, x, stream); break;
      case 10: launch_cfg<16, 256, 128, 1, 8, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 11: launch_cfg<16, 128, 128, 1, 8, 16, 6, SMODE, ODT>(p, x, stream); break;
      case 12: launch_cfg<32, 128, 128, 1, 8, 16, 6, SMODE, ODT>(p, x, stream); break;
      case 13: launch_cfg<64, 128, 128, 2, 4, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 15: launch_cfg<128, 128, 128, 2, 4, 32, 3, SMODE, ODT>(p, x, stream); break;
      case 16: launch_cfg<256, 256, 128, 2, 4, 16, 2, SMODE, ODT>(p, x, stream); break;
      case 17: launch_cfg<128, 256, 128, 2, 4, 32, 3, SMODE, ODT>(p, x, stream); break;
      case 18: launch_cfg<192, 256, 128, 2, 4, 32, 2, SMODE, ODT>(p, x, stream); break;
      case 19: launch_cfg<192, 256, 128, 2, 4, 16, 2, SMODE, ODT>(p, x, stream); break;
      case 20: launch_cfg<128, 256, 128, 2, 4, 16, 3, SMODE, ODT>(p, x, stream); break;
      case 23: launch_cfg<16, 144, 128, 1, 9, 16, 6, SMODE, ODT>(p, x, stream); break;
      default: launch_cfg<256, 256, 128, 2, 4, 32, 3, SMODE, ODT>(p, x, stream); break;
    }
  } else {
    switch (p.kind) {
      case 0: launch_cfg<256, 256, 64, 2, 4, 32, 4, SMODE, ODT>(p, x, stream); break;
      case 1: launch_cfg<256, 256, 128, 2, 4, 32, 2, SMODE, ODT>(p, x, stream); break;
      case 2: launch_cfg<128, 128, 128, 2, 2, 32, 3, SMODE, ODT>(p, x, stream); break;
      case 3: launch_cfg<16, 256, 128, 1, 4, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 4: launch_cfg<32, 256, 128, 1, 4, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 5: launch_cfg<64, 128, 128, 1, 4, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 6: launch_cfg<16, 128, 128, 1, 4, 16, 6, SMODE, ODT>(p, x, stream); break;
      case 7: launch_cfg<128, 128, 64, 2, 2, 32, 6, SMODE, ODT>(p, x, stream); break;
      case 8: launch_cfg<256, 128, 64, 2, 2, 32, 6, SMODE, ODT>(p, x, stream); break;
      case 10: launch_cfg<16, 256, 128, 1, 8, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 11: launch_cfg<16, 128, 128, 1, 8, 16, 6, SMODE, ODT>(p, x, stream); break;
      case 12: launch_cfg<32, 128, 128, 1, 8, 16, 6, SMODE, ODT>(p, x, stream); break;
      case 13: launch_cfg<64, 128, 128, 2, 4, 16, 4, SMODE, ODT>(p, x, stream); break;
      case 15: launch_cfg<128, 128, 128, 2, 4, 32, 3, SMODE, ODT>(p, x, stream); break;
      case 16: launch_cfg<256, 256, 128, 2, 4, 16, 2, SMODE, ODT>(p, x, stream); break;
      case 17: launch_cfg<128, 256, 128, 2, 4, 32, 3, SMODE, ODT>(p, x, stream); break;
      case 18: launch_cfg<192, 256, 128, 2, 4, 32, 2, SMODE, ODT>(p, x, stream); break;
      case 19: launch_cfg<192, 256, 128, 2, 4, 16, 2, SMODE, ODT>(p, x, stream); break;
      case 20: launch_cfg<128, 256, 128, 2, 4, 16, 3, SMODE, ODT>(p, x, stream); break;
      case 21: launch_cfg<64, 224, 128, 1, 7, 32, 4, SMODE, ODT>(p, x, stream); break;
      case 22:  // the plan maps it to kind 9 in block mode (its fold would spill at 12 waves)
        if constexpr (SMODE != 1) launch_cfg<256, 96, 128, 4, 3, 32, 3, SMODE, ODT>(p, x, stream);
        break;
      case 23: launch_cfg<16, 144, 128, 1, 9, 16, 6, SMODE, ODT>(p, x, stream); break;
      case 14:
        if constexpr (SMODE == 0 || SMODE == 3) launch_cfg<256, 256, 128, 4, 4, 32, 2, SMODE, ODT>(p, x, stream);
        break;
      default: launch_cfg<256, 128, 128, 4, 2, 32, 3, SMODE, ODT>(p, x, stream); break;
    }
  }
}

const int kBM[kNumKinds] = {256, 256, 128, 16, 32, 64, 16, 128, 256, 256, 16, 16, 32, 64, 256, 128, 256, 128, 192, 192, 128, 64, 256, 16};
const int kBN[kNumKinds] = {256, 256, 128, 256, 256, 128, 128, 128, 128, 128, 256, 128, 128, 128, 256, 128, 256, 256,
                            256, 256, 256, 224, 96, 144};

int env_int(const char* name, int dflt) {
  const char* e = getenv(name);
  return (e && *e) ? atoi(e) : dflt;
}

}  // namespace

GemmPlan make_gemm_plan(int M, int N, int K, int smode) {
  GemmPlan p;
  const int KT = K / 128;
  // Power-of-two block FP8 runs the per-token loop (the MFMA applies the
  // scales; no fold), so it takes the per-token plan; power-of-two MXFP4 the
  // MXFP4 plan.
  if (smode == 3) smode = 0;
  if (smode == 4) smode = 2;
  // Measured on MI355X at the Llama-3-70B / DeepSeek-V3 shapes (BASELINE
  // configs 2 and 3): skinny M streams B with 16- to 64-row tiles, split over
  // K when too few column tiles cover the 256 CUs; larger M takes the largest
  // tile that still gives every CU a workgroup (256x256, then 256x128 from 144
  // tiles -- 128 with block or MXFP4 scales -- then 128x128).
  auto tiles = [&](int bm, int bn) { return (long)cdiv(M, bm) * cdiv(N, bn); };
  // fraction of the last wave of 256 workgroups that is occupied, over all waves
  auto fill = [](long t) { return (double)t / (double)(cdiv((int)t, 256) * 256); };
  int splits = 1;
  if (M <= 4 && (smode != 0 || tiles(16, 256) >= 128)) {
    // 4-wave 16x256 tiles; split over K below 128 column tiles: up to 4 ways,
    // 8 at deep K.  (Per-token FP8 below 128 such tiles takes the 8-wave 16x128
    // split below instead: config-2 qkv M=1 17 -> 16 us, down M=1 46 -> 43 us.)
    p.kind = 3;
    const long t = tiles(16, 256);
    const int cap = K >= 16384 ? 8 : 4;
    splits = t >= 128 ? 1 : (int)(cdiv(256, (int)t) < cap ? cdiv(256, (int)t) : cap);
  } else if (M <= 16) {
    // 8-wave 16x128 tiles: two waves per SIMD hide each other's per-step
    // LDS/MFMA latency (12-24% faster than the 4-wave tile at M=16).
    // Below 128 column tiles split over K, four ways when that stays within
    // 256 workgroups, else two (config-2 qkv M=16: 23 -> 17 us).
    p.kind = 11;
    const long t = tiles(16, 128);
    if (t < 128) splits = t * 4 <= 256 ? 4 : 2;
    else if (t < 256 && 2 * tiles(16, 144) <= 256 && fill(2 * tiles(16, 144)) > fill(t) + 0.1) {
      // 9-wave 16x144 tiles split in two where N = 9 * 2^k (config-3 a,
      // N=18432: 256 workgroups instead of 144; block FP8 27 -> 23 us, MXFP4
      // 22.4 -> 15.7 us)
      p.kind = 23;
      splits = 2;
    } else if (smode == 2 && t < 256 && 2 * tiles(16, 256) <= 256) {
      // MXFP4 (64-byte e2m1 rows per K step): 8-wave 16x256 tiles split in two
      // stream more bytes per step for the same workgroup count (config-3-shape
      // c, N=24576: 22.8 -> 19.8 us)
      p.kind = 10;
      splits = 2;
    }
  } else if (smode == 0 && M <= 64 && fill(tiles(64, 224)) > fill(tiles(M <= 32 ? 32 : 64, 128)) + 0.05 &&
             tiles(64, 224) >= 192) {
    // 7-wave 64x224 tiles where N = 7 * 2^k gives a whole number of waves of
    // 256 workgroups and 128-column tiles do not (config-2 gate_up, N=57344:
    // 256 tiles instead of 448, M=64 94 -> 88 us, M=32 87 -> 83 us).
    p.kind = 21;
  } else if (M <= 32) {
    p.kind = 12;
    splits = tiles(32, 128) >= 128 ? 1 : 2;
  } else if (M <= 64) {
    // 64x128 8-wave tiles; below 128 column tiles, split over K two or four
    // ways, as many as keep the grid within 256 workgroups (config-2 qkv M=64:
    // 29 -> 24 us; block FP8 K=18432 N=7168: 90 -> 31 us).
    p.kind = 13;
    const long t = tiles(64, 128);
    if (t < 128) splits = t * 4 <= 256 ? 4 : 2;
  } else if (M <= 128) {
    // Per-token and block FP8: 4-wave 128x128 tiles from 256 of them, the
    // 8-wave 128x128 tile split in two from 72 (config-2 qkv M=128: 36 -> 31
    // us; config-3 a: 66 -> 55 us); else, and for MXFP4, 8-wave 64x128 split
    // over K when fewer than 160 tiles (4 ways for MXFP4 at deep K).
    if (smode != 2 && tiles(128, 128) >= 256) {
      p.kind = 2;
    } else if (smode != 2 && tiles(128, 128) >= 72) {
      p.kind = 15;
      splits = 2;
    } else {
      p.kind = 13;
      splits = tiles(64, 128) >= 160 ? 1 : ((smode == 2 && K >= 16384) ? 4 : 2);
    }
  } else if (tiles(256, 256) >= 256) {
    // Per-token FP8 runs the 256x256 tile on 16 waves (4 per SIMD, 64x64 wave
    // tiles: 4-10% faster).  The block / MXFP4 folds need more registers than
    // 16 waves leave; they keep 8 waves with 16x16x128 MFMAs, whose 4-register
    // partial sums leave room to fold one tile while the next one's MFMAs run
    // (2-4% over the 32x32x64 form).
    p.kind = smode == 0 ? 14 : 16;
  } else if (smode == 0 && tiles(256, 128) >= 144 && tiles(256, 96) <= 256 &&
             fill(tiles(256, 96)) > fill(tiles(256, 128)) + 0.1) {
    // 12-wave 256x96 tiles when they fill the 256 CUs better than 256x128
    // ones (config-2 qkv M=512, N=10240: 214 instead of 160 tiles, 74 -> 60 us)
    p.kind = 22;
  } else if (smode == 2 && M <= 256 && tiles(256, 128) >= 128) {
    // MXFP4 at M <= 256: 128x256 tiles (the same workgroup count as 256x128 at
    // M=256, half the e2m1 slab re-reads): config-3-shape a and c 3-6% faster
    p.kind = 17;
  } else if (tiles(256, 128) >= (smode >= 1 ? 128 : 144)) {
    p.kind = 9;
  } else if (smode == 0 && tiles(256, 128) >= 64) {
    // per-token FP8 between 64 and 144 256x128 tiles: split over K in two
    // (config-2 down M=512: 151 -> 140 us)
    p.kind = 9;
    splits = 2;
  } else {
    // 128x128 on 8 waves (64x32 wave tiles) -- 64x128 for MXFP4 when it gives
    // 192 tiles -- split over K up to 128 128x128 tiles.
    p.kind = (smode == 2 && tiles(64, 128) >= 192) ? 13 : 15;
    splits = tiles(128, 128) > 128 ? 1 : 2;
  }
  p.kind = env_int("TI_ROCM_FP8_KIND", p.kind);
  if (p.kind < 0 || p.kind >= kNumKinds) p.kind = 1;
  if (smode == 2 && (p.kind == 0 || p.kind == 4 || p.kind == 7 || p.kind == 8 || p.kind == 21 || p.kind == 22))
    p.kind = 1;  // not built for e2m1
  if (smode != 0 && p.kind == 14) p.kind = 1;  // per-token only (the scaled folds would spill)
  if (smode == 1 && p.kind == 22) p.kind = 9;
  p.group_m = env_int("TI_ROCM_FP8_GROUP_M", 4);
  if (p.group_m < 1) p.group_m = 1;
  p.tiles_m = cdiv(M, kBM[p.kind]);
  p.tiles_n = cdiv(N, kBN[p.kind]);
  splits = env_int("TI_ROCM_FP8_SPLITS", splits);
  splits = splits > KT / 4 ? KT / 4 : splits;  // at least 4 K blocks per split
  p.splits = splits < 1 ? 1 : splits;
  return p;
}

int grouped_bm(int kind) { return kBM[kind]; }
int grouped_bn(int kind) { return kBN[kind]; }

template <int SMODE>
void launch_grouped_smode(int kind, const GemmArgs& x, int max_mtiles, hipStream_t stream) {
  switch (kind) {
    case 2: launch_grouped_cfg<128, 128, 128, 2, 2, 32, 3, SMODE>(x, max_mtiles, stream); break;
    case 5: launch_grouped_cfg<64, 128, 128, 1, 4, 16, 4, SMODE>(x, max_mtiles, stream); break;
    case 9: launch_grouped_cfg<256, 128, 128, 4, 2, 32, 3, SMODE>(x, max_mtiles, stream); break;
    case 16: launch_grouped_cfg<256, 256, 128, 2, 4, 16, 2, SMODE>(x, max_mtiles, stream); break;
    case 11: launch_grouped_cfg<16, 128, 128, 1, 8, 16, 6, SMODE>(x, max_mtiles, stream); break;
    case 3: launch_grouped_cfg<16, 256, 128, 1, 4, 16, 4, SMODE>(x, max_mtiles, stream); break;
    case 4: launch_grouped_cfg<32, 256, 128, 1, 4, 16, 4, SMODE>(x, max_mtiles, stream); break;
    case 10: launch_grouped_cfg<16, 256, 128, 1, 8, 16, 4, SMODE>(x, max_mtiles, stream); break;
    case 12: launch_grouped_cfg<32, 128, 128, 1, 8, 16, 6, SMODE>(x, max_mtiles, stream); break;
    case 13: launch_grouped_cfg<64, 128, 128, 2, 4, 16, 4, SMODE>(x, max_mtiles, stream); break;
    case 15: launch_grouped_cfg<128, 128, 128, 2, 4, 32, 3, SMODE>(x, max_mtiles, stream); break;
    case 17: launch_grouped_cfg<128, 256, 128, 2, 4, 32, 3, SMODE>(x, max_mtiles, stream); break;
    case 18: launch_grouped_cfg<192, 256, 128, 2, 4, 32, 2, SMODE>(x, max_mtiles, stream); break;
    case 19: launch_grouped_cfg<192, 256, 128, 2, 4, 16, 2, SMODE>(x, max_mtiles, stream); break;
    case 20: launch_grouped_cfg<128, 256, 128, 2, 4, 16, 3, SMODE>(x, max_mtiles, stream); break;
    case 14:
      if constexpr (SMODE == 3) launch_grouped_cfg<256, 256, 128, 4, 4, 32, 2, SMODE>(x, max_mtiles, stream);
      break;
    default: launch_grouped_cfg<16, 128, 128, 1, 4, 16, 6, SMODE>(x, max_mtiles, stream); break;
  }
}

void launch_gemm_grouped(int kind, int smode, const GemmArgs& x, int max_mtiles, hipStream_t stream) {
  if (smode == 2) launch_grouped_smode<2>(kind, x, max_mtiles, stream);
  else if (smode == 3) launch_grouped_smode<3>(kind, x, max_mtiles, stream);
  else if (smode == 4) launch_grouped_smode<4>(kind, x, max_mtiles, stream);
  else launch_grouped_smode<1>(kind, x, max_mtiles, stream);
}

// Split-K partials: every split's accumulators of every (whole) tile.
static size_t gemm_partial_bytes(const GemmPlan& p) {
  return p.splits > 1 ? (size_t)p.splits * p.tiles_m * p.tiles_n * kBM[p.kind] * kBN[p.kind] * sizeof(float) : 0;
}

size_t gemm_workspace_bytes(const GemmPlan& p, int M, int N) {
  if (p.splits <= 1) return 0;
  (void)M;
  (void)N;
  const size_t part = gemm_partial_bytes(p);
  const size_t tick = ((size_t)p.tiles_m * p.tiles_n * sizeof(int) + 255) & ~(size_t)255;
  return part + tick + 256;
}

size_t gemm_ticket_bytes(const GemmPlan& p) {
  return ((size_t)p.tiles_m * p.tiles_n * sizeof(int) + 255) & ~(size_t)255;
}

void launch_gemm(const GemmPlan& p, int smode, int odt, const GemmArgs& x, hipStream_t stream) {
  if (smode == 0) {
    if (odt == TI_DTYPE_F16) launch_kind<0, TI_DTYPE_F16>(p, x, stream);
    else launch_kind<0, TI_DTYPE_BF16>(p, x, stream);
  } else if (smode == 2) {
    if (odt == TI_DTYPE_F16) launch_kind<2, TI_DTYPE_F16>(p, x, stream);
    else launch_kind<2, TI_DTYPE_BF16>(p, x, stream);
  } else if (smode == 3) {
    if (odt == TI_DTYPE_F16) launch_kind<3, TI_DTYPE_F16>(p, x, stream);
    else launch_kind<3, TI_DTYPE_BF16>(p, x, stream);
  } else if (smode == 4) {
    if (odt == TI_DTYPE_F16) launch_kind<4, TI_DTYPE_F16>(p, x, stream);
    else launch_kind<4, TI_DTYPE_BF16>(p, x, stream);
  } else {
    if (odt == TI_DTYPE_F16) launch_kind<1, TI_DTYPE_F16>(p, x, stream);
    else launch_kind<1, TI_DTYPE_BF16>(p, x, stream);
  }
}

}  // namespace fp8
}  // namespace ti

using namespace ti;
using namespace ti::fp8;

static int gemm_common(const char* name, int smode, const uint8_t* a, const float* a_scale,
                       int a_scale_stride, const uint8_t* b, const float* b_scale, int b_scale_stride,
                       void* out, int out_dtype, int M, int N, int K, void* workspace,
                       size_t workspace_bytes, hipStream_t stream, int a_scale_layout = 0,
                       int b_tiled = 0) {
  TI_CHECK_ARG(a && b && a_scale && b_scale && out, "%s: null pointer", name);
  TI_CHECK_ARG(out_dtype == TI_DTYPE_BF16 || out_dtype == TI_DTYPE_F16, "%s: out dtype must be bf16 or fp16",
               name);
  TI_CHECK_SHAPE(M >= 0 && N > 0 && K > 0 && K % 128 == 0, "%s: need K %% 128 == 0 (M=%d N=%d K=%d)", name,
                 M, N, K);
  TI_CHECK_ARG(((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0, "%s: a and b must be 16-byte aligned",
               name);
  TI_CHECK_ARG(((uintptr_t)out & 1) == 0 && ((uintptr_t)a_scale & 3) == 0 && ((uintptr_t)b_scale & 3) == 0,
               "%s: misaligned out or scales", name);
  if (M == 0) return TI_OK;
  GemmPlan p = make_gemm_plan(M, N, K, smode);
  if (b_tiled && (p.kind == 0 || p.kind == 7 || p.kind == 8)) p.kind = 1;  // tiles are 128-K steps
  GemmArgs x{};
  x.a = a; x.b = b; x.sa = a_scale; x.sb = b_scale;
  x.sa_stride = a_scale_stride; x.sb_stride = b_scale_stride;
  x.sb_layout = (smode == 2 || smode == 4) ? b_scale_stride : 0;
  x.b_tiled = b_tiled;
  x.sa_layout = smode >= 1 ? a_scale_layout : 0;
  x.out = (uint16_t*)out;
  x.M = M; x.N = N; x.K = K;
  x.splits = p.splits; x.tiles_m = p.tiles_m; x.tiles_n = p.tiles_n; x.group_m = p.group_m;
  const size_t need = gemm_workspace_bytes(p, M, N);
  if (need) {
    if (!workspace || workspace_bytes < need) {
      set_error("%s: workspace of %zu bytes required (got %zu)", name, need, workspace_bytes);
      return TI_ERR_WORKSPACE;
    }
    TI_CHECK_ARG(((uintptr_t)workspace & 15) == 0, "%s: workspace must be 16-byte aligned", name);
    x.partial = (float*)workspace;
    const uintptr_t end = ((uintptr_t)workspace + workspace_bytes) & ~(uintptr_t)255;
    x.tickets = (int*)(end - gemm_ticket_bytes(p));
  }
  launch_gemm(p, smode, out_dtype, x, stream);
  TI_CHECK_LAUNCH(name);
  return TI_OK;
}

extern "C" size_t ti_fp8_gemm_workspace_bytes(int M, int N, int K, int scale_mode) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128) return 0;
  return gemm_workspace_bytes(make_gemm_plan(M, N, K, scale_mode), M, N);
}

extern "C" size_t ti_fp8_gemm_workspace_bytes_max(int max_m, int N, int K, int scale_mode) {
  if (max_m <= 0 || N <= 0 || K <= 0 || K % 128) return 0;
  size_t pmax = 0, tmax = 0;
  for (int m = 1; m <= max_m; ++m) {
    GemmPlan p = make_gemm_plan(m, N, K, scale_mode);
    if (p.splits <= 1) continue;
    const size_t part = gemm_partial_bytes(p);
    pmax = part > pmax ? part : pmax;
    tmax = gemm_ticket_bytes(p) > tmax ? gemm_ticket_bytes(p) : tmax;
  }
  return pmax ? pmax + tmax + 256 : 0;
}

extern "C" int ti_fp8_gemm_rowcol(const uint8_t* a, const float* a_scale, int a_scale_per_row,
                                  const uint8_t* b, const float* b_scale, int b_scale_per_col, void* out,
                                  int out_dtype, int M, int N, int K, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  return gemm_common("ti_fp8_gemm_rowcol", 0, a, a_scale, a_scale_per_row ? 1 : 0, b, b_scale,
                     b_scale_per_col ? 1 : 0, out, out_dtype, M, N, K, workspace, workspace_bytes, stream);
}

extern "C" int ti_fp8_gemm_rowcol_tiled(const uint8_t* a, const float* a_scale, int a_scale_per_row,
                                        const uint8_t* b_tiled, const float* b_scale, int b_scale_per_col,
                                        void* out, int out_dtype, int M, int N, int K, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream) {
  TI_CHECK_SHAPE(N % 128 == 0, "ti_fp8_gemm_rowcol_tiled: need N %% 128 == 0 (N=%d)", N);
  return gemm_common("ti_fp8_gemm_rowcol_tiled", 0, a, a_scale, a_scale_per_row ? 1 : 0, b_tiled, b_scale,
                     b_scale_per_col ? 1 : 0, out, out_dtype, M, N, K, workspace, workspace_bytes, stream, 0, 1);
}

namespace ti {
namespace fp8 {
namespace {

// w [N, K] -> [N/128][K/128][128][128]: thread per 16-byte chunk of a row.
__global__ __launch_bounds__(256) void tile_weight_kernel(const uint4* __restrict__ w, uint4* __restrict__ out,
                                                          int N, int K) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;  // chunk index in [N, K/16]
  const int cpr = K / 16;
  if (i >= (long)N * cpr) return;
  const int n = (int)(i / cpr), c = (int)(i % cpr);
  const long dst = (((long)(n >> 7) * (K / 128) + (c >> 3)) * 128 + (n & 127)) * 8 + (c & 7);
  out[dst] = w[i];
}

}  // namespace
}  // namespace fp8
}  // namespace ti

extern "C" int ti_fp8_tile_weight(const uint8_t* w, int N, int K, uint8_t* w_tiled, hipStream_t stream) {
  TI_CHECK_ARG(w && w_tiled, "ti_fp8_tile_weight: null pointer");
  TI_CHECK_SHAPE(N > 0 && K > 0 && N % 128 == 0 && K % 128 == 0,
                 "ti_fp8_tile_weight: need N %% 128 == 0 and K %% 128 == 0 (N=%d K=%d)", N, K);
  TI_CHECK_ARG(((uintptr_t)w & 15) == 0 && ((uintptr_t)w_tiled & 15) == 0,
               "ti_fp8_tile_weight: w and w_tiled must be 16-byte aligned");
  const long chunks = (long)N * (K / 16);
  hipLaunchKernelGGL(ti::fp8::tile_weight_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream,
                     (const uint4*)w, (uint4*)w_tiled, N, K);
  TI_CHECK_LAUNCH("ti_fp8_tile_weight");
  return TI_OK;
}

extern "C" int ti_fp8_gemm_block(const uint8_t* a, const float* a_scale, int a_scale_layout, const uint8_t* b,
                                 const float* b_scale, void* out, int out_dtype, int M, int N, int K,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  TI_CHECK_ARG(a_scale_layout == 0 || a_scale_layout == 1, "ti_fp8_gemm_block: a_scale_layout must be 0 or 1");
  return gemm_common("ti_fp8_gemm_block", 1, a, a_scale, 0, b, b_scale, 0, out, out_dtype, M, N, K, workspace,
                     workspace_bytes, stream, a_scale_layout);
}

extern "C" int ti_fp8_gemm_block_pow2(const uint8_t* a, const float* a_scale, int a_scale_layout,
                                      const uint8_t* b, const float* b_scale, void* out, int out_dtype, int M,
                                      int N, int K, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  TI_CHECK_ARG(a_scale_layout == 0 || a_scale_layout == 1,
               "ti_fp8_gemm_block_pow2: a_scale_layout must be 0 or 1");
  return gemm_common("ti_fp8_gemm_block_pow2", 3, a, a_scale, 0, b, b_scale, 0, out, out_dtype, M, N, K,
                     workspace, workspace_bytes, stream, a_scale_layout);
}

extern "C" int ti_fp4_gemm_pow2(const uint8_t* a, const float* a_scale, int a_scale_layout, const uint8_t* b,
                                const uint8_t* b_scale, int b_scale_layout, void* out, int out_dtype, int M, int N,
                                int K, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  TI_CHECK_ARG(a_scale_layout == 0 || a_scale_layout == 1, "ti_fp4_gemm_pow2: a_scale_layout must be 0 or 1");
  TI_CHECK_ARG(b_scale_layout == 0 || b_scale_layout == 1, "ti_fp4_gemm_pow2: b_scale_layout must be 0 or 1");
  return gemm_common("ti_fp4_gemm_pow2", 4, a, a_scale, 0, b, (const float*)b_scale, b_scale_layout, out,
                     out_dtype, M, N, K, workspace, workspace_bytes, stream, a_scale_layout);
}

extern "C" int ti_fp4_gemm(const uint8_t* a, const float* a_scale, int a_scale_layout, const uint8_t* b,
                           const uint8_t* b_scale, int b_scale_layout, void* out, int out_dtype, int M, int N, int K,
                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
  TI_CHECK_ARG(a_scale_layout == 0 || a_scale_layout == 1, "ti_fp4_gemm: a_scale_layout must be 0 or 1");
  TI_CHECK_ARG(b_scale_layout == 0 || b_scale_layout == 1, "ti_fp4_gemm: b_scale_layout must be 0 or 1");
  return gemm_common("ti_fp4_gemm", 2, a, a_scale, 0, b, (const float*)b_scale, b_scale_layout, out, out_dtype, M,
                     N, K, workspace, workspace_bytes, stream, a_scale_layout);
}

namespace {
// [N, K/32] e8m0 -> step-major [K/128][N][4]: one thread per (step, row) dword.
__global__ __launch_bounds__(256) void scale_stepmajor_kernel(const uint32_t* __restrict__ src, int N, int KS,
                                                              uint32_t* __restrict__ dst) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)N * KS) return;
  const int kk = (int)(i / N), n = (int)(i % N);
  dst[i] = src[(long)n * KS + kk];
}
}  // namespace

extern "C" int ti_fp4_scale_stepmajor(const uint8_t* src, int N, int K, uint8_t* dst, hipStream_t stream) {
  TI_CHECK_ARG(src && dst, "ti_fp4_scale_stepmajor: null pointer");
  TI_CHECK_SHAPE(N > 0 && K > 0 && K % 128 == 0, "ti_fp4_scale_stepmajor: need K %% 128 == 0 (N=%d K=%d)", N, K);
  TI_CHECK_ARG(((uintptr_t)src & 3) == 0 && ((uintptr_t)dst & 3) == 0, "ti_fp4_scale_stepmajor: misaligned");
  const long n = (long)N * (K / 128);
  hipLaunchKernelGGL(scale_stepmajor_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     (const uint32_t*)src, N, K / 128, (uint32_t*)dst);
  TI_CHECK_LAUNCH("ti_fp4_scale_stepmajor");
  return TI_OK;
}
