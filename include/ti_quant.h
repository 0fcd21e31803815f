/*
 * ti_quant.h -- C ABI of libti_quant.so, the gfx950 (MI355X) quantized-linear
 * kernels of torchinferno_amd.
 *
 * Conventions for every entry point:
 *   - pointers are device pointers, row-major and contiguous unless stated;
 *   - work is enqueued on `stream` (NULL = the null stream); nothing is
 *     allocated and nothing synchronises with the host, so calls may be
 *     captured into a HIP graph;
 *   - the return value is a ti_status; on failure ti_last_error() holds a
 *     message for the calling thread and no kernel has been launched.
 *
 * Each declaration names the reference interface it replaces (paths relative
 * to the TorchInferno source tree).
 */
#ifndef TI_QUANT_H_
#define TI_QUANT_H_

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum ti_status {
  TI_OK = 0,
  TI_ERR_INVALID = 1,      /* bad pointer, dtype or argument */
  TI_ERR_UNSUPPORTED = 2,  /* shape outside the kernel's supported region */
  TI_ERR_WORKSPACE = 3,    /* workspace missing or too small */
  TI_ERR_HIP = 4           /* a HIP runtime call failed */
} ti_status;

typedef enum ti_dtype {
  TI_DTYPE_F16 = 1,
  TI_DTYPE_BF16 = 2,
  TI_DTYPE_F32 = 3,
  TI_DTYPE_E4M3 = 4 /* OCP float8 e4m3fn, torch.float8_e4m3fn */
} ti_dtype;

/* Library version (major*10000 + minor*100 + patch). */
int ti_version(void);

/* Message describing the last failed call on this thread ("" if none). */
const char* ti_last_error(void);

/* ---------------------------------------------------------------------------
 * int4 W4A16, group-wise symmetric ("uint4b8": code q in [0,15], value
 * (q - 8) * scale), one scale per (group of G rows of K, output column).
 *
 * Canonical boundary layout: qweight int32 [K/8, N], nibble i (bits 4i..4i+3)
 * of word [r, n] = code of k = 8r + i; scales [K/G, N] in the activation
 * dtype.  ti_int4_repack converts it once to the kernel layout (replaces the
 * Marlin permutation + packing in src/torchinferno/kernels/marlin.py:57-131).
 * ------------------------------------------------------------------------- */

/* Bytes of the kernel-layout weight / scale buffers for a [K, N] weight. */
size_t ti_int4_packed_weight_bytes(int K, int N);
size_t ti_int4_packed_scale_bytes(int K, int N, int group_size);

/* Canonical -> kernel layout.  Requires K % group_size == 0, group_size == 128,
 * N % 16 == 0.  scale_dtype is TI_DTYPE_F16 or TI_DTYPE_BF16. */
int ti_int4_repack(const int32_t* qweight, const void* scales, int scale_dtype,
                   int K, int N, int group_size,
                   int32_t* packed_weight, void* packed_scales, hipStream_t stream);

/* Symmetric round-to-nearest int4 quantization of a [K, N] fp16/bf16 weight
 * (K-major: the reference passes weight.t()) into the canonical layout:
 * per (128-row group, column) w is rounded to fp16, s = max(|max/7|, |min/-8|)
 * clamped >= 1e-8 (fp32), q = clamp(rint(w/s), -8, 7) + 8, scales stored in
 * scale_dtype.  Replaces the quantizer of quantize_to_marlin_int4
 * (src/torchinferno/kernels/marlin.py:117-128); bit-identical to the same
 * formula evaluated with IEEE fp32 division on the host. */
int ti_int4_quantize_rtn(const void* weight_kn, int weight_dtype, int K, int N, int group_size,
                         int scale_dtype, int32_t* qweight, void* scales, hipStream_t stream);

/* Dequantize a kernel-layout weight to fp32 [K, N]: out = (q - 8) * s, exact.
 * Shares the in-register unpack of ti_w4a16_gemm (bit-exactness check). */
int ti_int4_dequant(const int32_t* packed_weight, const void* packed_scales, int scale_dtype,
                    int K, int N, int group_size, float* out, hipStream_t stream);

/* Workspace bytes ti_w4a16_gemm needs for this problem (0 if none), and for
 * every M in [1, max_m] with one shared buffer.  The workspace must be
 * zero-filled once when allocated; every call leaves its ticket words zero
 * again.  Calls sharing one workspace must be stream-ordered. */
size_t ti_w4a16_workspace_bytes(int M, int N, int K, int group_size);
size_t ti_w4a16_workspace_bytes_max(int max_m, int N, int K, int group_size);

/* Name and parameters of the kernel plan ti_w4a16_gemm would launch for this
 * problem, written to buf (introspection and tuning; no counterpart in the
 * reference).  Returns TI_ERR_UNSUPPORTED if no valid plan exists. */
int ti_w4a16_plan_name(int M, int N, int K, int group_size, char* buf, size_t len);

/* out[M, N] = a[M, K] @ dequant(W), fp32 accumulation, out in a's dtype.
 * Replaces torch.ops._C.marlin_gemm as called by marlin_int4_mm
 * (src/torchinferno/kernels/marlin.py:142-171).  dtype: TI_DTYPE_F16 or
 * TI_DTYPE_BF16 (activations, scales and output share it, as Marlin requires,
 * marlin.py:113-115).  Requires K % 128 == 0, N % 64 == 0, M >= 1. */
int ti_w4a16_gemm(const void* a, int dtype, const int32_t* packed_weight,
                  const void* packed_scales, void* out, int M, int N, int K, int group_size,
                  void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Asymmetric zero points (GPTQ / AWQ checkpoints; the reference has only the
 * symmetric lazy RTN of src/torchinferno/kernels/marlin.py:108-131 that they
 * replace): with W = (q - z) * s, after ti_w4a16_gemm computed the symmetric
 * part (q - 8) * s into out, adds sum_g rowsum_g(a[m]) * zero_offset[g, n] where
 * zero_offset = (8 - z) * s (fp32 [K/128, N]), in fp32, and rounds to dtype.
 * a [M, K] and out [M, N] in dtype; N % 4 == 0, K % 128 == 0. */
int ti_w4a16_zero_point_add(const void* a, int dtype, const float* zero_offset, void* out,
                            int M, int N, int K, hipStream_t stream);

/* Allocation-free ti_w4a16_gemm (no counterpart in the reference): for callers
 * that cannot allocate device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Same arguments and results
 * as ti_w4a16_gemm without the workspace: split-K partials and tickets live in
 * a static per-GPU device buffer of ti_w4a16_noalloc_scratch_bytes() (16 MiB),
 * set up on the first call on each device.  Problems needing more split-K
 * scratch than that return TI_ERR_WORKSPACE.  All calls on one GPU share the
 * buffer: calls that overlap on one GPU (unordered streams or threads) race. */
int ti_w4a16_gemm_noalloc(const void* a, int dtype, const int32_t* packed_weight,
                          const void* packed_scales, void* out, int M, int N, int K,
                          int group_size, hipStream_t stream);
size_t ti_w4a16_noalloc_scratch_bytes(void);

/* ---------------------------------------------------------------------------
 * FP8 e4m3 (OCP float8_e4m3fn) quantizers.  fp32 arithmetic with IEEE
 * division, round-to-nearest-even cast: codes and scales are bit-identical to
 * the reference formulas evaluated by torch.
 * ------------------------------------------------------------------------- */

/* Per-row dynamic quant: xs[m] = max(amax_k |x[m,k]| / 448, eps),
 * xq[m,k] = e4m3(x[m,k] / xs[m]).  Replaces the per-token activation quant
 * (Triton _row_scale_cast_fp8 / sgl_per_token_quant_fp8,
 * src/torchinferno/kernels/fp8.py:53-72,99-116,234-238; eps 1e-10).
 * x fp16/bf16 [M,K] 16-byte aligned, K % 8 == 0; xq [M,K] 8-byte aligned; xs [M]. */
int ti_fp8_quant_per_token(const void* x, int x_dtype, int M, int K, float eps,
                           uint8_t* xq, float* xs, hipStream_t stream);

/* Per-output-channel weight quant: ws[n] = max(amax_k |w[n,k]| * fl32(1/448), 1e-10),
 * wq[n,k] = e4m3(w[n,k] / ws[n]).  Replaces quantize_weight_fp8_per_channel
 * (src/torchinferno/kernels/fp8.py:129-138), whose ``amax.float() / 448.0`` torch
 * evaluates on the GPU as a multiply by the fp32 reciprocal.  w fp16/bf16 [N,K]
 * 16-byte aligned, K % 8 == 0; wq [N,K] 8-byte aligned; ws [N]. */
int ti_fp8_quant_weight_per_channel(const void* w, int w_dtype, int N, int K, uint8_t* wq,
                                    float* ws, hipStream_t stream);

/* Self-check of the e4m3 encoders (no reference counterpart: test support).
 * Runs every fp32 bit pattern through the software round-to-nearest-even
 * encoder and the gfx950 conversion instruction and adds to counts[0] the
 * disagreements on finite |x| < 480, to counts[1] those elsewhere.  counts:
 * two zeroed device uint64. */
int ti_fp8_e4m3_selfcheck(unsigned long long* counts, hipStream_t stream);

/* Self-check of the fp32 -> bf16 roundings (no reference counterpart: test
 * support): every fp32 bit pattern through the integer round-to-nearest-even
 * and the gfx950 conversion instruction the kernels use; adds to counts[0] the
 * disagreements on
 * non-NaN inputs, to counts[1] those on NaN inputs.  counts: two zeroed device
 * uint64. */
int ti_bf16_round_selfcheck(unsigned long long* counts, hipStream_t stream);

/* 1 x block_size activation quant (block_size == 128): per (row, block)
 * s = max(amax, 1e-4) * (1/448) -- or 2^ceil(log2(that)) if round_scale --
 * xq = e4m3(clamp(x / s, -448, 448)).  Replaces act_quant
 * (src/torchinferno/kernels/deepseek_v4_tilelang.py:147-173, kernel
 * deepseek_v4_tilelang_definitions.py:273-331).  xs [M, K/128] for
 * scale_layout 0 (the reference's), [K/128, M] ("step-major") for 1, the
 * layout the block and FP4 GEMMs read fastest. */
int ti_fp8_quant_block(const void* x, int x_dtype, int M, int K, int block_size,
                       int round_scale, uint8_t* xq, float* xs, int scale_layout, hipStream_t stream);

/* Tensor-scale cast xq = e4m3(x * inv_scale[0]) over n elements (n % 8 == 0).
 * Replaces the Triton _scale_cast_fp8 of quantize_activation_fp8
 * (src/torchinferno/kernels/fp8.py:43-51,141-181). */
int ti_fp8_quant_tensor(const void* x, int x_dtype, long n, const float* inv_scale,
                        uint8_t* xq, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Fused activation -> per-token e4m3 producers (the step before the W8A8 GEMM).
 * Rows of n elements (n % 8 == 0); outputs xq [rows, n] e4m3 and xs [rows]
 * fp32 with xs = max(amax/448, 1e-10) over the activation-dtype-rounded row.
 * The reduction and transcendental roundings are fixed (fp64 sum of squares
 * rounded once, rsqrt = 1/sqrtf, exp in fp64 rounded to fp32) so the output is
 * reproducible bit for bit.
 * ------------------------------------------------------------------------- */

/* (add +) RMSNorm -> FP8: h = x (+ residual); normed = h * rsqrt(mean(h^2) + eps)
 * * weight, rounded to dtype, then per-token quant.  With residual != NULL,
 * hidden_out receives h in dtype.  Replaces triton_rms_norm_fp8_per_token /
 * triton_add_rms_norm_fp8_per_token (src/torchinferno/kernels/triton_ops.py:
 * 2127-2182, 2226-2297). */
int ti_fp8_rmsnorm_quant_per_token(const void* x, const void* residual, const void* weight, int dtype,
                                   int rows, int n, float eps, void* hidden_out, uint8_t* xq, float* xs,
                                   hipStream_t stream);

/* SwiGLU -> FP8: act = g / (1 + exp(-g)) * u rounded to dtype, then per-token
 * quant; gate / up rows are row_stride elements apart (split views allowed).
 * Replaces triton_swiglu_fp8_per_token (triton_ops.py:2185-2223, 2300-2333). */
int ti_fp8_swiglu_quant_per_token(const void* gate, long gate_row_stride, const void* up,
                                  long up_row_stride, int dtype, int rows, int n, uint8_t* xq, float* xs,
                                  hipStream_t stream);

/* ---------------------------------------------------------------------------
 * FP8 W8A8 GEMMs: out[M,N] = a[M,K] . b[N,K]^T (both e4m3, K-contiguous, the
 * "b = weight.t(), column-major" layout of torch._scaled_mm), fp32
 * accumulation, out bf16 or fp16.  Requires K % 128 == 0; M, N arbitrary.
 * Skinny M may split K across workgroups: pass a workspace of
 * ti_fp8_gemm_workspace_bytes() (zero-filled once when allocated; every call
 * leaves its ticket words zero again; calls sharing one workspace must be
 * stream-ordered).  scale_mode: 0 = row/column scales, 1 = 128x128 blocks,
 * 2 = MXFP4 weights (ti_fp4_gemm), 3 = power-of-two 128x128 blocks
 * (ti_fp8_gemm_block_pow2), 4 = MXFP4 with power-of-two activation scales
 * (ti_fp4_gemm_pow2).
 * ------------------------------------------------------------------------- */
size_t ti_fp8_gemm_workspace_bytes(int M, int N, int K, int scale_mode);
size_t ti_fp8_gemm_workspace_bytes_max(int max_m, int N, int K, int scale_mode);

/* out = (a . b^T) * a_scale[m] * b_scale[n]; a_scale_per_row / b_scale_per_col
 * = 0 broadcast a single scale (tensorwise).  Replaces torch._scaled_mm /
 * aten::_scaled_mm.out as called by fp8_prefill_linear and
 * fp8_per_token_linear_quantized (src/torchinferno/kernels/fp8.py:184-327),
 * sgl fp8_scaled_mm, and torchinferno_sgl_fp8::scaled_mm_out
 * (src/torchinferno/kernels/csrc/sgl_fp8_out.cpp:17-83, no M <= 64 limit). */
int ti_fp8_gemm_rowcol(const uint8_t* a, const float* a_scale, int a_scale_per_row,
                       const uint8_t* b, const float* b_scale, int b_scale_per_col,
                       void* out, int out_dtype, int M, int N, int K,
                       void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ti_fp8_gemm_rowcol with the weight in the tiled layout ti_fp8_tile_weight
 * writes (N % 128 == 0).  No reference counterpart: the reference hands
 * torch._scaled_mm the [N, K] weight; this build keeps its load-time FP8
 * weight caches (the hooks' per-layer weight caches, tensor_parallel.py:
 * 2958-2983) tiled, so that each 128-K step of a 128-row block is one
 * contiguous 16 KiB run of HBM instead of 128 runs 128 bytes long. */
int ti_fp8_gemm_rowcol_tiled(const uint8_t* a, const float* a_scale, int a_scale_per_row,
                             const uint8_t* b_tiled, const float* b_scale, int b_scale_per_col,
                             void* out, int out_dtype, int M, int N, int K,
                             void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Re-lays an e4m3 weight w [N, K] (N, K % 128 == 0) as
 * w_tiled[N/128][K/128][128][128]: block (n/128, k/128), row n % 128, byte
 * k % 128.  N * K bytes; the weight format of ti_fp8_gemm_rowcol_tiled. */
int ti_fp8_tile_weight(const uint8_t* w, int N, int K, uint8_t* w_tiled, hipStream_t stream);

/* Block-scaled: out[m,n] = sum_kb (a . b^T over K block kb) * a_scale[m,kb] *
 * b_scale[n/128, kb]; b_scale [ceil(N/128), K/128] fp32; a_scale fp32
 * [M, K/128] for a_scale_layout 0 (the reference's), step-major [K/128, M]
 * for 1 (one contiguous read per tile and K step; ti_fp8_quant_block writes it).
 * Replaces fp8_gemm (src/torchinferno/kernels/deepseek_v4_tilelang.py:207-223,
 * kernel deepseek_v4_tilelang_definitions.py:436-485). */
int ti_fp8_gemm_block(const uint8_t* a, const float* a_scale, int a_scale_layout, const uint8_t* b,
                      const float* b_scale, void* out, int out_dtype, int M, int N, int K,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* FP8 activations x MXFP4 weights: out[m,n] = sum_k a[m,k] * a_scale[m, k/128]
 * * w[n,k] * 2^(e[n, k/32] - 127).  a e4m3 [M,K] with fp32 1x128 scales
 * ([M, K/128] for a_scale_layout 0, step-major [K/128, M] for 1); b e2m1 [N, K/2] (two values per byte along K, element 2i in the
 * low nibble -- torch float4_e2m1fn_x2); b_scale E8M0 bytes, layout 0 = the
 * checkpoint's [N, K/32], layout 1 = step-major [K/128][N][4] (the 4 scales
 * of a 128-wide K step of each row adjacent to the next row's, so a tile's
 * scales are one contiguous read; build it once with ti_fp4_scale_stepmajor).
 * The e8m0 scales are applied inside the MFMA (gfx950 block-scaled f8f6f4).
 * Replaces fp4_gemm (src/torchinferno/kernels/deepseek_v4_tilelang.py,
 * kernel deepseek_v4_tilelang_definitions.py:674-769).  K % 128 == 0. */
int ti_fp4_gemm(const uint8_t* a, const float* a_scale, int a_scale_layout, const uint8_t* b,
                const uint8_t* b_scale, int b_scale_layout, void* out, int out_dtype, int M, int N, int K, void* workspace,
                size_t workspace_bytes, hipStream_t stream);

/* ti_fp8_gemm_block and ti_fp4_gemm for DeepSeek-V4's "ue8m0" scale format:
 * every a_scale (and, for the block GEMM, every b_scale) value is a power of
 * two in the E8M0 range, 2^-127 .. 2^127, stored as fp32 -- the scales
 * act_quant writes with a scale_fmt and the float8_e8m0fnu weight scales of
 * the reference's scale_dtype=float8_e8m0fnu path (deepseek_v4_tilelang.py:
 * 207-223, tensor_parallel.py:1211-1212).  The MFMA applies the scales as
 * exponents (gfx950 block-scaled f8f6f4), so the per-128-K fold of the fp32
 * paths disappears; the result is the same sum, differing only in fp32
 * accumulation order.  Only the exponent field of each scale is read: other
 * values are not rejected but give wrong results.  Same arguments, layouts
 * and workspace (scale_mode 3 and 4) as the fp32-scale entry points. */
int ti_fp8_gemm_block_pow2(const uint8_t* a, const float* a_scale, int a_scale_layout, const uint8_t* b,
                           const float* b_scale, void* out, int out_dtype, int M, int N, int K,
                           void* workspace, size_t workspace_bytes, hipStream_t stream);
int ti_fp4_gemm_pow2(const uint8_t* a, const float* a_scale, int a_scale_layout, const uint8_t* b,
                     const uint8_t* b_scale, int b_scale_layout, void* out, int out_dtype, int M, int N, int K,
                     void* workspace, size_t workspace_bytes, hipStream_t stream);

/* E8M0 scales [N, K/32] -> step-major [K/128][N][4] (weight preparation, run
 * once per weight; no counterpart in the reference, whose kernels read the
 * checkpoint layout). */
int ti_fp4_scale_stepmajor(const uint8_t* src, int N, int K, uint8_t* dst, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Routed FP8 block-scaled MoE (DeepSeek expert shapes).
 * ------------------------------------------------------------------------- */

/* Router: per token, softmax over E fp32 logits, top-k experts (descending,
 * ties to the lower index), their softmax scores, renormalised to sum 1
 * (w / max(sum, 1e-20)) when renormalize != 0, times route_scale.  Replaces
 * DSv4 Gate.forward (src/torchinferno/models/deepseek_v4/tensor_parallel.py:
 * 760-780) / DeepSeekMoEGate.forward (src/torchinferno/models/deepseek_v32/
 * model.py:692-722) for softmax scoring without group limits.
 * logits [T,E] (E <= 1024), k <= 16; weights fp32 [T,k], ids int32 [T,k]. */
int ti_moe_route_topk(const float* logits, int T, int E, int k, int renormalize,
                      float route_scale, float* topk_weights, int32_t* topk_ids,
                      hipStream_t stream);

/* Workspace bytes of ti_fp8_moe (all intermediates; no allocation inside). */
size_t ti_fp8_moe_workspace_bytes(int T, int k, int E, int H, int I);

/* out[t] = bf16( sum over t's routed experts e, in expert order, of
 *   w2_e( bf16( w[t,e] * silu(w1_e x) * (w3_e x) ) ) )
 * with every w*_e a 128x128 block-scaled e4m3 Linear (1x128 activation quant,
 * bf16 output).  Replaces fused_mxfp4_moe and its align/grouped GEMMs
 * (src/torchinferno/kernels/deepseek_v4_marlin.py:267-411) and computes the
 * per-expert loop of MoE.forward (tensor_parallel.py:882-914).
 *   hidden bf16 [T,H]; topk_weights fp32 [T,k]; topk_ids int32 [T,k] (ids
 *   outside [0,E) are skipped); w13 e4m3 [E, 2I, H] = [w1; w3] per expert,
 *   s13 fp32 [E, 2I/128, H/128]; w2 e4m3 [E, H, I], s2 fp32 [E, H/128, I/128];
 *   clamp_limit > 0 clamps gate <= limit and |up| <= limit (swiglu_limit);
 *   round_scale != 0 gives both activation quants power-of-two scales
 *   (act_quant with scale_fmt "ue8m0", the DSv4 checkpoint setting,
 *   tensor_parallel.py:195-207,1199-1211); round_scale 2 also declares every
 *   s13 / s2 value a power of two (E8M0 weight scales), and the grouped GEMMs
 *   then apply all scales inside the MFMA, as ti_fp8_gemm_block_pow2;
 *   out bf16 [T,H].  H, I multiples of 128.  Deterministic. */
int ti_fp8_moe(const void* hidden, const float* topk_weights, const int32_t* topk_ids,
               int T, int k, const uint8_t* w13, const float* s13, const uint8_t* w2,
               const float* s2, int E, int H, int I, float clamp_limit, int round_scale,
               void* out, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* The same routed experts with MXFP4 weights (DSv4 expert_dtype "fp4"): every
 * w*_e is an e2m1 Linear with E8M0 scales per 32 K, applied as ti_fp4_gemm
 * (1x128 FP8 activations) -- the arithmetic of the reference's "tilelang-mxfp4"
 * expert path (Expert -> linear -> act_quant + fp4_gemm, tensor_parallel.py:
 * 195-207).  Replaces fused_mxfp4_moe (deepseek_v4_marlin.py:311-411).
 *   w13 e2m1 [E, 2I, H/2], s13 E8M0 per expert [2I, H/32] (scale_layout 0) or
 *   step-major [H/128][2I][4] (scale_layout 1); w2 e2m1 [E, H, I/2], s2 per
 *   expert [H, I/32] or [I/128][H][4]; workspace as ti_fp8_moe_workspace_bytes.
 *   round_scale 2: as 1, with the power-of-two activation scales applied
 *   inside the MFMA next to the weight's, as ti_fp4_gemm_pow2. */
int ti_fp4_moe(const void* hidden, const float* topk_weights, const int32_t* topk_ids,
               int T, int k, const uint8_t* w13, const uint8_t* s13, const uint8_t* w2,
               const uint8_t* s2, int scale_layout, int E, int H, int I, float clamp_limit,
               int round_scale, void* out, void* workspace, size_t workspace_bytes,
               hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TI_QUANT_H_ */
