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

/* out[M, N] = a[M, K] @ dequant(W), fp32 accumulation, out in a's dtype.
 * Replaces torch.ops._C.marlin_gemm as called by marlin_int4_mm
 * (src/torchinferno/kernels/marlin.py:142-171).  dtype: TI_DTYPE_F16 or
 * TI_DTYPE_BF16 (activations, scales and output share it, as Marlin requires,
 * marlin.py:113-115).  Requires K % 128 == 0, N % 64 == 0, M >= 1. */
int ti_w4a16_gemm(const void* a, int dtype, const int32_t* packed_weight,
                  const void* packed_scales, void* out, int M, int N, int K, int group_size,
                  void* workspace, size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TI_QUANT_H_ */
