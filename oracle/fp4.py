"""Oracle for MXFP4 weights and the FP8-activation x FP4-weight GEMM (test
infrastructure only).

Reference arithmetic followed:

* Weight format -- src/torchinferno/kernels/deepseek_v4_tilelang_definitions.py:
  674-769 (``fp4_gemm_kernel`` / ``fp4_gemm``): ``B`` is ``[N, K//2]``
  ``float4_e2m1fn_x2``, two e2m1 values per byte packed along K (element 2i in
  the low nibble, 2i+1 in the high nibble, torch's packing), with one E8M0
  scale per 32 consecutive K elements of a row (``scales_b [N, K//32]``).
* e2m1 (OCP MX): sign, 2 exponent bits (bias 1), 1 mantissa bit; exponent 0 is
  subnormal.  The 8 magnitudes are 0, 0.5, 1, 1.5, 2, 3, 4, 6.
* E8M0: value ``2^(byte - 127)``; byte 255 is NaN.
* GEMM -- :703-742: per 32-wide K block, ``C_local = A_fp8 @ B_fp8^T`` (the fp4
  values cast to e4m3 exactly through fp32), then
  ``C += C_local * scale_a[m, k // 128] * scale_b[n, k // 32]`` in fp32;
  activations are the 1x128 block-FP8 ``act_quant`` output (oracle/fp8.py).

Pinning (tests/test_oracle_fp4.py): the e2m1 table against the OCP formula
and against torch's own ``float4_e2m1fn_x2`` packing where torch can convert;
e8m0 against torch's ``float8_e8m0fnu`` conversion; nibble order against
torch's ``float4_e2m1fn_x2`` element view; the GEMM against an fp64
dequantize-then-matmul (a different association of the same sum) and against
one-hot closed forms.
"""
from __future__ import annotations

import numpy as np

from .numerics import e4m3_decode

F32 = np.float32
E2M1_MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=F32)


def e2m1_decode(codes: np.ndarray) -> np.ndarray:
    """4-bit codes (0..15) -> fp32 values."""
    c = np.asarray(codes).astype(np.int64) & 0xF
    mag = E2M1_MAGNITUDES[c & 7]
    return np.where(c & 8, -mag, mag).astype(F32)


def unpack_fp4(packed: np.ndarray) -> np.ndarray:
    """[..., K//2] uint8 -> [..., K] codes, low nibble first."""
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


def pack_fp4(codes: np.ndarray) -> np.ndarray:
    c = np.asarray(codes, dtype=np.uint8) & 0xF
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def e8m0_decode(b: np.ndarray) -> np.ndarray:
    e = np.asarray(b).astype(np.int64)
    v = np.ldexp(np.ones(e.shape, dtype=np.float64), e - 127).astype(F32)
    return np.where(e == 255, np.float32(np.nan), v).astype(F32)


def dequantize_fp4(packed_nk: np.ndarray, scale_e8m0: np.ndarray) -> np.ndarray:
    """[N, K//2] packed + [N, K//32] e8m0 -> fp32 [N, K] (exact: every product of
    an e2m1 value and a power of two is representable)."""
    w = e2m1_decode(unpack_fp4(packed_nk))
    s = np.repeat(e8m0_decode(scale_e8m0), 32, axis=1)[:, : w.shape[1]]
    return (w.astype(np.float64) * s.astype(np.float64)).astype(F32)


def fp4_gemm(a_codes: np.ndarray, a_s: np.ndarray, b_packed: np.ndarray, b_s: np.ndarray) -> np.ndarray:
    """FP8 [M,K] (1x128 fp32 scales a_s [M, K//128]) x FP4 [N,K] (e8m0 b_s
    [N, K//32]) -> fp32 [M, N], following the reference's per-32-block fp32
    accumulation order."""
    a = e4m3_decode(a_codes).astype(np.float64)
    b = e2m1_decode(unpack_fp4(b_packed)).astype(np.float64)
    m, k = a.shape
    n = b.shape[0]
    bs = e8m0_decode(b_s)
    out = np.zeros((m, n), dtype=F32)
    for j in range(k // 32):
        ks = slice(j * 32, (j + 1) * 32)
        part = (a[:, ks] @ b[:, ks].T).astype(F32)
        sc = (np.asarray(a_s, dtype=F32)[:, (j * 32) // 128][:, None] * bs[:, j][None, :]).astype(F32)
        out = (out + part * sc).astype(F32)
    return out


def fp4_gemm_f64(a_codes: np.ndarray, a_s: np.ndarray, b_packed: np.ndarray, b_s: np.ndarray) -> np.ndarray:
    """The same product in one fp64 matmul of the dequantized operands."""
    a = e4m3_decode(a_codes).astype(np.float64) * np.repeat(np.asarray(a_s, np.float64), 128, axis=1)
    return a @ dequantize_fp4(b_packed, b_s).astype(np.float64).T
