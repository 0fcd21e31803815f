"""Oracle for the int4 W4A16 group-128 path (test infrastructure only).

Reference arithmetic followed:

* Symmetric "uint4b8" codes: stored q in [0, 15], value (q - 8) * s, one scale
  per (128-row K group, output column) -- src/torchinferno/kernels/marlin.py:108-131
  (quantizer) and the kernel contract at marlin.py:142-171.
* The dequantize-then-matmul reference the reference's own GPU test compares
  Marlin against -- tests/test_marlin_int4.py:40-49 (``_dequant_ref``):
  ``deq = q * s`` in fp32, ``a.float() @ deq``.

Canonical packed layout (the boundary format of this build, not Marlin's
permuted one): ``qweight`` int32 [K/8, N]; nibble i (bits 4i..4i+3, LSB first)
of word [r, n] is the code of row k = 8r + i, column n.  Scales are [K/G, N].

Pinning (tests/test_oracle_int4.py): pack/unpack on hand-built words; dequant
closed forms (code 8 -> 0, code 0 -> -8s, code 15 -> 7s, exact in fp32); the
GEMM reference on constructed weights whose product is known without the
formula (selection matrices give ``out = a`` / a permutation of ``a``'s
columns, all-ones codes give row sums); the RTN quantizer's scale rule and
reconstruction bound; fp64 brute force on tiny shapes.
"""
from __future__ import annotations

import numpy as np

from .numerics import round_to

ZERO_POINT = 8


def pack_int4(codes_kn: np.ndarray) -> np.ndarray:
    """codes uint8 [K, N] in [0,15] -> int32 [K/8, N], 8 nibbles per word along K."""
    codes = np.asarray(codes_kn, dtype=np.uint32)
    k, n = codes.shape
    if k % 8:
        raise ValueError("K must be a multiple of 8")
    if codes.max(initial=0) > 15:
        raise ValueError("codes must be in [0, 15]")
    c = codes.reshape(k // 8, 8, n)
    word = np.zeros((k // 8, n), dtype=np.uint32)
    for i in range(8):
        word |= c[:, i, :] << np.uint32(4 * i)
    return word.view(np.int32)


def unpack_int4(qweight: np.ndarray) -> np.ndarray:
    """int32 [K/8, N] -> codes uint8 [K, N]."""
    w = np.asarray(qweight).view(np.uint32)
    kw, n = w.shape
    out = np.empty((kw, 8, n), dtype=np.uint8)
    for i in range(8):
        out[:, i, :] = (w >> np.uint32(4 * i)) & 0xF
    return out.reshape(kw * 8, n)


def dequant_int4(qweight: np.ndarray, scales: np.ndarray, group_size: int = 128) -> np.ndarray:
    """(q - 8) * s as fp32 [K, N].  The product of a 4-bit integer and an fp16 or
    bf16 scale is exact in fp32, so this value is unique (tests/test_marlin_int4.py:47)."""
    codes = unpack_int4(qweight).astype(np.int32) - ZERO_POINT
    s = np.asarray(scales, dtype=np.float32)
    k, n = codes.shape
    if s.shape != (k // group_size, n):
        raise ValueError(f"scales must be [K/{group_size}, N], got {s.shape}")
    s_full = np.repeat(s, group_size, axis=0)
    return codes.astype(np.float32) * s_full


def dequant_int4_zp(qweight: np.ndarray, scales: np.ndarray, zeros: np.ndarray,
                    group_size: int = 128) -> np.ndarray:
    """Asymmetric group-wise int4 (GPTQ / AWQ checkpoints): (q - z) * s as fp32 [K, N],
    z the per-(group, column) zero point in [0, 15] -- the published GPTQ / AWQ
    dequantization (AWQ stores z, GPTQ "v1" stores z - 1; the caller passes z).
    Exact in fp32 for the same reason as ``dequant_int4``."""
    codes = unpack_int4(qweight).astype(np.int32)
    s = np.asarray(scales, dtype=np.float32)
    z = np.asarray(zeros, dtype=np.int32)
    k, n = codes.shape
    if s.shape != (k // group_size, n) or z.shape != s.shape:
        raise ValueError(f"scales and zeros must be [K/{group_size}, N]")
    return (codes - np.repeat(z, group_size, axis=0)).astype(np.float32) * np.repeat(s, group_size, axis=0)


def w4a16_reference(a: np.ndarray, qweight: np.ndarray, scales: np.ndarray,
                    group_size: int = 128, out_dtype: str | None = None) -> np.ndarray:
    """``a.float() @ dequant(W)`` with fp32 accumulation (tests/test_marlin_int4.py:49).

    ``a`` and ``scales`` are fp32 arrays holding fp16/bf16 values.  Returns fp32,
    or fp32 holding values rounded to ``out_dtype`` when given.
    """
    deq = dequant_int4(qweight, scales, group_size)
    out = np.asarray(a, dtype=np.float32) @ deq
    return round_to(out, out_dtype) if out_dtype else out


def w4a16_reference_zp(a: np.ndarray, qweight: np.ndarray, scales: np.ndarray, zeros: np.ndarray,
                       group_size: int = 128) -> np.ndarray:
    """``a.float() @ ((q - z) * s)`` with fp32 accumulation (asymmetric checkpoints)."""
    return np.asarray(a, dtype=np.float32) @ dequant_int4_zp(qweight, scales, zeros, group_size)


def quantize_int4_rtn(weight_kn: np.ndarray, group_size: int = 128,
                      scale_dtype: str = "bf16") -> tuple[np.ndarray, np.ndarray]:
    """Round-to-nearest symmetric int4 quantizer, restating
    src/torchinferno/kernels/marlin.py:117-128 on the canonical layout.

    weight_kn holds fp32 values already rounded to fp16 (the reference casts to
    fp16 first, marlin.py:117).  Per group and column:
    ``s = max(|max/7|, |min/-8|)`` clamped >= 1e-8 (fp32), ``q = clamp(rint(w/s),
    -8, 7) + 8`` (rint = half-to-even, like torch.round).  Codes are computed
    with the fp32 scale and the returned scale is then rounded to
    ``scale_dtype`` (marlin.py:127) -- the same order as the reference.
    Returns (qweight int32 [K/8, N], scales fp32 holding scale_dtype values).
    """
    w = np.asarray(weight_kn, dtype=np.float32)
    k, n = w.shape
    g = w.reshape(k // group_size, group_size, n)
    mx = g.max(axis=1)
    mn = g.min(axis=1)
    s = np.maximum(np.abs(mx / np.float32(7.0)), np.abs(mn / np.float32(-8.0)))
    s = np.maximum(s, np.float32(1e-8)).astype(np.float32)
    q = np.clip(np.rint(g / s[:, None, :]), -8, 7).astype(np.int32) + ZERO_POINT
    codes = q.reshape(k, n).astype(np.uint8)
    return pack_int4(codes), round_to(s, scale_dtype)
