"""Bit-level number formats used by the quantized path (oracle side).

* OCP float8 e4m3fn ("e4m3"): 1 sign, 4 exponent (bias 7), 3 mantissa bits,
  subnormals, no infinities, NaN = S.1111.111, max finite 448.  This is the
  format of ``torch.float8_e4m3fn`` that the reference stores FP8 weights and
  activations in (src/torchinferno/kernels/fp8.py:23-25).
* bfloat16: the upper half of an IEEE fp32.

Encoders round to nearest, ties to even (RNE), the rounding of a CUDA/Triton
``cvt.rn`` conversion and of torch's CPU ``.to(float8_e4m3fn)``.  Out-of-range
handling follows torch's non-saturating CPU cast: |x| >= 480 (the midpoint
above 448) encodes NaN; 448 <= |x| < 480 rounds to 448.  The quantizers on this
path divide by ``amax/448`` so they never reach that region.

Pinned by tests/test_oracle_numerics.py: exhaustive agreement with torch's own
casts (all 2^16 bf16 patterns, all 256 e4m3 codes, 10^6 random fp32 values).
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def e4m3_decode_table() -> np.ndarray:
    """fp32 value of each of the 256 e4m3fn codes, from the format definition."""
    out = np.empty(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = np.nan
        elif exp == 0:
            out[code] = sign * (man / 8.0) * 2.0 ** -6
        else:
            out[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return out


_E4M3_TABLE = e4m3_decode_table()


_E4M3_TABLE64 = _E4M3_TABLE.astype(np.float64)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    return _E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def e4m3_decode64(codes: np.ndarray) -> np.ndarray:
    """e4m3 codes -> exact values as fp64 (one table lookup)."""
    return _E4M3_TABLE64[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn codes (uint8), round-to-nearest-even."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    a = np.abs(x)
    abits = a.view(np.uint32).astype(np.uint64)
    # Normal range (|x| >= 2^-6): round the 23-bit mantissa to 3 bits (RNE),
    # then rebias the exponent from 127 to 7.
    lsb = (abits >> 20) & 1
    rounded = (abits + 0x7FFFF + lsb) >> 20
    normal = (rounded - (120 << 3)).astype(np.int64)
    # Subnormal range: value = m * 2^-9, m = rint(|x| * 2^9) (exact scaling,
    # numpy rint is half-to-even).  m == 8 is the smallest normal, code 0x08.
    sub = np.rint(np.where(np.isnan(a), 0.0, np.minimum(a, 1.0)).astype(np.float64) * 512.0).astype(np.int64)
    mag = np.where(a < 2.0 ** -6, sub, normal)
    mag = np.where(a >= 480.0, 0x7F, mag)
    mag = np.where(np.isnan(a), 0x7F, mag)
    mag = np.minimum(mag, 0x7F)  # 448 < |x| < 480 already rounds to 0x7E
    return (mag.astype(np.uint8) | sign).astype(np.uint8)


def e4m3_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest e4m3 value, returned as fp32."""
    return e4m3_decode(e4m3_encode(x))


def bf16_encode(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), RNE; NaN stays a quiet NaN."""
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    r = ((bits + 0x7FFF + lsb) >> 16).astype(np.uint32)
    r = np.where(np.isnan(x), (bits >> 16).astype(np.uint32) | 0x40, r)
    return r.astype(np.uint16)


def bf16_decode(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    return bf16_decode(bf16_encode(x))


def f16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest fp16 value (numpy's cast is IEEE RNE), as fp32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 values to a 16-bit activation dtype ("fp16" | "bf16")."""
    if dtype == "fp16":
        return f16_round(x)
    if dtype == "bf16":
        return bf16_round(x)
    if dtype == "fp32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)
