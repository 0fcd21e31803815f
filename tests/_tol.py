"""Elementwise error bounds for GEMM outputs against the oracle.

A bf16 output differs from the exact (fp64-accumulated) value by its own
rounding, at most half a bf16 ulp, plus the fp32 accumulation error, which is
bounded by a multiple of the unit round-off times the sum of |terms|.  The
bound used here is ``ulps * ulp_bf16(|ref|) + rel_sum * sum|terms|`` per
element: a dropped K block, a wrong scale index or a transposed operand moves
an element by a sizeable fraction of its own magnitude and fails it even where
the max-normalised metric ``max|y - ref| / max|ref|`` would not.
"""
from __future__ import annotations

import numpy as np


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    a = np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def abs_codes(codes: np.ndarray) -> np.ndarray:
    """e4m3 codes with the sign bit cleared (|value|), for the sum of |terms|."""
    return (np.asarray(codes, dtype=np.uint8) & 0x7F).astype(np.uint8)


def elementwise_ratio(got: np.ndarray, ref: np.ndarray, ref_abs: np.ndarray, ulps: float = 1.0,
                      rel_sum: float = 2.0 ** -16) -> float:
    """max over elements of |got - ref| / bound; <= 1 passes."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bound = ulps * bf16_ulp(ref) + rel_sum * np.abs(np.asarray(ref_abs, dtype=np.float64)) + 1e-30
    return float((np.abs(got - ref) / bound).max())
