"""Oracle for the fused activation -> per-token FP8 producers (test infrastructure only).

Reference arithmetic followed (src/torchinferno/kernels/triton_ops.py):

* RMSNorm -> FP8 (``_rms_norm_fp8_per_token_kernel``, :2127-2150):
  ``var = sum(x^2)/n``, ``normed = x * rsqrt(var + eps) * w`` in fp32, rounded
  to the activation dtype, ``s = max(amax/448, 1e-10)``, ``q = e4m3(normed/s)``.
* add + RMSNorm -> FP8 (:2153-2182): ``h = x + residual`` in fp32, stored in
  the activation dtype; the norm uses the fp32 ``h``.
* SwiGLU -> FP8 (:2185-2223): ``act = g / (1 + exp(-g)) * u`` in fp32, rounded to
  the activation dtype, then the same per-token quant.

The reference leaves three roundings implementation-defined (Triton's fp32 tree
sum, its approximate ``rsqrt`` and ``exp``).  This restatement -- and the GPU
kernels it checks -- fixes them: the sum of squares is accumulated in fp64 and
rounded once to fp32, ``rsqrt(v) = 1/sqrt(v)`` with IEEE fp32 sqrt and division,
and ``exp`` is evaluated in fp64 and rounded to fp32.  Parity with the reference
is the restore tolerance of its own tests
(tests/test_conversion_and_kernels.py:390-435); the producers equal "norm, then
per-token quant" by construction (pinned in tests/test_oracle_fused.py).
"""
from __future__ import annotations

import numpy as np

from .fp8 import quantize_activation_per_token
from .numerics import round_to

F32 = np.float32


def _rms(h: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    n = h.shape[-1]
    ss = (h.astype(np.float64) ** 2).sum(axis=-1, keepdims=True).astype(F32)
    var = (ss / F32(n)).astype(F32)
    r = (F32(1.0) / np.sqrt((var + F32(eps)).astype(F32))).astype(F32)
    return ((h * r).astype(F32) * w.astype(F32)).astype(F32)


def rms_norm_fp8_per_token(x: np.ndarray, w: np.ndarray, eps: float, act: str):
    """x [rows, n] values of the activation dtype `act` ("bf16"/"fp16") -> (codes, scale [rows,1])."""
    normed = round_to(_rms(np.asarray(x, F32), np.asarray(w, F32), eps), act)
    return quantize_activation_per_token(normed)


def add_rms_norm_fp8_per_token(x: np.ndarray, residual: np.ndarray, w: np.ndarray, eps: float, act: str):
    """-> (hidden in the activation dtype, codes, scale)."""
    h = (np.asarray(x, F32) + np.asarray(residual, F32)).astype(F32)
    normed = round_to(_rms(h, np.asarray(w, F32), eps), act)
    q, s = quantize_activation_per_token(normed)
    return round_to(h, act), q, s


def swiglu_activation(gate: np.ndarray, up: np.ndarray, act: str) -> np.ndarray:
    g = np.asarray(gate, F32)
    e = np.exp(-g.astype(np.float64)).astype(F32)
    return round_to(((g / (F32(1.0) + e)).astype(F32) * np.asarray(up, F32)).astype(F32), act)


def swiglu_fp8_per_token(gate: np.ndarray, up: np.ndarray, act: str):
    return quantize_activation_per_token(swiglu_activation(gate, up, act))
