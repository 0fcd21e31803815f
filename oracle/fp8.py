"""Oracle for FP8 e4m3 quantizers and W8A8 GEMMs (test infrastructure only).

Reference arithmetic followed (all fp32, IEEE division, RNE cast to e4m3):

* Per-output-channel weight quant -- src/torchinferno/kernels/fp8.py:129-138:
  ``s[n] = max(amax_k |W[n,k]| / 448, 1e-10)``, ``Wq = W / s`` -> e4m3.  The
  reference evaluates ``amax.to(float32) / 448.0`` with torch on the weight's
  GPU, where ATen turns division by a host Python scalar into a multiply by the
  fp32 reciprocal: ``s = amax * fl32(1/448)`` (that differs from the quotient in
  about half of all amax values, by one ulp).  ``W.float() / s`` divides by a
  device tensor, so that one is an IEEE quotient.
* Tensorwise weight quant -- fp8.py:119-126:
  ``(W.abs().amax() / 448).clamp(min=1e-6).to(float32)``: the amax, the
  product by fl32(1/448) and the clamp all stay in the weight's dtype, so the
  product is rounded to bf16/fp16 before the clamp (whose bound is
  ``dtype(1e-6)``) and the cast to fp32.
* Per-token activation quant -- the Triton ``_row_scale_cast_fp8`` at
  fp8.py:53-72: ``s[m] = max(amax_k |x[m,k]| / 448, 1e-10)``, ``xq = x / s``.
* Tensorwise activation quant -- fp8.py:141-181: the same dtype-rounded
  ``max(amax/448, 1e-6)`` as the tensorwise weight scale (fp8.py:154-155), or a
  caller scale; ``inv = 1/s`` (``scale.reciprocal()``, an IEEE fp32 quotient),
  ``xq = x * inv`` (fp8.py:49-51).
* The per-token activation scale comes from a Triton or sgl-kernel provider
  (fp8.py:53-72,234-238) that divides ``amax / 448.0``; its rounding is the
  provider's and is not pinned by anything in the reference, so the oracle uses
  the IEEE quotient.
* W8A8 linear -- fp8.py:250-327 (``_scaled_mm`` with ``scale_a [M,1]``,
  ``scale_b [1,N]``): ``out[m,n] = (sum_k xq[m,k] wq[n,k]) * xs[m] * ws[n]``.
* DeepSeek 1x128 activation quant -- src/torchinferno/kernels/
  deepseek_v4_tilelang_definitions.py:273-331: ``amax = max(amax, 1e-4)``,
  ``s = amax * (1/448)`` (or ``2^ceil(log2(amax/448))`` when a scale format is
  set, :255-270), ``y = clamp(x / s, -448, 448)`` -> e4m3.
* Block-scaled GEMM -- deepseek_v4_tilelang_definitions.py:436-485:
  ``C[m,n] = sum_j (sum_{k in block j} A[m,k] B[n,k]) * (a_s[m,j] * b_s[n//128, j])``.
* Block dequant -- src/torchinferno/models/deepseek_v4/ops.py:180-188.
* 128x128 weight block quant (block absmax/448); the
  weight-side quantizer is not in the reference (DeepSeek checkpoints ship
  quantized), so its formula comes from the benchmark definition.

Pinning (tests/test_oracle_fp8.py): e4m3 cast exhaustive vs torch; the
reference's known answer (tests/test_deepseek_v4.py:546-552) for block
dequant; the reference tests' restore tolerances (tests/test_conversion_and_
kernels.py:186-220, seeds 15/16); closed forms (scales are exactly amax/448,
the max element encodes as +-448); GEMM vs fp64 dequantize-then-matmul (the two
association orders of the same sum) and vs selection-matrix products.
"""
from __future__ import annotations

import numpy as np

from .numerics import E4M3_MAX, e4m3_decode, e4m3_decode64, e4m3_encode, round_to

F32 = np.float32
_INV_MAX = F32(1.0) / F32(E4M3_MAX)  # 1/448 rounded to fp32, the TileLang constant


def quantize_weight_fp8_per_channel(w_nk: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[N,K] fp32 (bf16 values) -> (codes uint8 [N,K], scale fp32 [1,N]).
    ``s = max(amax * fl32(1/448), 1e-10)`` -- ATen's GPU division by a host scalar."""
    w = np.asarray(w_nk, dtype=F32)
    s = np.maximum((np.abs(w).max(axis=1, keepdims=True) * _INV_MAX).astype(F32), F32(1e-10)).astype(F32)
    return e4m3_encode(w / s), s.T.copy()


def tensor_scale(amax: float, dtype: str = "bf16", eps: float = 1e-6) -> np.float32:
    """``(amax / 448).clamp(min=eps).to(float32)`` evaluated by torch on a GPU tensor
    of ``dtype`` (fp8.py:125,154-155): the product by fl32(1/448) is computed in
    fp32 and rounded to ``dtype``, the clamp bound is ``dtype(eps)``, then the
    value is widened to fp32.  ``amax`` is already a ``dtype`` value."""
    v = round_to(np.array([F32(amax) * _INV_MAX], F32), dtype)[0]
    lo = round_to(np.array([eps], F32), dtype)[0]
    return F32(max(v, lo))


def quantize_weight_fp8(w_nk: np.ndarray, dtype: str = "bf16") -> tuple[np.ndarray, np.float32]:
    """Tensorwise weight quant (fp8.py:119-126) of a ``dtype`` weight held as fp32."""
    w = np.asarray(w_nk, dtype=F32)
    s = tensor_scale(np.abs(w).max(), dtype)
    return e4m3_encode(w / s), s


def quantize_activation_per_token(x_mk: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """[M,K] -> (codes [M,K], scale fp32 [M,1])."""
    x = np.asarray(x_mk, dtype=F32)
    s = np.maximum(np.abs(x).max(axis=1, keepdims=True) / F32(E4M3_MAX), F32(1e-10)).astype(F32)
    return e4m3_encode(x / s), s


def quantize_activation_tensor(x: np.ndarray, scale: np.float32 | None = None,
                               dtype: str = "bf16") -> tuple[np.ndarray, np.float32]:
    """Tensorwise activation quant (fp8.py:141-181) of a ``dtype`` tensor held as fp32:
    dynamic scale as ``tensor_scale`` unless given, then ``x * (1/s)`` -> e4m3."""
    x = np.asarray(x, dtype=F32)
    if scale is None:
        scale = tensor_scale(np.abs(x).max(), dtype)
    inv = F32(F32(1.0) / F32(scale))
    return e4m3_encode(x * inv), F32(scale)


def fp8_linear_rowcol(xq: np.ndarray, xs: np.ndarray, wq: np.ndarray, ws: np.ndarray,
                      accum=np.float64) -> np.ndarray:
    """``(xq @ wq.T) * xs * ws`` -- scales broadcast: xs [M,1] or scalar, ws [1,N] or scalar.
    Returns fp32 (pre output rounding)."""
    a = e4m3_decode(xq).astype(accum)
    b = e4m3_decode(wq).astype(accum)
    acc = a @ b.T
    return (acc * np.asarray(xs, dtype=accum) * np.asarray(ws, dtype=accum)).astype(F32)


def _pow2_ceil_scale(amax: np.ndarray) -> np.ndarray:
    """2^ceil(log2(amax/448)) via the exponent/mantissa bits, as
    deepseek_v4_tilelang_definitions.py:255-270 computes it."""
    v = (np.asarray(amax, dtype=F32) * _INV_MAX).astype(F32)
    bits = v.view(np.uint32)
    e = ((bits >> 23) & 0xFF).astype(np.int64) - 127 + ((bits & 0x7FFFFF) != 0)
    return ((e + 127).astype(np.uint32) << 23).view(F32)


def act_quant_block(x_mk: np.ndarray, block: int = 128, round_scale: bool = False
                    ) -> tuple[np.ndarray, np.ndarray]:
    """[M,K] -> (codes [M,K], scale fp32 [M, K/block])."""
    x = np.asarray(x_mk, dtype=F32)
    m, k = x.shape
    if k % block:
        raise ValueError("K must be a multiple of the block size")
    xb = x.reshape(m, k // block, block)
    amax = np.maximum(np.abs(xb).max(axis=2), F32(1e-4)).astype(F32)
    s = _pow2_ceil_scale(amax) if round_scale else (amax * _INV_MAX).astype(F32)
    y = np.clip(xb / s[:, :, None], F32(-E4M3_MAX), F32(E4M3_MAX)).astype(F32)
    return e4m3_encode(y.reshape(m, k)), s


def quantize_weight_block(w_nk: np.ndarray, block: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """128x128 block weight quant: s = block absmax / 448.
    Returns (codes uint8 [N,K], scales fp32 [ceil(N/128), ceil(K/128)])."""
    w = np.asarray(w_nk, dtype=F32)
    n, k = w.shape
    nb, kb = -(-n // block), -(-k // block)
    pad = np.zeros((nb * block, kb * block), dtype=F32)
    pad[:n, :k] = w
    blocks = pad.reshape(nb, block, kb, block)
    amax = np.abs(blocks).max(axis=(1, 3))
    s = np.where(amax > 0, amax / F32(E4M3_MAX), F32(1.0)).astype(F32)
    s_full = np.repeat(np.repeat(s, block, 0), block, 1)[:n, :k]
    return e4m3_encode(w / s_full), s


def dequantize_block_fp8(codes_nk: np.ndarray, scale: np.ndarray, block: int = 128) -> np.ndarray:
    """ops.py:180-188: ``W.float() * repeat_interleave(scale, 128, both dims)``."""
    w = e4m3_decode(codes_nk)
    rows, cols = w.shape
    exp = (-(-rows // block), -(-cols // block))
    if tuple(scale.shape) != exp:
        raise ValueError(f"expected FP8 scale shape {exp}, got {tuple(scale.shape)}")
    full = np.repeat(np.repeat(np.asarray(scale, dtype=F32), block, 0), block, 1)
    return w * full[:rows, :cols]


def fp8_gemm_block(a_codes: np.ndarray, a_s: np.ndarray, b_codes: np.ndarray,
                   b_s: np.ndarray, block: int = 128) -> np.ndarray:
    """Per-K-block partial sums scaled by a_s[m,j]*b_s[n//128,j], accumulated in
    fp32 (deepseek_v4_tilelang_definitions.py:470-483).  Returns fp32 [M,N]."""
    a = e4m3_decode64(a_codes)
    b = e4m3_decode64(b_codes)
    m, k = a.shape
    n = b.shape[0]
    kb = -(-k // block)
    out = np.zeros((m, n), dtype=F32)
    bs_full = np.repeat(np.asarray(b_s, dtype=F32), block, axis=0)[:n]  # [N, kb]
    for j in range(kb):
        ks = slice(j * block, min(k, (j + 1) * block))
        part = (a[:, ks] @ b[:, ks].T).astype(F32)
        sc = (np.asarray(a_s, dtype=F32)[:, j:j + 1] * bs_full[:, j][None, :]).astype(F32)
        out = (out + part * sc).astype(F32)
    return out
