"""DeepSeek-style 128x128 block-scaled FP8 on MI355X -- drop-in for the reference's
``act_quant`` / ``fp8_gemm`` (src/torchinferno/kernels/deepseek_v4_tilelang.py:147-173,
207-223; kernels deepseek_v4_tilelang_definitions.py:273-331,436-485).

``act_quant(x)``: 1x128 activation quant, ``s = max(amax, 1e-4) / 448`` (or the
power-of-two ceiling when ``scale_fmt`` is set), ``y = clamp(x / s, +-448)``.
``fp8_gemm(a, a_s, b, b_s)``: ``C = sum_kb (a . b^T)_kb * a_s[:, kb] * b_s[n/128, kb]``,
bf16 out.  ``fp4_gemm(a, a_s, b, b_s)``: FP8 activations x MXFP4 weights
(deepseek_v4_tilelang_definitions.py:674-769): ``b`` e2m1 ``[N, K/2]``, ``b_s`` one
E8M0 scale per 32 K (``float8_e8m0fnu``, or fp32 powers of two).  All run
libti_quant.so's gfx950 kernels.  Block scales may be stored as fp32 or, as the
reference's ``scale_dtype=float8_e8m0fnu`` (tensor_parallel.py:1211-1212), as
E8M0 bytes: those are powers of two, widened to fp32 exactly before the GEMM;
E8M0 activation scales are produced only with a ``scale_fmt`` (power-of-two
scales), the only combination the reference model configures.  When every scale
of a GEMM is a power of two -- ``scale_dtype=float8_e8m0fnu``, or ``linear`` with a
``scale_fmt`` and E8M0 weight scales (MXFP4 weights always have them) -- the GEMM
applies the scales as MFMA exponents (``ti_fp8_gemm_block_pow2`` /
``ti_fp4_gemm_pow2``) instead of folding each 128-K partial sum in fp32.
"""
from __future__ import annotations

import torch
from torch import Tensor

import os

from .. import _lib
from .fp8 import FP8_E4M3, _ws_args

BLOCK = 128


def _pow2_enabled() -> bool:
    """Power-of-two (E8M0) scales go to the GEMMs that apply them inside the MFMA
    unless ``TI_ROCM_POW2_MFMA=0`` (then the fp32-scale GEMMs run them)."""
    return os.environ.get("TI_ROCM_POW2_MFMA", "1") != "0"


E8M0 = torch.float8_e8m0fnu


def _check_scale_dtype(scale_dtype: torch.dtype) -> None:
    if scale_dtype not in (torch.float32, E8M0):
        raise ValueError("block scales must be stored as float32 or float8_e8m0fnu")


def _f32_scales(s: Tensor) -> Tensor:
    """fp32 view of block scales: fp32 as is, E8M0 widened (exact: powers of two)."""
    if s.dtype == torch.float32:
        return s
    if s.dtype == E8M0:
        return s.float()
    raise ValueError("block scales must be float32 or float8_e8m0fnu")


def _weight_scales_f32(weight: Tensor, weight_scale: Tensor) -> Tensor:
    """``weight_scale`` as fp32, cached on the weight when it is stored as E8M0
    (weight preparation: the conversion runs once per weight)."""
    if weight_scale.dtype == torch.float32:
        return weight_scale
    cached = getattr(weight, "_ti_scale_f32", None)
    if cached is None or cached[0] is not weight_scale:
        cached = (weight_scale, _f32_scales(weight_scale).contiguous())
        weight._ti_scale_f32 = cached
    return cached[1]


def act_quant(
    x: Tensor,
    block_size: int = BLOCK,
    scale_fmt: str | None = None,
    scale_dtype: torch.dtype = torch.float32,
    inplace: bool = False,
) -> Tensor | tuple[Tensor, Tensor]:
    """Block-wise FP8 activation quant.  Returns ``(y e4m3 [..., N], s fp32 [..., N/128])``;
    with ``inplace=True`` writes the quantize-dequantize round trip back into ``x``
    (bf16/fp16) and returns it, as the reference does."""
    n = x.size(-1)
    if block_size != BLOCK:
        raise ValueError("FP8 block quantization supports block_size=128 only")
    if n % block_size:
        raise ValueError("FP8 quantization width must be divisible by block size")
    _check_scale_dtype(scale_dtype)
    if scale_dtype == E8M0 and scale_fmt is None:
        raise ValueError("float8_e8m0fnu activation scales need a scale_fmt (power-of-two scales)")
    _lib.require_device(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("FP8 block quantization input must be bf16 or fp16")
    value = x.contiguous()
    rows = value.numel() // n
    y = torch.empty(value.shape, dtype=FP8_E4M3, device=x.device)
    s = torch.empty((*value.shape[:-1], n // block_size), dtype=torch.float32, device=x.device)
    _lib.call("ti_fp8_quant_block", value.data_ptr(), _lib.dtype_code(value.dtype), rows, n, block_size,
              int(scale_fmt is not None), y.data_ptr(), s.data_ptr(), 0, _lib.stream_of(value))
    if inplace:
        deq = y.view(rows, n // block_size, block_size).float() * s.view(rows, -1, 1)
        x.copy_(deq.view(x.shape).to(x.dtype))
        return x
    return y, (s if scale_dtype == torch.float32 else s.to(E8M0))


def fp8_gemm(
    a: Tensor,
    a_s: Tensor,
    b: Tensor,
    b_s: Tensor,
    scale_dtype: torch.dtype = torch.float32,
) -> Tensor:
    """``C[M,N] = A[M,K] @ B[N,K]^T`` with per-128 block FP8 scaling on both A and B
    (bf16 out).  ``a`` e4m3 ``[..., K]``, ``a_s`` fp32 ``[..., K/128]``, ``b`` e4m3 ``[N, K]``,
    ``b_s`` fp32 ``[ceil(N/128), K/128]``."""
    if not all(t.is_contiguous() for t in (a, a_s, b, b_s)):
        raise ValueError("FP8 GEMM inputs and scales must be contiguous")
    _check_scale_dtype(scale_dtype)
    if a.dtype != FP8_E4M3 or b.dtype != FP8_E4M3:
        raise ValueError("FP8 GEMM operands must be float8_e4m3fn")
    if a_s.dtype != scale_dtype or b_s.dtype != scale_dtype:
        raise ValueError("FP8 GEMM scales must have the given scale_dtype")
    pow2 = scale_dtype == E8M0
    a_s, b_s = _f32_scales(a_s), _f32_scales(b_s)
    _lib.require_device(a, a_s, b, b_s)
    k = a.size(-1)
    m = a.numel() // k
    n = b.size(0)
    if b.ndim != 2 or b.size(1) != k:
        raise ValueError("FP8 GEMM weight must be [N, K] with the activation's K")
    if a_s.numel() != m * (k // BLOCK) or tuple(b_s.shape) != (-(-n // BLOCK), -(-k // BLOCK)):
        raise ValueError("FP8 GEMM block scales must be a_s [M, K/128] and b_s [ceil(N/128), K/128]")
    return _fp8_gemm_raw(a, a_s, 0, b, b_s, pow2)


def _fp8_gemm_raw(a: Tensor, a_s: Tensor, a_layout: int, b: Tensor, b_s: Tensor, pow2: bool = False) -> Tensor:
    """Block GEMM; ``pow2``: every scale is a power of two (E8M0 values), which
    ``ti_fp8_gemm_block_pow2`` applies inside the MFMA."""
    k = a.size(-1)
    m = a.numel() // k
    n = b.size(0)
    out = torch.empty((*a.shape[:-1], n), dtype=torch.bfloat16, device=a.device)
    if m == 0:
        return out
    pow2 = pow2 and _pow2_enabled()
    ws, ws_bytes = _ws_args(a.device, m, n, k, 3 if pow2 else 1)
    _lib.call("ti_fp8_gemm_block_pow2" if pow2 else "ti_fp8_gemm_block", a.data_ptr(), a_s.data_ptr(), a_layout,
              b.data_ptr(), b_s.data_ptr(), out.data_ptr(), _lib.TI_DTYPE_BF16, m, n, k, ws, ws_bytes,
              _lib.stream_of(a))
    return out


def _act_quant_stepmajor(x: Tensor, round_scale: bool = False) -> tuple[Tensor, Tensor]:
    """1x128 quant with the scales step-major, ``[K/128, rows]`` (the layout the
    GEMMs read as one contiguous run per tile and K step); power-of-two scales
    when ``round_scale``."""
    _lib.require_device(x)
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("FP8 block quantization input must be bf16 or fp16")
    n = x.size(-1)
    if n % BLOCK:
        raise ValueError("FP8 quantization width must be divisible by block size")
    value = x.contiguous()
    rows = value.numel() // n
    y = torch.empty(value.shape, dtype=FP8_E4M3, device=x.device)
    s = torch.empty((n // BLOCK, rows), dtype=torch.float32, device=x.device)
    if rows:
        _lib.call("ti_fp8_quant_block", value.data_ptr(), _lib.dtype_code(value.dtype), rows, n, BLOCK,
                  int(round_scale), y.data_ptr(), s.data_ptr(), 1, _lib.stream_of(value))
    return y, s


FP4 = torch.float4_e2m1fn_x2


def e8m0_bytes(scale: Tensor) -> Tensor:
    """MXFP4 weight scales as E8M0 bytes: ``float8_e8m0fnu`` (or uint8) storage as
    is; fp32 only when every value is an exact power of two, else ValueError."""
    if scale.dtype == torch.float8_e8m0fnu:
        return scale.contiguous().view(torch.uint8)
    if scale.dtype == torch.uint8:
        return scale.contiguous()
    if scale.dtype != torch.float32:
        raise ValueError("MXFP4 scales must be float8_e8m0fnu, uint8 E8M0 bytes or fp32 powers of two")
    b = scale.to(torch.float8_e8m0fnu)
    if not torch.equal(b.float(), scale):
        raise ValueError("fp32 MXFP4 scales must be exact powers of two")
    return b.contiguous().view(torch.uint8)


def fp4_scale_stepmajor(scale_bytes: Tensor) -> Tensor:
    """E8M0 bytes ``[..., N, K/32]`` -> step-major ``[..., K/128, N, 4]`` (one
    contiguous read per tile and K step in the GEMM); weight preparation."""
    _lib.require_device(scale_bytes)
    *lead, n, kb = scale_bytes.shape
    if kb % 4:
        raise ValueError("MXFP4 scales need K divisible by 128")
    src = scale_bytes.contiguous().view(-1, n, kb)
    dst = torch.empty((src.size(0), kb // 4, n, 4), dtype=torch.uint8, device=src.device)
    for i in range(src.size(0)):
        _lib.call("ti_fp4_scale_stepmajor", src[i].data_ptr(), n, kb * 32, dst[i].data_ptr(),
                  _lib.stream_of(src))
    return dst.view(*lead, kb // 4, n, 4)


def _fp4_gemm_raw(a: Tensor, a_s: Tensor, a_layout: int, b: Tensor, eb: Tensor, layout: int, n: int,
                  pow2: bool = False) -> Tensor:
    """MXFP4 GEMM; ``pow2``: the activation scales are powers of two, which
    ``ti_fp4_gemm_pow2`` applies inside the MFMA with the weight's."""
    k = a.size(-1)
    m = a.numel() // k
    out = torch.empty((*a.shape[:-1], n), dtype=torch.bfloat16, device=a.device)
    if m == 0:
        return out
    pow2 = pow2 and _pow2_enabled()
    ws, ws_bytes = _ws_args(a.device, m, n, k, 4 if pow2 else 2)
    _lib.call("ti_fp4_gemm_pow2" if pow2 else "ti_fp4_gemm", a.data_ptr(), a_s.data_ptr(), a_layout, b.data_ptr(),
              eb.data_ptr(), layout, out.data_ptr(), _lib.TI_DTYPE_BF16, m, n, k, ws, ws_bytes, _lib.stream_of(a))
    return out


def fp4_gemm(
    a: Tensor,
    a_s: Tensor,
    b: Tensor,
    b_s: Tensor,
    scale_dtype: torch.dtype = torch.float32,
) -> Tensor:
    """``C[M,N] = A_fp8[M,K] @ B_fp4[N,K]^T`` (bf16 out): ``a`` e4m3 ``[..., K]`` with
    fp32 1x128 scales ``a_s [..., K/128]``; ``b`` ``float4_e2m1fn_x2`` (or uint8)
    ``[N, K/2]``; ``b_s`` per-32 E8M0 scales ``[N, K/32]``."""
    if not all(t.is_contiguous() for t in (a, a_s, b, b_s)):
        raise ValueError("FP4 GEMM inputs and scales must be contiguous")
    _check_scale_dtype(scale_dtype)
    if a.dtype != FP8_E4M3 or b.dtype not in (FP4, torch.uint8):
        raise ValueError("FP4 GEMM operands must be float8_e4m3fn activations and float4_e2m1fn_x2 weights")
    if a_s.dtype != scale_dtype:
        raise ValueError("FP4 GEMM activation scales must have the given scale_dtype")
    pow2 = scale_dtype == E8M0
    a_s = _f32_scales(a_s)
    _lib.require_device(a, a_s, b, b_s)
    k = a.size(-1)
    m = a.numel() // k
    n = b.size(0)
    if b.ndim != 2 or b.size(1) * 2 != k:
        raise ValueError("FP4 GEMM weight must be [N, K/2] packed e2m1 with the activation's K")
    if k % BLOCK:
        raise ValueError("FP4 GEMM needs K divisible by 128")
    eb = e8m0_bytes(b_s)
    if a_s.numel() != m * (k // BLOCK) or tuple(eb.shape) != (n, k // 32):
        raise ValueError("FP4 GEMM scales must be a_s [M, K/128] and b_s [N, K/32]")
    return _fp4_gemm_raw(a, a_s, 0, b, eb, 0, n, pow2)


def linear(x: Tensor, weight: Tensor, weight_scale: Tensor, scale_fmt: str | None = None,
           scale_dtype: torch.dtype = torch.float32) -> Tensor:
    """DeepSeek ``linear`` for an e4m3 or MXFP4 weight (src/torchinferno/models/
    deepseek_v4/tensor_parallel.py:195-207): ``act_quant(x, 128, scale_fmt,
    scale_dtype)`` then ``fp8_gemm`` / ``fp4_gemm``, bf16 out.  ``scale_fmt`` set
    ("ue8m0" on the DSv4 checkpoint path) rounds the activation scales up to powers
    of two.  The activation scales stay internal, so they are kept fp32 and
    step-major (``[K/128, rows]``), which the GEMMs read fastest; E8M0 storage of
    them would hold the same powers of two."""
    _check_scale_dtype(scale_dtype)
    if scale_dtype == E8M0 and scale_fmt is None:
        raise ValueError("float8_e8m0fnu activation scales need a scale_fmt (power-of-two scales)")
    round_scale = scale_fmt is not None
    if weight.dtype == FP4:
        # The step-major copy of the weight's scales is built on first use and
        # cached on the weight (like the reference's per-layer weight caches).
        cached = getattr(weight, "_ti_fp4_scale_stepmajor", None)
        if cached is None or cached[0] is not weight_scale:
            eb = e8m0_bytes(weight_scale)
            if eb.ndim != 2 or tuple(eb.shape) != (weight.size(0), weight.size(1) // 16):
                raise ValueError("MXFP4 weight scale must be [N, K/32]")
            cached = (weight_scale, fp4_scale_stepmajor(eb))
            weight._ti_fp4_scale_stepmajor = cached
        if x.size(-1) != weight.size(1) * 2:
            raise ValueError("MXFP4 weight K does not match the activation")
        xq, xs = _act_quant_stepmajor(x, round_scale)
        return _fp4_gemm_raw(xq, xs, 1, weight, cached[1], 1, weight.size(0), round_scale)
    if weight.dtype != FP8_E4M3 or weight_scale.dtype not in (torch.float32, E8M0):
        raise ValueError("block-FP8 linear needs a float8_e4m3fn weight with fp32 or E8M0 block scales")
    k = x.size(-1)
    n = weight.size(0)
    if weight.ndim != 2 or weight.size(1) != k:
        raise ValueError("FP8 GEMM weight must be [N, K] with the activation's K")
    if tuple(weight_scale.shape) != (-(-n // BLOCK), -(-k // BLOCK)):
        raise ValueError("FP8 GEMM weight scale must be [ceil(N/128), K/128]")
    _lib.require_device(weight, weight_scale)
    sb = _weight_scales_f32(weight, weight_scale)
    xq, xs = _act_quant_stepmajor(x, round_scale)
    # ue8m0 activations with E8M0 weight scales: all scales are powers of two
    return _fp8_gemm_raw(xq, xs, 1, weight.contiguous(), sb.contiguous(), round_scale and weight_scale.dtype == E8M0)
