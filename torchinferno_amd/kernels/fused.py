"""Fused activation -> per-token FP8 producers on MI355X.

Drop-ins for the three producers the reference's Llama3 decode path imports
from ``torchinferno.kernels.triton_ops`` (tensor_parallel.py:3073-3187):

* ``rms_norm_fp8_per_token(x, weight, eps) -> (q, scale)``
  (``triton_rms_norm_fp8_per_token``, triton_ops.py:2239-2265)
* ``add_rms_norm_fp8_per_token(x, residual, weight, eps) -> (hidden, q, scale)``
  (``triton_add_rms_norm_fp8_per_token``, triton_ops.py:2268-2297)
* ``swiglu_fp8_per_token(gate, up) -> (q, scale)``
  (``triton_swiglu_fp8_per_token``, triton_ops.py:2300-2333)

Same arguments, output shapes (``q`` viewed like the input, ``scale [rows, 1]``
fp32) and ``ValueError`` checks; the ``triton_*`` names are aliases.  Each is one
libti_quant.so launch, one 1024-thread workgroup per row with the row held in
registers: each input byte is read from HBM once, and only the e4m3 codes, the
scale and (add variant) the summed hidden state are written.  Widths up to 65536
(the reference stops at 8192).

The norm's weight is read in the activation dtype (a weight of another dtype is
cast first).  Roundings are fixed: fp64 sum of squares rounded once to fp32,
``rsqrt(v) = 1/sqrtf(v)``, ``exp`` in fp64 rounded to fp32.
"""
from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib

_ACT = (torch.bfloat16, torch.float16)
MAX_WIDTH = 65536  # a row is held in one workgroup's registers


def _outputs(x: Tensor) -> tuple[Tensor, Tensor, int, int]:
    # triton_ops.py:2226-2236
    if not x.is_cuda or x.ndim < 2:
        raise ValueError("per-token FP8 fusion requires a CUDA activation matrix")
    n = x.size(-1)
    rows = x.numel() // n if n else 0
    if n % 8:
        raise ValueError("per-token FP8 fusion requires a width divisible by 8")
    if n > MAX_WIDTH:
        raise ValueError(f"per-token FP8 fusion supports widths up to {MAX_WIDTH}")
    q = torch.empty((rows, n), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((rows, 1), dtype=torch.float32, device=x.device)
    return q, s, rows, n


def _norm_weight(x: Tensor, weight: Tensor) -> Tensor:
    if x.size(-1) != weight.numel() or weight.device != x.device:
        raise ValueError("RMSNorm weight must match the activation width and device")
    return weight.reshape(-1).to(x.dtype).contiguous()


def rms_norm_fp8_per_token(x: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """RMS-normalize and dynamically quantize each row to e4m3 in one pass."""
    if x.dtype not in _ACT:
        raise ValueError("fused RMSNorm FP8 quantization requires BF16 or FP16")
    w = _norm_weight(x, weight)
    q, s, rows, n = _outputs(x)
    _lib.require_device(x)
    if rows == 0:
        return q.view_as(x), s
    x2 = x.contiguous()
    _lib.call("ti_fp8_rmsnorm_quant_per_token", x2.data_ptr(), None, w.data_ptr(), _lib.dtype_code(x.dtype),
              rows, n, float(eps), None, q.data_ptr(), s.data_ptr(), _lib.stream_of(x))
    return q.view_as(x), s


def add_rms_norm_fp8_per_token(x: Tensor, residual: Tensor, weight: Tensor,
                               eps: float) -> tuple[Tensor, Tensor, Tensor]:
    """Add the residual, RMS-normalize, quantize; returns (x + residual, q, scale)."""
    if x.dtype not in _ACT:
        raise ValueError("fused add+RMSNorm FP8 quantization requires BF16 or FP16")
    if x.shape != residual.shape or x.device != residual.device or x.dtype != residual.dtype:
        raise ValueError("x and residual tensors must have matching shapes and devices")
    w = _norm_weight(x, weight)
    q, s, rows, n = _outputs(x)
    _lib.require_device(x)
    x2, r2 = x.contiguous(), residual.contiguous()
    hidden = torch.empty_like(x2)
    if rows == 0:
        return hidden.view_as(x), q.view_as(x), s
    _lib.call("ti_fp8_rmsnorm_quant_per_token", x2.data_ptr(), r2.data_ptr(), w.data_ptr(),
              _lib.dtype_code(x.dtype), rows, n, float(eps), hidden.data_ptr(), q.data_ptr(), s.data_ptr(),
              _lib.stream_of(x))
    return hidden.view_as(x), q.view_as(x), s


def swiglu_fp8_per_token(gate: Tensor, up: Tensor) -> tuple[Tensor, Tensor]:
    """SwiGLU (``silu(gate) * up``) then per-token e4m3; gate/up may be split views."""
    if gate.dtype not in _ACT:
        raise ValueError("fused SwiGLU FP8 quantization requires BF16 or FP16")
    if gate.shape != up.shape or gate.device != up.device or gate.dtype != up.dtype:
        raise ValueError("gate and up tensors must have matching shapes and devices")
    if gate.stride(-1) != 1 or up.stride(-1) != 1:
        raise ValueError("gate and up tensors must have contiguous last dimensions")
    q, s, rows, n = _outputs(gate)
    _lib.require_device(gate)
    if rows == 0:
        return q.view_as(gate), s
    g2, u2 = gate.view(-1, n), up.view(-1, n)  # rows strided, like the reference's views
    if rows > 1 and (g2.stride(0) % 8 or u2.stride(0) % 8):
        g2, u2 = g2.contiguous(), u2.contiguous()
    if g2.data_ptr() % 16 or u2.data_ptr() % 16:
        g2, u2 = g2.contiguous(), u2.contiguous()
    _lib.call("ti_fp8_swiglu_quant_per_token", g2.data_ptr(), g2.stride(0) if rows > 1 else n,
              u2.data_ptr(), u2.stride(0) if rows > 1 else n, _lib.dtype_code(gate.dtype), rows, n,
              q.data_ptr(), s.data_ptr(), _lib.stream_of(gate))
    return q.view_as(gate), s


triton_rms_norm_fp8_per_token = rms_norm_fp8_per_token
triton_add_rms_norm_fp8_per_token = add_rms_norm_fp8_per_token
triton_swiglu_fp8_per_token = swiglu_fp8_per_token
