"""FP8 e4m3 W8A8 linears on MI355X -- drop-in for the reference's FP8 kernel module.

Mirrors the public surface of src/torchinferno/kernels/fp8.py (``quantize_weight_fp8``,
``quantize_weight_fp8_per_channel``, ``quantize_activation_fp8``,
``fp8_prefill_linear``, ``fp8_per_token_linear``, ``fp8_per_token_linear_quantized``,
``fp8_available``; fp8.py:119-331) and of ``scaled_mm_out``
(src/torchinferno/kernels/sgl_fp8_out.py:134-183): same argument meaning, same
``ValueError`` checks, same caller-owned ``out`` contract, and ``scaled_mm_out``
returns ``None`` outside its supported region.  Every quantizer and GEMM runs on
libti_quant.so's gfx950 kernels (``ti_fp8_*``); torch supplies only the tensorwise
``amax`` reduction and the reciprocal, as in the reference.

The GEMMs take weights in the reference's ``[N, K]`` e4m3 layout, so checkpoints
and caches prepared for the reference load unchanged, and also in this build's
tiled layout (``tile_weight_fp8``: ``[N/128, K/128, 128, 128]``, each 128-K step
of 128 rows one contiguous 16 KiB run), which the hooks' load-time weight caches
use: measured 20-33% faster than ``[N, K]`` for the config-2 gate_up weight
(470 MB) at decode M, where the row layout's 128-byte runs at an 8 KiB stride
stream at 4.7 TB/s and the tiles at 5.9 TB/s.
"""
from __future__ import annotations

import threading

import torch
from torch import Tensor

from .. import _lib

FP8_E4M3 = torch.float8_e4m3fn
FP8_E4M3_MAX = 448.0
_FP8_MAX = FP8_E4M3_MAX
_OUT_DTYPES = (torch.bfloat16, torch.float16)
_ACT_DTYPES = (torch.bfloat16, torch.float16)
K_ALIGN = 128  # K granularity of the GEMM kernels

_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], Tensor] = {}


def fp8_available() -> bool:
    """True when libti_quant.so loads (fp8.py:330-331 reports Triton availability)."""
    return _lib.available()


def gemm_workspace(device: torch.device, nbytes: int) -> Tensor | None:
    """Zero-filled split-K workspace of at least ``nbytes`` for ``device``, shared by
    the FP8 GEMMs of this process.  Kernels leave its ticket words zero, so it is
    reused across calls; calls sharing it must be ordered on one stream.  It grows
    (allocates) only when a larger problem arrives -- prepare the largest shape
    once before capturing graphs."""
    if nbytes <= 0:
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, 0)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() * 4 < nbytes:
            ws = torch.zeros((nbytes + 3) // 4, dtype=torch.int32, device=device)
            _workspaces[key] = ws
        return ws


def _ws_args(device: torch.device, m: int, n: int, k: int, mode: int) -> tuple[int | None, int]:
    need = int(_lib.lib().ti_fp8_gemm_workspace_bytes(m, n, k, mode))
    ws = gemm_workspace(device, need)
    if ws is None:
        return None, 0
    return ws.data_ptr(), ws.numel() * 4


# --------------------------------------------------------------------------- quantizers


def quantize_weight_fp8(weight: Tensor) -> tuple[Tensor, Tensor]:
    """One-time tensorwise e4m3 quant of an [N,K] weight (fp8.py:119-126):
    ``scale = max(amax / 448, 1e-6)``, ``wq = weight / scale``.  Weight preparation,
    run once before any graph capture."""
    scale = (weight.abs().amax() / _FP8_MAX).clamp(min=1e-6).to(torch.float32)
    wq = (weight.to(torch.float32) / scale).to(FP8_E4M3)
    return wq, scale


def _per_row_quant(x2d: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    _lib.require_device(x2d)
    if x2d.dtype not in _ACT_DTYPES:
        raise ValueError("FP8 quantization input must be bf16 or fp16")
    x2d = x2d.contiguous()
    rows, cols = x2d.shape
    xq = torch.empty((rows, cols), dtype=FP8_E4M3, device=x2d.device)
    xs = torch.empty((rows, 1), dtype=torch.float32, device=x2d.device)
    _lib.call("ti_fp8_quant_per_token", x2d.data_ptr(), _lib.dtype_code(x2d.dtype), rows, cols, eps,
              xq.data_ptr(), xs.data_ptr(), _lib.stream_of(x2d))
    return xq, xs


def quantize_weight_fp8_per_channel(weight: Tensor) -> tuple[Tensor, Tensor]:
    """Quantize an [N, K] weight with one FP8 scale per output channel (fp8.py:129-138):
    ``s[n] = max(amax_k |W[n,k]| / 448, 1e-10)`` with the division done as torch does
    it on a GPU tensor (a multiply by fl32(1/448)); returns ``(wq [N,K], s [1,N])``."""
    if weight.ndim != 2:
        raise ValueError("FP8 linear weights must have shape [N, K]")
    _lib.require_device(weight)
    if weight.dtype not in _ACT_DTYPES:
        raise ValueError("FP8 quantization input must be bf16 or fp16")
    w = weight.contiguous()
    n, k = w.shape
    wq = torch.empty((n, k), dtype=FP8_E4M3, device=w.device)
    ws = torch.empty((1, n), dtype=torch.float32, device=w.device)
    _lib.call("ti_fp8_quant_weight_per_channel", w.data_ptr(), _lib.dtype_code(w.dtype), n, k,
              wq.data_ptr(), ws.data_ptr(), _lib.stream_of(w))
    return wq, ws


def quantize_activation_fp8_per_token(x: Tensor) -> tuple[Tensor, Tensor]:
    """Dynamic per-token quant of ``x [..., K]`` -> (xq [rows, K] e4m3, scale [rows, 1]);
    the ``_row_scale_cast_fp8`` / ``sgl_per_token_quant_fp8`` step of
    fp8_per_token_linear (fp8.py:99-116,226-238)."""
    return _per_row_quant(x.reshape(-1, x.size(-1)), 1e-10)


def quantize_activation_fp8(
    x: Tensor,
    *,
    scale: Tensor | None = None,
    inverse_scale: Tensor | None = None,
    out: Tensor | None = None,
) -> tuple[Tensor, Tensor]:
    """Tensorwise activation quant (fp8.py:141-181): ``scale = max(amax/448, 1e-6)``
    unless given, ``xq = e4m3(x * (1/scale))``.  Returns (xq same shape, scale)."""
    _lib.require_device(x)
    if scale is None:
        scale = (x.abs().amax() / _FP8_MAX).clamp(min=1e-6).to(torch.float32)
    elif scale.numel() != 1 or scale.device != x.device:
        raise ValueError("FP8 activation scale must be a scalar on the input device")
    else:
        scale = scale.to(torch.float32)
    if inverse_scale is None:
        inverse_scale = scale.reciprocal()
    elif inverse_scale.numel() != 1 or inverse_scale.device != x.device:
        raise ValueError("FP8 inverse activation scale must be a scalar on the input device")
    else:
        inverse_scale = inverse_scale.to(torch.float32)
    xq = out if out is not None else torch.empty(x.shape, device=x.device, dtype=FP8_E4M3)
    if xq.shape != x.shape or xq.device != x.device or xq.dtype != FP8_E4M3:
        raise ValueError("FP8 activation output must match the input shape and device")
    if x.dtype not in _ACT_DTYPES:
        raise ValueError("FP8 activation quantization input must be bf16 or fp16")
    xc = x.contiguous()
    inv = inverse_scale.reshape(1).contiguous()
    _lib.call("ti_fp8_quant_tensor", xc.data_ptr(), _lib.dtype_code(xc.dtype), xc.numel(), inv.data_ptr(),
              xq.data_ptr(), _lib.stream_of(xc))
    return xq, scale


# --------------------------------------------------------------------------- GEMMs


def is_tiled_weight(w: Tensor) -> bool:
    """A weight in the layout ``tile_weight_fp8`` writes."""
    return w.ndim == 4 and w.dtype == FP8_E4M3 and w.size(2) == 128 and w.size(3) == 128


def weight_nk(w: Tensor) -> tuple[int, int]:
    """Logical ``(N, K)`` of an ``[N, K]`` or tiled e4m3 weight."""
    if is_tiled_weight(w):
        return w.size(0) * 128, w.size(1) * 128
    return w.size(0), w.size(1)


def tile_weight_fp8(weight_q: Tensor) -> Tensor:
    """``[N, K]`` e4m3 weight -> ``[N/128, K/128, 128, 128]`` (N, K multiples of 128):
    block (n // 128, k // 128), row n % 128, byte k % 128.  No reference counterpart."""
    if weight_q.ndim != 2 or weight_q.dtype != FP8_E4M3:
        raise ValueError("tile_weight_fp8 expects an [N, K] e4m3 weight")
    n, k = weight_q.shape
    if n % 128 or k % 128:
        raise ValueError("tile_weight_fp8 needs N and K multiples of 128")
    _lib.require_device(weight_q)
    src = weight_q.contiguous()
    out = torch.empty((n // 128, k // 128, 128, 128), dtype=FP8_E4M3, device=weight_q.device)
    _lib.call("ti_fp8_tile_weight", src.data_ptr(), n, k, out.data_ptr(), _lib.stream_of(src))
    return out


def maybe_tile_weight_fp8(weight_q: Tensor) -> Tensor:
    """The tiled form when the shape allows it (and ``TI_ROCM_FP8_TILED_WEIGHTS`` is
    not ``0``), else the weight unchanged."""
    import os
    if os.environ.get("TI_ROCM_FP8_TILED_WEIGHTS", "1") == "0":
        return weight_q
    if (weight_q.ndim == 2 and weight_q.dtype == FP8_E4M3 and weight_q.size(0) % 128 == 0
            and weight_q.size(1) % 128 == 0 and weight_q.is_cuda):
        return tile_weight_fp8(weight_q)
    return weight_q


def _pad_k(t: Tensor, k_pad: int) -> Tensor:
    out = torch.zeros((t.size(0), k_pad), dtype=t.dtype, device=t.device)
    out[:, : t.size(1)] = t
    return out


def _gemm_rowcol(a: Tensor, a_scale: Tensor, b_nk: Tensor, b_scale: Tensor, out: Tensor) -> None:
    """out[M,N] = (a . b_nk^T) * a_scale * b_scale on the ti kernel.  The kernel walks
    K in 128-byte steps; other K (the reference accepts K % 16 == 0) are zero-padded
    here -- zero codes add exact zeros, so the result is unchanged.  A tiled ``b_nk``
    (``tile_weight_fp8``) runs ``ti_fp8_gemm_rowcol_tiled``."""
    if is_tiled_weight(b_nk):
        m, k = a.shape
        n = b_nk.size(0) * 128
        ws, ws_bytes = _ws_args(a.device, m, n, k, 0)
        _lib.call("ti_fp8_gemm_rowcol_tiled", a.data_ptr(), a_scale.data_ptr(), int(a_scale.numel() != 1),
                  b_nk.data_ptr(), b_scale.data_ptr(), int(b_scale.numel() != 1), out.data_ptr(),
                  _lib.dtype_code(out.dtype), m, n, k, ws, ws_bytes, _lib.stream_of(a))
        return
    if a.size(1) % K_ALIGN:
        k_pad = -(-a.size(1) // K_ALIGN) * K_ALIGN
        a, b_nk = _pad_k(a, k_pad), _pad_k(b_nk, k_pad)
    m, k = a.shape
    n = b_nk.size(0)
    ws, ws_bytes = _ws_args(a.device, m, n, k, 0)
    _lib.call("ti_fp8_gemm_rowcol", a.data_ptr(), a_scale.data_ptr(), int(a_scale.numel() != 1),
              b_nk.data_ptr(), b_scale.data_ptr(), int(b_scale.numel() != 1), out.data_ptr(),
              _lib.dtype_code(out.dtype), m, n, k, ws, ws_bytes, _lib.stream_of(a))


def fp8_prefill_linear(
    x: Tensor,
    wq: Tensor,
    weight_scale: Tensor,
    *,
    activation_scale: Tensor | None = None,
    activation_inverse_scale: Tensor | None = None,
) -> Tensor:
    """``x @ weight.t()`` with tensorwise FP8 scales (fp8.py:184-205): dynamic (or
    static) tensorwise activation quant, then the W8A8 GEMM; returns bf16."""
    n, k = weight_nk(wq)
    x2d = x.reshape(-1, k)
    xq, sa = quantize_activation_fp8(x2d, scale=activation_scale,
                                     inverse_scale=activation_inverse_scale)
    out = torch.empty((x2d.size(0), n), dtype=torch.bfloat16, device=x.device)
    _gemm_rowcol(xq, sa.reshape(1).contiguous(), wq.contiguous(),
                 weight_scale.to(torch.float32).reshape(1).contiguous(), out)
    return out.reshape(*x.shape[:-1], n)


def fp8_per_token_linear(
    x: Tensor,
    weight_q: Tensor,
    weight_scale: Tensor,
    *,
    out: Tensor | None = None,
    use_fast_accum: bool = False,
) -> Tensor:
    """W8A8 with dynamic per-token and per-channel scales (fp8.py:208-247)."""
    if x.ndim < 2 or (weight_q.ndim != 2 and not is_tiled_weight(weight_q)):
        raise ValueError("FP8 linear expects an activation matrix and [N, K] weight")
    if weight_q.dtype != FP8_E4M3 or weight_q.device != x.device:
        raise ValueError("FP8 weight must use e4m3 on the activation device")
    n, k = weight_nk(weight_q)
    if k != x.size(-1):
        raise ValueError("FP8 activation and weight inner dimensions must match")
    if weight_scale.shape != (1, n) or weight_scale.device != x.device:
        raise ValueError("per-channel FP8 weight scale must have shape [1, N]")
    x_q, x_scale = quantize_activation_fp8_per_token(x)
    return fp8_per_token_linear_quantized(
        x_q.view(*x.shape[:-1], x.size(-1)),
        x_scale,
        weight_q,
        weight_scale,
        out_dtype=x.dtype,
        out=out,
        use_fast_accum=use_fast_accum,
    )


def fp8_per_token_linear_quantized(
    x_q: Tensor,
    x_scale: Tensor,
    weight_q: Tensor,
    weight_scale: Tensor,
    *,
    out_dtype: torch.dtype,
    out: Tensor | None = None,
    use_fast_accum: bool = False,
) -> Tensor:
    """W8A8 from an already per-token-quantized activation (fp8.py:250-327).
    ``use_fast_accum`` is accepted for signature parity; the kernel always
    accumulates in fp32 (there is no reduced-precision accumulation mode)."""
    if x_q.ndim < 2 or x_q.dtype != FP8_E4M3:
        raise ValueError("quantized FP8 activation must be an e4m3 matrix")
    if (weight_q.ndim != 2 and not is_tiled_weight(weight_q)) or weight_q.dtype != FP8_E4M3:
        raise ValueError("FP8 weight must be an e4m3 matrix")
    n, k = weight_nk(weight_q)
    if x_q.device != weight_q.device or x_q.size(-1) != k:
        raise ValueError("FP8 activation and weight must have matching devices and inner dimensions")
    rows = x_q.numel() // x_q.size(-1)
    if x_scale.shape != (rows, 1) or x_scale.device != x_q.device:
        raise ValueError("per-token FP8 activation scale must have shape [rows, 1]")
    if weight_scale.shape != (1, n) or weight_scale.device != x_q.device:
        raise ValueError("per-channel FP8 weight scale must have shape [1, N]")
    if out_dtype not in _OUT_DTYPES:
        raise ValueError("FP8 linear output dtype must be bf16 or fp16")
    _lib.require_device(x_q)
    expected_shape = (*x_q.shape[:-1], n)
    if out is not None:
        if tuple(out.shape) != expected_shape or out.device != x_q.device or out.dtype != out_dtype:
            raise ValueError("FP8 output buffer must match the projected output")
        if not out.is_contiguous():
            raise ValueError("FP8 output buffer must be contiguous")
        result = out
    else:
        result = torch.empty(expected_shape, dtype=out_dtype, device=x_q.device)
    x_2d = x_q.reshape(rows, x_q.size(-1)).contiguous()
    _gemm_rowcol(x_2d, x_scale.to(torch.float32).contiguous(), weight_q.contiguous(),
                 weight_scale.to(torch.float32).contiguous(), result.view(rows, n))
    return result


def scaled_mm_out(
    out: Tensor,
    a: Tensor,
    b: Tensor,
    a_scales: Tensor,
    b_scales: Tensor,
) -> Tensor | None:
    """``torchinferno_sgl_fp8::scaled_mm_out`` (sgl_fp8_out.py:134-183,
    csrc/sgl_fp8_out.cpp:17-83): ``out = (a @ b) * a_scales * b_scales`` into the
    caller's buffer, with ``b`` the column-major ``weight.t()`` view.  Returns
    ``None`` for inputs outside the supported region (the reference's convention:
    K and N multiples of 16, contiguous row-major ``a``, column-major ``b``); unlike
    the reference's SM90 provider there is no M <= 64 limit."""
    rows = a.size(0) if a.ndim == 2 else 0
    inner = a.size(1) if a.ndim == 2 else 0
    cols = b.size(1) if b.ndim == 2 else 0
    if (
        a.ndim != 2
        or b.ndim != 2
        or out.ndim != 2
        or rows < 1
        or inner % 16 != 0
        or cols % 16 != 0
        or b.size(0) != inner
        or tuple(out.shape) != (rows, cols)
        or a.dtype != FP8_E4M3
        or b.dtype != FP8_E4M3
        or out.dtype not in _OUT_DTYPES
        or a.device != b.device
        or a.device != out.device
        or a.device != a_scales.device
        or a.device != b_scales.device
        or a.device.type != "cuda"
        or a_scales.dtype != torch.float32
        or b_scales.dtype != torch.float32
        or tuple(a_scales.shape) != (rows, 1)
        or tuple(b_scales.shape) != (1, cols)
        or not a.is_contiguous()
        or b.stride() != (1, inner)
        or not out.is_contiguous()
        or not a_scales.is_contiguous()
        or not b_scales.is_contiguous()
        or not _lib.available()
    ):
        return None
    _gemm_rowcol(a, a_scales, b.t(), b_scales, out)
    return out
