"""int4 W4A16 group-128 linear on MI355X -- drop-in for the reference's Marlin module.

Mirrors the public surface of src/torchinferno/kernels/marlin.py:
``load_marlin_ops`` / ``quantize_to_marlin_int4`` / ``make_workspace`` /
``marlin_int4_mm`` / ``marlin_supports_shape`` (marlin.py:36-175), with the
same argument meaning, caller-owned ``out`` contract and ``ValueError`` on a
bad output buffer (marlin.py:155-167).  The GEMM itself is the gfx950 kernel
``ti_w4a16_gemm`` of libti_quant.so.

Differences a caller sees:
* the packed weight is this build's tile-group layout (see
  ``csrc/int4_gemm.hip``), produced from the canonical [K/8, N] int32 layout by
  ``repack_int4`` -- Marlin's permuted bytes are not reproduced;
* ``make_workspace`` takes the problem's K and the largest M it will serve,
  because the split-K workspace scales with them (Marlin's is N-only,
  marlin.py:134-136).
"""
from __future__ import annotations

import torch
from torch import Tensor

from .. import _lib

GROUP_SIZE = 128
MIN_THREAD_N = 64  # N granularity of the GEMM (same constraint as Marlin, marlin.py:174-175)
TILE_K = 128       # K granularity (one quantization group)
ZERO_POINT = 8
_SCALE_DTYPES = (torch.float16, torch.bfloat16)


def load_int4_ops() -> bool:
    """True when libti_quant.so loads (the analogue of load_marlin_ops, marlin.py:36-52)."""
    return _lib.available()


def int4_supports_shape(size_n: int, size_k: int) -> bool:
    return size_n % MIN_THREAD_N == 0 and size_k % TILE_K == 0 and size_n > 0 and size_k > 0


def pack_int4(codes_kn: Tensor) -> Tensor:
    """codes [K, N] in [0, 15] -> canonical int32 [K/8, N] (nibble i of a word = row 8r+i)."""
    if codes_kn.ndim != 2 or codes_kn.size(0) % 8:
        raise ValueError("codes must be [K, N] with K % 8 == 0")
    k, n = codes_kn.shape
    c = codes_kn.to(torch.int64).reshape(k // 8, 8, n)
    shifts = (4 * torch.arange(8, device=codes_kn.device, dtype=torch.int64)).view(1, 8, 1)
    word = (c << shifts).sum(dim=1)
    return torch.where(word >= 2**31, word - 2**32, word).to(torch.int32)


def quantize_int4_rtn(weight_kn: Tensor, group_size: int = GROUP_SIZE,
                      scale_dtype: torch.dtype = torch.bfloat16) -> tuple[Tensor, Tensor]:
    """Symmetric round-to-nearest int4, the quantizer of marlin.py:117-128, producing
    the canonical layout: (qweight int32 [K/8, N], scales [K/G, N] in scale_dtype).

    GPU tensors run the ``ti_int4_quantize_rtn`` kernel (IEEE fp32 division, round
    half to even -- bit-identical to the host formula); host tensors (weight
    preparation off the GPU) run the same formula in torch on the CPU."""
    if weight_kn.ndim != 2:
        raise ValueError("weight must be [K, N]")
    k, n = weight_kn.shape
    if k % group_size:
        raise ValueError("K must be a multiple of group_size")
    if weight_kn.device.type == "cuda":
        if weight_kn.dtype not in _SCALE_DTYPES or scale_dtype not in _SCALE_DTYPES:
            raise ValueError("weight and scale dtypes must be fp16 or bf16")
        wc = weight_kn.contiguous()
        q = torch.empty((k // 8, n), dtype=torch.int32, device=wc.device)
        s = torch.empty((k // group_size, n), dtype=scale_dtype, device=wc.device)
        _lib.call("ti_int4_quantize_rtn", wc.data_ptr(), _lib.dtype_code(wc.dtype), k, n, group_size,
                  _lib.dtype_code(scale_dtype), q.data_ptr(), s.data_ptr(), _lib.stream_of(wc))
        return q, s
    w = weight_kn.to(torch.float16).float()
    g = w.reshape(k // group_size, group_size, n)
    mx = g.amax(dim=1)
    mn = g.amin(dim=1)
    s = torch.maximum((mx / 7.0).abs(), (mn / -8.0).abs()).clamp(min=1e-8)
    q = torch.round(g / s[:, None, :]).clamp(-8, 7).to(torch.int32) + ZERO_POINT
    return pack_int4(q.reshape(k, n)), s.to(scale_dtype)


def repack_int4(qweight: Tensor, scales: Tensor, group_size: int = GROUP_SIZE
                ) -> tuple[Tensor, Tensor]:
    """Canonical (qweight [K/8, N] int32, scales [K/G, N]) -> kernel layout, on the GPU."""
    _lib.require_device(qweight, scales)
    if qweight.dtype != torch.int32 or qweight.ndim != 2:
        raise ValueError("qweight must be int32 [K/8, N]")
    if scales.dtype not in _SCALE_DTYPES:
        raise ValueError("scales must be fp16 or bf16")
    k, n = qweight.size(0) * 8, qweight.size(1)
    if scales.shape != (k // group_size, n):
        raise ValueError(f"scales must be [K/{group_size}, N] = {(k // group_size, n)}")
    qweight, scales = qweight.contiguous(), scales.contiguous()
    packed_w = torch.empty((n // 16, k // group_size, 256), dtype=torch.int32, device=qweight.device)
    packed_s = torch.empty((n // 16, k // group_size, 16), dtype=scales.dtype, device=qweight.device)
    _lib.call("ti_int4_repack", qweight.data_ptr(), scales.data_ptr(), _lib.dtype_code(scales.dtype),
              k, n, group_size, packed_w.data_ptr(), packed_s.data_ptr(), _lib.stream_of(qweight))
    return packed_w, packed_s


def quantize_to_int4(weight_kn: Tensor, group_size: int = GROUP_SIZE,
                     scale_dtype: torch.dtype = torch.bfloat16) -> tuple[Tensor, Tensor]:
    """fp16/bf16 weight [K, N] -> (packed weight, packed scales); the analogue of
    quantize_to_marlin_int4 (marlin.py:108-131).  The scale dtype must match the
    activation dtype later passed to int4_mm."""
    q, s = quantize_int4_rtn(weight_kn, group_size, scale_dtype)
    return repack_int4(q, s, group_size)


def dequantize_int4(packed_w: Tensor, packed_s: Tensor, size_k: int, size_n: int,
                    group_size: int = GROUP_SIZE) -> Tensor:
    """Kernel-layout weight -> fp32 [K, N] = (q - 8) * s, computed on the GPU by the
    GEMM's own unpack path (exact)."""
    _lib.require_device(packed_w, packed_s)
    out = torch.empty((size_k, size_n), dtype=torch.float32, device=packed_w.device)
    _lib.call("ti_int4_dequant", packed_w.data_ptr(), packed_s.data_ptr(),
              _lib.dtype_code(packed_s.dtype), size_k, size_n, group_size, out.data_ptr(),
              _lib.stream_of(packed_w))
    return out


def workspace_bytes(size_m: int, size_n: int, size_k: int, group_size: int = GROUP_SIZE) -> int:
    return int(_lib.lib().ti_w4a16_workspace_bytes(size_m, size_n, size_k, group_size))


def make_workspace(size_n: int, device, *, size_k: int | None = None, max_m: int = 128,
                   group_size: int = GROUP_SIZE) -> Tensor:
    """Zero-filled workspace serving every M in [1, max_m] for an [K, N] weight.
    Kernels leave it zeroed; calls sharing it must be ordered on one stream.

    Called as the reference calls Marlin's (``make_workspace(n, device)``,
    marlin.py:134-136) -- without ``size_k`` -- it returns a minimal buffer, and
    ``int4_mm`` then uses a per-device shared workspace that grows on demand (do a
    first call at the largest M before capturing graphs)."""
    if size_k is None:
        return torch.zeros(4, dtype=torch.int32, device=device)
    need = int(_lib.lib().ti_w4a16_workspace_bytes_max(max_m, size_n, size_k, group_size))
    return torch.zeros(max(4, (need + 3) // 4), dtype=torch.int32, device=device)


_shared_ws: dict[int, Tensor] = {}


def _shared_workspace(device: torch.device, nbytes: int) -> Tensor:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _shared_ws.get(idx)
    if ws is None or ws.numel() * 4 < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("int4 workspace must be sized before graph capture (run the largest M once)")
        ws = torch.zeros((nbytes + 3) // 4, dtype=torch.int32, device=device)
        _shared_ws[idx] = ws
    return ws


def int4_mm(a: Tensor, q_weight: Tensor, scales: Tensor, workspace: Tensor, size_n: int,
            size_k: int, *, out: Tensor | None = None) -> Tensor:
    """a [M, K] @ int4 weight -> [M, N] in a.dtype (marlin_int4_mm, marlin.py:142-171).

    ``a`` must be 2-D contiguous fp16/bf16 and ``scales`` must share its dtype.
    When ``out`` is given it is written in place and returned."""
    m = a.shape[0]
    expected_shape = (m, size_n)
    if out is None:
        out = torch.empty(expected_shape, dtype=a.dtype, device=a.device)
    elif (
        tuple(out.shape) != expected_shape
        or out.dtype != a.dtype
        or out.device != a.device
        or not out.is_contiguous()
    ):
        raise ValueError("int4 output buffer must be contiguous with shape [M, N], matching input dtype/device")
    if a.ndim != 2 or a.shape[1] != size_k or not a.is_contiguous():
        raise ValueError("a must be a contiguous [M, K] matrix")
    if a.dtype not in _SCALE_DTYPES or scales.dtype != a.dtype:
        raise ValueError("a must be fp16/bf16 and scales must match its dtype")
    _lib.require_device(a, q_weight, scales)
    if q_weight.numel() * 8 != size_k * size_n:
        raise ValueError("q_weight does not hold a [size_k, size_n] int4 weight")
    ws_bytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    need = workspace_bytes(m, size_n, size_k)
    if need > ws_bytes:
        workspace = _shared_workspace(a.device, need)
        ws_bytes = workspace.numel() * 4
    _lib.call("ti_w4a16_gemm", a.data_ptr(), _lib.dtype_code(a.dtype), q_weight.data_ptr(),
              scales.data_ptr(), out.data_ptr(), m, size_n, size_k, GROUP_SIZE,
              _lib.ptr(workspace), ws_bytes, _lib.stream_of(a))
    return out


# Names of the reference module, so callers of marlin.py can switch by import.
load_marlin_ops = load_int4_ops
marlin_supports_shape = int4_supports_shape
quantize_to_marlin_int4 = quantize_to_int4
marlin_int4_mm = int4_mm
