"""ctypes binding of libti_quant.so (the C ABI declared in include/ti_quant.h).

The library is required: there is no CPU or PyTorch fallback for any kernel.
If it is missing, :func:`lib` raises with the command that builds it.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("TI_ROCM_QUANT_LIB", _PKG / "libti_quant.so"))

TI_OK, TI_ERR_INVALID, TI_ERR_UNSUPPORTED, TI_ERR_WORKSPACE, TI_ERR_HIP = range(5)
TI_DTYPE_F16, TI_DTYPE_BF16, TI_DTYPE_F32, TI_DTYPE_E4M3 = 1, 2, 3, 4

_DTYPE_CODES = {
    torch.float16: TI_DTYPE_F16,
    torch.bfloat16: TI_DTYPE_BF16,
    torch.float32: TI_DTYPE_F32,
    torch.float8_e4m3fn: TI_DTYPE_E4M3,
}

_vp, _i, _sz, _u64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_uint64
_f = ctypes.c_float

# name -> (restype, argtypes).  Every exported entry point of include/ti_quant.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ti_version": (_i, []),
    "ti_last_error": (ctypes.c_char_p, []),
    "ti_int4_packed_weight_bytes": (_sz, [_i, _i]),
    "ti_int4_packed_scale_bytes": (_sz, [_i, _i, _i]),
    "ti_int4_repack": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "ti_int4_dequant": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _vp]),
    "ti_int4_quantize_rtn": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp]),
    "ti_w4a16_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "ti_w4a16_workspace_bytes_max": (_sz, [_i, _i, _i, _i]),
    "ti_w4a16_gemm": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ti_w4a16_gemm_noalloc": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "ti_w4a16_noalloc_scratch_bytes": (_sz, []),
    "ti_w4a16_zero_point_add": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _vp]),
    "ti_w4a16_plan_name": (_i, [_i, _i, _i, _i, ctypes.c_char_p, _sz]),
    "ti_fp8_quant_per_token": (_i, [_vp, _i, _i, _i, _f, _vp, _vp, _vp]),
    "ti_fp8_quant_weight_per_channel": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "ti_fp8_quant_block": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp]),
    "ti_fp8_e4m3_selfcheck": (_i, [_vp, _vp]),
    "ti_bf16_round_selfcheck": (_i, [_vp, _vp]),
    "ti_fp8_quant_tensor": (_i, [_vp, _i, ctypes.c_long, _vp, _vp, _vp]),
    "ti_fp8_rmsnorm_quant_per_token": (_i, [_vp, _vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp, _vp]),
    "ti_fp8_swiglu_quant_per_token": (_i, [_vp, ctypes.c_long, _vp, ctypes.c_long, _i, _i, _i, _vp, _vp, _vp]),
    "ti_fp8_gemm_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "ti_fp8_gemm_workspace_bytes_max": (_sz, [_i, _i, _i, _i]),
    "ti_fp8_gemm_rowcol": (_i, [_vp, _vp, _i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ti_fp8_gemm_rowcol_tiled": (_i, [_vp, _vp, _i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ti_fp8_tile_weight": (_i, [_vp, _i, _i, _vp, _vp]),
    "ti_fp8_gemm_block": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ti_fp4_gemm": (_i, [_vp, _vp, _i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ti_fp8_gemm_block_pow2": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ti_fp4_gemm_pow2": (_i, [_vp, _vp, _i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, _sz, _vp]),
    "ti_fp4_scale_stepmajor": (_i, [_vp, _i, _i, _vp, _vp]),
    "ti_moe_route_topk": (_i, [_vp, _i, _i, _i, _i, _f, _vp, _vp, _vp]),
    "ti_fp8_moe_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "ti_fp8_moe": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _i, _vp, _vp, _sz, _vp]),
    "ti_fp4_moe": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _vp, _vp, _sz, _vp]),
}


class TiError(RuntimeError):
    """A libti_quant call returned a non-zero status."""

    def __init__(self, name: str, status: int, message: str):
        super().__init__(f"{name} failed (status {status}): {message}")
        self.status = status


class TiUnsupported(TiError):
    """Shape outside a kernel's supported region (TI_ERR_UNSUPPORTED)."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m torchinferno_amd.build_lib` "
                    "(or __graft_entry__.build()) first")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def available() -> bool:
    try:
        lib()
        return True
    except (OSError, RuntimeError):
        return False


def call(name: str, *args) -> None:
    """Call an int-status entry point and raise on failure."""
    status = getattr(lib(), name)(*args)
    if status != TI_OK:
        msg = lib().ti_last_error().decode(errors="replace")
        cls = TiUnsupported if status == TI_ERR_UNSUPPORTED else TiError
        raise cls(name, status, msg)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """Handle of the current HIP stream of t's device (the stream ops enqueue on)."""
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("torchinferno_amd kernels need tensors on a ROCm GPU device")
