"""Model-dispatch hooks: plug this package's kernels into the reference's Llama3
and DeepSeek model paths as a drop-in.

The reference selects its quantized projections per layer, M-gated, in methods
of ``_Llama3TensorParallelLayer`` (src/torchinferno/models/llama3/
tensor_parallel.py:2732-2983) and in DSv4's module-level ``linear`` and
``MoE.forward`` (src/torchinferno/models/deepseek_v4/tensor_parallel.py:195-207,
882-914).  This module restates those methods -- the same environment knobs,
gates, lazily-filled per-key caches on the layer (``_marlin_{key}_q`` ...) and
the ``None``-means-fall-back-to-bf16 contract with a sticky ``_{...}_failed``
flag -- with the kernel calls routed to ``torchinferno_amd.kernels``.

* :func:`patch_llama3_layer_class` installs ``_marlin_proj``, ``_fp8_proj``,
  ``_fp8_per_token_proj``, ``_prepare_fp8_per_token_weight`` and
  ``_fp8_decode_shape_enabled`` on the layer class (returns an undo callable);
* :func:`patch_deepseek_v4_module` replaces the module's ``linear`` (block-FP8
  weights carry ``.scale``, as the reference's ``Linear`` attaches it) and gives
  ``MoE`` classes a ``prepare_fused_experts``/``forward`` pair backed by the routed
  FP8 MoE kernels.

Nothing here imports the reference: callers pass the class / module objects.
"""
from __future__ import annotations

import os
import sys
import types
import warnings
from typing import Callable

import torch
from torch import Tensor

_FALSE = {"", "0", "false", "no", "off"}


def _flag(name: str, default: bool) -> bool:
    raw = os.environ.get(name)
    return default if raw is None else raw.strip().lower() not in _FALSE


def _int(name: str, default: int, minimum: int | None = None) -> int:
    raw = os.environ.get(name)
    v = default if raw is None else int(raw)
    return max(minimum, v) if minimum is not None else v


def _float(name: str, default: float, minimum: float | None = None) -> float:
    raw = os.environ.get(name)
    v = default if raw is None else float(raw)
    return max(minimum, v) if minimum is not None else v


def _capturing(device: torch.device) -> bool:
    return device.type == "cuda" and torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def _optional_failure(key: str, exc: BaseException) -> None:
    if _flag("TORCHINFERNO_OPTIONAL_WARNINGS", False):
        warnings.warn(f"torchinferno_amd optional path disabled for {key}: {exc}", stacklevel=3)


# --------------------------------------------------------------------------- Llama3


def marlin_proj(self, hidden: Tensor, key: str, weight: Tensor, *, out: Tensor | None = None) -> Tensor | None:
    """int4 W4A16 column-parallel projection, M-gated (tensor_parallel.py:2732-2794).
    Returns ``[..., N]`` or ``None`` (the caller falls back to bf16)."""
    from .kernels import int4 as _int4

    if not _flag("TORCHINFERNO_MARLIN_INT4_DECODE", True):
        return None
    if not bool(getattr(self, "_runtime_marlin_int4_decode_enabled", True)):
        return None
    if not hidden.is_cuda:
        return None
    if hidden.numel() // hidden.size(-1) > _int("TORCHINFERNO_MARLIN_INT4_MAX_M", 128, minimum=1):
        return None
    if getattr(self, f"_marlin_{key}_failed", False):
        return None
    if getattr(self, f"_marlin_{key}_q", None) is None:
        try:
            n, k = int(weight.size(0)), int(weight.size(1))
            if not _int4.load_int4_ops() or not _int4.int4_supports_shape(n, k):
                setattr(self, f"_marlin_{key}_failed", True)
                return None
            q, s = _int4.quantize_to_int4(weight.t().contiguous(), 128, scale_dtype=hidden.dtype)
            setattr(self, f"_marlin_{key}_q", q)
            setattr(self, f"_marlin_{key}_s", s)
            setattr(self, f"_marlin_{key}_ws", _int4.make_workspace(n, weight.device, size_k=k, max_m=128))
            setattr(self, f"_marlin_{key}_n", n)
            setattr(self, f"_marlin_{key}_k", k)
        except Exception as exc:  # noqa: BLE001 -- optional path, as in the reference
            _optional_failure(f"llama3_tensor_parallel.marlin_{key}", exc)
            setattr(self, f"_marlin_{key}_failed", True)
            return None
    n = getattr(self, f"_marlin_{key}_n")
    k = getattr(self, f"_marlin_{key}_k")
    x2d = hidden.reshape(-1, k).contiguous()
    out_2d = out.reshape(-1, n) if out is not None else None
    res = _int4.int4_mm(x2d, getattr(self, f"_marlin_{key}_q"), getattr(self, f"_marlin_{key}_s"),
                        getattr(self, f"_marlin_{key}_ws"), n, k, out=out_2d)
    return res.reshape(*hidden.shape[:-1], n)


def fp8_decode_shape_enabled(hidden: Tensor) -> bool:
    """tensor_parallel.py:3118-3126."""
    if not _flag("TORCHINFERNO_FP8_DECODE", False):
        return False
    if hidden.ndim != 3 or hidden.size(1) != 1:
        return False
    rows = hidden.numel() // hidden.size(-1)
    return rows <= _int("TORCHINFERNO_FP8_DECODE_MAX_M", 128, minimum=1)


def fp8_proj(self, hidden: Tensor, key: str, weight: Tensor, *, out: Tensor | None = None) -> Tensor | None:
    """FP8 W8A8 projection, M-gated prefill / opt-in decode (tensor_parallel.py:2796-2896)."""
    from .kernels import fp8 as _fp8

    if key == "gu" and not _flag("TORCHINFERNO_FP8_GATE_UP", True):
        return None
    if key == "down" and not _flag("TORCHINFERNO_FP8_DOWN", True):
        return None
    decode_enabled = self._fp8_decode_shape_enabled(hidden)
    env_configured = "TORCHINFERNO_FP8_PREFILL" in os.environ
    env_enabled = _flag("TORCHINFERNO_FP8_PREFILL", False) if env_configured else False
    runtime_enabled = bool(getattr(self, "_runtime_fp8_prefill_enabled", False))
    if env_configured and not env_enabled:
        runtime_enabled = False
    if not decode_enabled and not env_enabled and not runtime_enabled:
        return None
    if not hidden.is_cuda:
        return None
    m = hidden.numel() // hidden.size(-1)
    if not decode_enabled:
        if "TORCHINFERNO_FP8_PREFILL_MIN_M" in os.environ:
            min_m = _int("TORCHINFERNO_FP8_PREFILL_MIN_M", 256, minimum=1)
        elif runtime_enabled and not env_enabled:
            min_m = int(getattr(self, "_runtime_fp8_prefill_min_m", 2048))
        else:
            min_m = 256
        if m <= max(1, min_m):
            return None
    if _flag("TORCHINFERNO_FP8_PER_TOKEN_SCALE", False):
        return self._fp8_per_token_proj(hidden, key, weight, out=out)
    if out is not None:
        return None
    if getattr(self, f"_fp8_{key}_failed", False):
        return None
    if getattr(self, f"_fp8_{key}_wq", None) is None:
        if _capturing(hidden.device):
            return None
        try:
            if not _fp8.fp8_available():
                setattr(self, f"_fp8_{key}_failed", True)
                return None
            wq, sb = _fp8.quantize_weight_fp8(weight)
            wq = _fp8.maybe_tile_weight_fp8(wq)  # the GEMM's tiled weight layout
            setattr(self, f"_fp8_{key}_wq", wq)
            setattr(self, f"_fp8_{key}_sb", sb)
        except Exception as exc:  # noqa: BLE001
            _optional_failure(f"llama3_tensor_parallel.fp8_{key}", exc)
            setattr(self, f"_fp8_{key}_failed", True)
            return None
    activation_scale = None
    activation_inverse_scale = None
    if decode_enabled or _flag("TORCHINFERNO_FP8_PREFILL_STATIC_ACTIVATION_SCALE", False):
        mode = "decode" if decode_enabled else "prefill"
        scale_name = f"_fp8_{key}_{mode}_activation_scale"
        inverse_name = f"_fp8_{key}_{mode}_activation_inverse_scale"
        activation_scale = getattr(self, scale_name, None)
        activation_inverse_scale = getattr(self, inverse_name, None)
        if activation_scale is None:
            if _capturing(hidden.device):
                return None
            margin = _float("TORCHINFERNO_FP8_DECODE_SCALE_MARGIN" if decode_enabled
                            else "TORCHINFERNO_FP8_PREFILL_STATIC_SCALE_MARGIN", 4.0, minimum=1.0)
            activation_scale = (hidden.abs().amax() / float(_fp8.FP8_E4M3_MAX)).clamp(min=1e-6).to(
                torch.float32) * margin
            activation_inverse_scale = activation_scale.reciprocal()
            setattr(self, scale_name, activation_scale)
            setattr(self, inverse_name, activation_inverse_scale)
    return _fp8.fp8_prefill_linear(hidden, getattr(self, f"_fp8_{key}_wq"), getattr(self, f"_fp8_{key}_sb"),
                                   activation_scale=activation_scale,
                                   activation_inverse_scale=activation_inverse_scale)


def prepare_fp8_per_token_weight(self, key: str, weight: Tensor) -> tuple[Tensor, Tensor] | None:
    """tensor_parallel.py:2958-2983."""
    from .kernels import fp8 as _fp8

    if getattr(self, f"_fp8_per_token_{key}_failed", False):
        return None
    wq = getattr(self, f"_fp8_per_token_{key}_wq", None)
    ws = getattr(self, f"_fp8_per_token_{key}_ws", None)
    if wq is not None and ws is not None:
        return wq, ws
    if _capturing(weight.device):
        return None
    try:
        wq, ws = _fp8.quantize_weight_fp8_per_channel(weight)
        wq = _fp8.maybe_tile_weight_fp8(wq)  # the GEMM's tiled weight layout
        setattr(self, f"_fp8_per_token_{key}_wq", wq)
        setattr(self, f"_fp8_per_token_{key}_ws", ws)
        return wq, ws
    except Exception as exc:  # noqa: BLE001
        _optional_failure(f"llama3_tensor_parallel.fp8_per_token_{key}", exc)
        setattr(self, f"_fp8_per_token_{key}_failed", True)
        return None


def fp8_per_token_proj(self, hidden, key: str, weight: Tensor, *, out: Tensor | None = None) -> Tensor | None:
    """Per-token x per-channel FP8 projection (tensor_parallel.py:2898-2956).  ``hidden``
    may be a pre-quantized activation object with ``.values`` / ``.scales``
    (the reference's ``_FP8PerTokenActivation``)."""
    from .kernels import fp8 as _fp8

    prepared = self._prepare_fp8_per_token_weight(key, weight)
    if prepared is None:
        return None
    wq, ws = prepared
    try:
        if hasattr(hidden, "values") and hasattr(hidden, "scales") and not isinstance(hidden, Tensor):
            return _fp8.fp8_per_token_linear_quantized(hidden.values, hidden.scales, wq, ws,
                                                       out_dtype=weight.dtype, out=out)
        return _fp8.fp8_per_token_linear(hidden, wq, ws, out=out)
    except Exception as exc:  # noqa: BLE001
        _optional_failure(f"llama3_tensor_parallel.fp8_per_token_{key}", exc)
        setattr(self, f"_fp8_per_token_{key}_failed", True)
        return None


_LLAMA3_METHODS = {
    "_marlin_proj": marlin_proj,
    "_fp8_proj": fp8_proj,
    "_fp8_per_token_proj": fp8_per_token_proj,
    "_prepare_fp8_per_token_weight": prepare_fp8_per_token_weight,
    "_fp8_decode_shape_enabled": staticmethod(fp8_decode_shape_enabled),
}


def patch_llama3_layer_class(cls: type) -> Callable[[], None]:
    """Install the MI355X projections on a layer class (the reference's
    ``_Llama3TensorParallelLayer``); returns a callable that restores the originals."""
    saved = {name: cls.__dict__.get(name) for name in _LLAMA3_METHODS}
    for name, fn in _LLAMA3_METHODS.items():
        setattr(cls, name, fn)

    def undo() -> None:
        for name, orig in saved.items():
            if orig is None:
                delattr(cls, name)
            else:
                setattr(cls, name, orig)

    return undo


_FUSED_NAMES = ("triton_rms_norm_fp8_per_token", "triton_add_rms_norm_fp8_per_token",
                "triton_swiglu_fp8_per_token")


def patch_fused_producers(module: types.ModuleType) -> Callable[[], None]:
    """Point the fused RMSNorm / add+RMSNorm / SwiGLU -> per-token FP8 producers of
    ``module`` (the reference's ``torchinferno.kernels.triton_ops``, which the
    Llama3 layer imports from at call time, tensor_parallel.py:3073-3187) at this
    package's kernels.  Returns undo."""
    from .kernels import fused

    saved = {n: getattr(module, n, None) for n in _FUSED_NAMES}
    for n in _FUSED_NAMES:
        setattr(module, n, getattr(fused, n))

    def undo() -> None:
        for n, orig in saved.items():
            if orig is None:
                delattr(module, n)
            else:
                setattr(module, n, orig)

    return undo


# --------------------------------------------------------------------------- DeepSeek-V4


def deepseek_linear(x: Tensor, weight: Tensor, bias: Tensor | None = None, *,
                    scale_fmt: str | None = None, scale_dtype: torch.dtype = torch.float32) -> Tensor:
    """DSv4 ``linear`` (tensor_parallel.py:195-207): e4m3 weights (``.scale``
    per 128x128 block) and MXFP4 weights (``float4_e2m1fn_x2``, ``.scale`` one
    E8M0 per 32 K) run ``act_quant(x, 128, scale_fmt, scale_dtype)`` + the
    block-FP8 / FP4 GEMM here; other dtypes keep ``F.linear``.  ``scale_fmt`` and
    ``scale_dtype`` are the model module's globals (set in ``MoE.__init__`` /
    the checkpoint path, tensor_parallel.py:1199-1212,1641);
    ``patch_deepseek_v4_module`` passes them at call time."""
    from .kernels import block_fp8

    assert bias is None
    if weight.dtype in (torch.float8_e4m3fn, torch.float4_e2m1fn_x2):
        return block_fp8.linear(x, weight, weight.scale, scale_fmt, scale_dtype)
    return torch.nn.functional.linear(x, weight)


def _module_scale_format(module: types.ModuleType | None) -> tuple[str | None, torch.dtype]:
    """The reference module's ``scale_fmt`` / ``scale_dtype`` globals as they are now
    (the model sets them after import, tensor_parallel.py:1199-1212)."""
    if module is None:
        return None, torch.float32
    return getattr(module, "scale_fmt", None), getattr(module, "scale_dtype", torch.float32)


def prepare_fused_fp8_experts(moe_module) -> bool:
    """Stack a DSv4 ``MoE``'s local block-FP8 or MXFP4 experts into the grouped
    layout (the role of ``MoE.prepare_fused_experts``, tensor_parallel.py:826-858)."""
    from .kernels import moe as _moe

    if getattr(moe_module, "_ti_fused_experts", None) is not None:
        return True
    start, end = moe_module.experts_start_idx, moe_module.experts_end_idx
    local = [moe_module.experts[i] for i in range(start, end)]
    if not local or local[0] is None:
        return False
    dtype = local[0].w1.weight.dtype
    if dtype not in (torch.float8_e4m3fn, torch.float4_e2m1fn_x2):
        return False
    st = torch.stack
    prepare = _moe.prepare_fp8_experts if dtype == torch.float8_e4m3fn else _moe.prepare_mxfp4_experts
    moe_module._ti_fused_experts = prepare(
        st([e.w1.weight for e in local]), st([e.w3.weight for e in local]), st([e.w2.weight for e in local]),
        st([e.w1.scale for e in local]), st([e.w3.scale for e in local]), st([e.w2.scale for e in local]),
        expert_start=start, global_num_experts=moe_module.n_routed_experts)
    return True


def moe_forward(self, x: Tensor, input_ids: Tensor) -> Tensor:
    """DSv4 ``MoE.forward`` (tensor_parallel.py:882-914) with the routed experts on
    the fused FP8 kernels when prepared; the gate, the shared expert and the
    cross-GPU reduction (``self._ti_all_reduce`` when set) are the model's own."""
    from .kernels import moe as _moe

    shape = x.size()
    x = x.view(-1, self.dim)
    weights, indices = self.gate(x, input_ids.flatten())
    fused = getattr(self, "_ti_fused_experts", None)
    if fused is not None:
        run = _moe.fused_mxfp4_moe if isinstance(fused, _moe.PreparedMxfp4Experts) else _moe.fused_fp8_moe
        scale_fmt, _ = _module_scale_format(sys.modules.get(type(self).__module__))
        y = run(x.contiguous(), weights.float().contiguous(), indices.int().contiguous(), fused,
                clamp_limit=float(getattr(self.shared_experts, "swiglu_limit", 0.0) or 0.0),
                scale_fmt=scale_fmt)
        y = y.float()
    else:
        y = torch.zeros_like(x, dtype=torch.float32)
        counts = torch.bincount(indices.flatten().long(), minlength=self.n_routed_experts).tolist()
        for i in range(self.experts_start_idx, self.experts_end_idx):
            if counts[i] == 0:
                continue
            idx, top = torch.where(indices == i)
            y[idx] += self.experts[i](x[idx], weights[idx, top, None])
    reduce = getattr(self, "_ti_all_reduce", None)
    if reduce is not None:
        reduce(y)
    y += self.shared_experts(x)
    return y.type_as(x).view(shape)


def patch_deepseek_v4_module(module: types.ModuleType, moe_cls: type | None = None) -> Callable[[], None]:
    """Replace ``module.linear`` (which ``Linear.forward`` looks up at call time) and,
    if given, ``moe_cls.forward`` / ``moe_cls.prepare_fused_experts``.  Returns undo."""
    saved_linear = module.linear

    def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
        scale_fmt, scale_dtype = _module_scale_format(module)
        return deepseek_linear(x, weight, bias, scale_fmt=scale_fmt, scale_dtype=scale_dtype)

    module.linear = linear
    saved_moe = {}
    if moe_cls is not None:
        saved_moe = {n: moe_cls.__dict__.get(n) for n in ("forward", "prepare_fused_experts")}
        moe_cls.forward = moe_forward
        moe_cls.prepare_fused_experts = prepare_fused_fp8_experts

    def undo() -> None:
        module.linear = saved_linear
        for n, orig in saved_moe.items():
            if orig is None:
                delattr(moe_cls, n)
            else:
                setattr(moe_cls, n, orig)

    return undo
