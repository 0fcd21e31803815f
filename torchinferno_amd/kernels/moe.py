"""Routed MoE on MI355X -- drop-in for the reference's grouped expert path
(src/torchinferno/kernels/deepseek_v4_marlin.py: ``prepare_mxfp4_experts``
:194-264, ``fused_mxfp4_moe`` :311-411), for DeepSeek-V3-style FP8 experts
(128x128 block scales: ``prepare_fp8_experts`` / ``fused_fp8_moe``) and for DSv4
MXFP4 experts (e2m1 weights, E8M0 scale per 32: ``prepare_mxfp4_experts`` /
``fused_mxfp4_moe``, same names and arguments as the reference).  Both run 1x128
FP8 activations through gfx950 block-scaled MFMAs; for MXFP4 that is the
arithmetic of the reference's TileLang expert path (act_quant + fp4_gemm), not
of its bf16-activation Marlin kernel.

``route_topk`` is the softmax gate (DSv4 ``Gate.forward``,
src/torchinferno/models/deepseek_v4/tensor_parallel.py:760-780; V3.2
``DeepSeekMoEGate.forward``, models/deepseek_v32/model.py:692-722 without group
limits).  ``fused_fp8_moe`` computes, for every token, the sum over its routed
experts of ``w2(w * silu(w1 x) * (w3 x))`` -- the per-expert loop of
``MoE.forward`` (tensor_parallel.py:882-914) -- as one stream-ordered sequence of
gfx950 kernels (``ti_fp8_moe``): no host synchronisation, deterministic output.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass

import torch
from torch import Tensor

from .. import _lib
from .block_fp8 import E8M0, FP4, _pow2_enabled, e8m0_bytes, fp4_scale_stepmajor
from .fp8 import FP8_E4M3

_ws_lock = threading.Lock()
_workspaces: dict[int, Tensor] = {}


@dataclass(frozen=True)
class PreparedFp8Experts:
    """One GPU's experts in the kernel layout: ``w13 = [w1; w3]`` per expert."""

    w13: Tensor        # e4m3 [E, 2I, H]
    w13_scale: Tensor  # fp32 [E, 2I/128, H/128]
    w2: Tensor         # e4m3 [E, H, I]
    w2_scale: Tensor   # fp32 [E, H/128, I/128]
    expert_map: Tensor  # int32 [global experts] -> local index or -1
    global_num_experts: int
    hidden_size: int
    intermediate_size: int
    scales_pow2: bool = False  # every block scale a power of two (E8M0 values)


def _all_pow2(*scales: Tensor) -> bool:
    """True when every scale is a power of two in the E8M0 range (2^-127..2^127):
    E8M0 storage always, fp32 when each value is (one pass at weight preparation)."""
    for s in scales:
        if s.dtype == E8M0:
            continue
        f = s.float()
        m, e = torch.frexp(f)
        if not bool(((m == 0.5) & (f >= 2.0 ** -127)).all()):
            return False
    return True


def prepare_fp8_experts(w1: Tensor, w3: Tensor, w2: Tensor, w1_scale: Tensor, w3_scale: Tensor,
                        w2_scale: Tensor, *, expert_start: int = 0,
                        global_num_experts: int | None = None) -> PreparedFp8Experts:
    """Stack one GPU's block-FP8 experts (the analogue of prepare_mxfp4_experts,
    deepseek_v4_marlin.py:194-264).  ``w1``/``w3`` e4m3 ``[E, I, H]``, ``w2`` ``[E, H, I]``,
    scales per 128x128 block, fp32 or ``float8_e8m0fnu``.  Weight preparation: run
    once, before capture."""
    if w1.ndim != 3 or w3.ndim != 3 or w2.ndim != 3:
        raise ValueError("expert weights must be stacked [experts, output, K]")
    if tuple(w1.shape) != tuple(w3.shape):
        raise ValueError("w1 and w3 expert shapes must match")
    e, inter, hidden = w1.shape
    if tuple(w2.shape) != (e, hidden, inter):
        raise ValueError("w2 expert shape does not match w1/w3")
    if any(t.dtype != FP8_E4M3 for t in (w1, w3, w2)):
        raise ValueError("expert weights must be float8_e4m3fn")
    if hidden % 128 or inter % 128:
        raise ValueError("hidden and intermediate sizes must be multiples of 128")
    global_num_experts = e if global_num_experts is None else global_num_experts
    expert_map = torch.full((global_num_experts,), -1, dtype=torch.int32, device=w1.device)
    expert_map[expert_start:expert_start + e] = torch.arange(e, dtype=torch.int32, device=w1.device)
    return PreparedFp8Experts(
        w13=torch.cat((w1, w3), dim=1).contiguous(),
        w13_scale=torch.cat((w1_scale.float(), w3_scale.float()), dim=1).contiguous(),
        w2=w2.contiguous(),
        w2_scale=w2_scale.float().contiguous(),
        expert_map=expert_map,
        global_num_experts=global_num_experts,
        hidden_size=hidden,
        intermediate_size=inter,
        scales_pow2=_all_pow2(w1_scale, w3_scale, w2_scale),
    )


@dataclass(frozen=True)
class PreparedMxfp4Experts:
    """One GPU's MXFP4 experts in the kernel layout: ``w13 = [w1; w3]`` per expert."""

    w13: Tensor        # e2m1 x2 (uint8) [E, 2I, H/2]
    w13_scale: Tensor  # E8M0 bytes, step-major [E, H/128, 2I, 4]
    w2: Tensor         # e2m1 x2 (uint8) [E, H, I/2]
    w2_scale: Tensor   # E8M0 bytes, step-major [E, I/128, H, 4]
    expert_map: Tensor  # int32 [global experts] -> local index or -1
    global_num_experts: int
    hidden_size: int
    intermediate_size: int


def prepare_mxfp4_experts(w1: Tensor, w3: Tensor, w2: Tensor, w1_scale: Tensor, w3_scale: Tensor,
                          w2_scale: Tensor, *, expert_start: int = 0,
                          global_num_experts: int | None = None) -> PreparedMxfp4Experts:
    """Stack one GPU's native MXFP4 experts (deepseek_v4_marlin.py:194-264, same
    arguments): ``w1``/``w3`` ``[E, I, H/2]`` and ``w2`` ``[E, H, I/2]``
    ``float4_e2m1fn_x2``; scales one E8M0 per 32 K (``[E, I, H/32]``,
    ``[E, H, I/32]``).  The weights keep the checkpoint layout; the scales are
    rearranged once to the step-major layout the kernels read contiguously."""
    if w1.ndim != 3 or w3.ndim != 3 or w2.ndim != 3:
        raise ValueError("expert weights must be stacked [experts, output, packed-K]")
    if tuple(w1.shape) != tuple(w3.shape):
        raise ValueError("w1 and w3 expert shapes must match")
    e, inter, half_h = w1.shape
    hidden = half_h * 2
    if tuple(w2.shape) != (e, hidden, inter // 2):
        raise ValueError("w2 expert shape does not match w1/w3")
    if any(t.dtype not in (FP4, torch.uint8) for t in (w1, w3, w2)):
        raise ValueError("expert weights must be float4_e2m1fn_x2")
    if hidden % 128 or inter % 128:
        raise ValueError("hidden and intermediate sizes must be multiples of 128")
    s1, s3, s2 = (e8m0_bytes(t) for t in (w1_scale, w3_scale, w2_scale))
    if tuple(s1.shape) != (e, inter, hidden // 32) or tuple(s3.shape) != tuple(s1.shape) \
            or tuple(s2.shape) != (e, hidden, inter // 32):
        raise ValueError("MXFP4 scales must be one E8M0 per 32 K of each weight row")
    global_num_experts = e if global_num_experts is None else global_num_experts
    expert_map = torch.full((global_num_experts,), -1, dtype=torch.int32, device=w1.device)
    expert_map[expert_start:expert_start + e] = torch.arange(e, dtype=torch.int32, device=w1.device)
    u8 = lambda t: t.contiguous().view(torch.uint8)  # noqa: E731
    return PreparedMxfp4Experts(
        w13=torch.cat((u8(w1), u8(w3)), dim=1).contiguous(),
        w13_scale=fp4_scale_stepmajor(torch.cat((s1, s3), dim=1)),
        w2=u8(w2),
        w2_scale=fp4_scale_stepmajor(s2),
        expert_map=expert_map,
        global_num_experts=global_num_experts,
        hidden_size=hidden,
        intermediate_size=inter,
    )


def route_topk(logits: Tensor, k: int, *, renormalize: bool = True,
               route_scale: float = 1.0) -> tuple[Tensor, Tensor]:
    """Softmax top-k router: (weights fp32 [T,k], ids int32 [T,k]), descending."""
    _lib.require_device(logits)
    if logits.ndim != 2:
        raise ValueError("router logits must be [tokens, experts]")
    z = logits.float().contiguous()
    t, e = z.shape
    w = torch.empty((t, k), dtype=torch.float32, device=z.device)
    ids = torch.empty((t, k), dtype=torch.int32, device=z.device)
    _lib.call("ti_moe_route_topk", z.data_ptr(), t, e, k, int(renormalize), float(route_scale),
              w.data_ptr(), ids.data_ptr(), _lib.stream_of(z))
    return w, ids


def _workspace(device: torch.device, nbytes: int) -> Tensor:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        ws = _workspaces.get(idx)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
            _workspaces[idx] = ws
        return ws


def _round_scale(scale_fmt: str | None, weight_scales_pow2: bool) -> int:
    """act_quant's ``scale_fmt`` (deepseek_v4_tilelang_definitions.py:255-331): any
    format rounds the 1x128 activation scales up to powers of two (1); with
    power-of-two weight scales too, the kernels apply all of them inside the
    MFMA (2)."""
    if scale_fmt is None:
        return 0
    return 2 if weight_scales_pow2 and _pow2_enabled() else 1


def _routed(entry: str, hidden_states: Tensor, topk_weights: Tensor, topk_ids: Tensor, experts,
            clamp_limit: float, scale_fmt: str | None) -> Tensor:
    if hidden_states.ndim != 2 or not hidden_states.is_contiguous():
        raise ValueError("hidden_states must be a contiguous matrix")
    if hidden_states.dtype != torch.bfloat16:
        raise ValueError("hidden_states must be bf16")
    tokens, hidden = hidden_states.shape
    if hidden != experts.hidden_size:
        raise ValueError("hidden size does not match prepared experts")
    if topk_ids.shape != topk_weights.shape or topk_ids.ndim != 2 or topk_ids.size(0) != tokens:
        raise ValueError("topk ids/weights must be [tokens, k]")
    _lib.require_device(hidden_states, topk_weights, topk_ids)
    k = topk_ids.size(1)
    local_ids = experts.expert_map[topk_ids.long()].to(torch.int32).contiguous()
    weights = topk_weights.float().contiguous()
    e_local = experts.w13.size(0)
    inter = experts.intermediate_size
    out = torch.empty((tokens, hidden), dtype=torch.bfloat16, device=hidden_states.device)
    if tokens == 0:
        return out
    need = int(_lib.lib().ti_fp8_moe_workspace_bytes(tokens, k, e_local, hidden, inter))
    ws = _workspace(hidden_states.device, need)
    base = ws.data_ptr()
    aligned = (base + 255) & ~255
    layout = (1,) if entry == "ti_fp4_moe" else ()  # MXFP4 scales are prepared step-major
    _lib.call(entry, hidden_states.data_ptr(), weights.data_ptr(), local_ids.data_ptr(), tokens, k,
              experts.w13.data_ptr(), experts.w13_scale.data_ptr(), experts.w2.data_ptr(),
              experts.w2_scale.data_ptr(), *layout, e_local, hidden, inter, float(clamp_limit),
              _round_scale(scale_fmt, entry == "ti_fp4_moe" or experts.scales_pow2), out.data_ptr(),
              aligned, ws.numel() - (aligned - base), _lib.stream_of(hidden_states))
    return out


def fused_fp8_moe(hidden_states: Tensor, topk_weights: Tensor, topk_ids: Tensor,
                  experts: PreparedFp8Experts, *, clamp_limit: float = 0.0,
                  scale_fmt: str | None = None) -> Tensor:
    """Grouped routed experts for one GPU (signature of fused_mxfp4_moe,
    deepseek_v4_marlin.py:311-318).  ``topk_ids`` are global expert ids; routes to
    experts this GPU does not hold contribute nothing.  ``scale_fmt`` is the
    model's act_quant scale format (DSv4 sets "ue8m0": power-of-two activation
    scales, tensor_parallel.py:195-207,1199-1211).  Returns bf16 [T, H]."""
    return _routed("ti_fp8_moe", hidden_states, topk_weights, topk_ids, experts, clamp_limit, scale_fmt)


def fused_mxfp4_moe(hidden_states: Tensor, topk_weights: Tensor, topk_ids: Tensor,
                    experts: PreparedMxfp4Experts, *, clamp_limit: float = 0.0,
                    scale_fmt: str | None = None) -> Tensor:
    """MXFP4 routed experts (deepseek_v4_marlin.py:311-411, same arguments and
    [T, H] bf16 result); see ``fused_fp8_moe`` for routing and ``scale_fmt``."""
    return _routed("ti_fp4_moe", hidden_states, topk_weights, topk_ids, experts, clamp_limit, scale_fmt)


def moe_forward(hidden_states: Tensor, router_logits: Tensor, experts: PreparedFp8Experts, k: int, *,
                renormalize: bool = True, route_scale: float = 1.0, clamp_limit: float = 0.0,
                scale_fmt: str | None = None) -> Tensor:
    """Router + routed experts: the routed part of DSv4 MoE.forward (without the
    shared expert and the cross-GPU all-reduce)."""
    w, ids = route_topk(router_logits, k, renormalize=renormalize, route_scale=route_scale)
    return fused_fp8_moe(hidden_states, w, ids, experts, clamp_limit=clamp_limit, scale_fmt=scale_fmt)
