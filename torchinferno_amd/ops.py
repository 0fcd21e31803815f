"""``torch.library`` custom ops of the quantized-linear path (namespace
``torchinferno_amd``), following the reference's custom-op pattern
(``torch.library.custom_op(..., mutates_args=...)`` + ``register_fake``,
src/torchinferno/kernels/ops.py:63-85) so the ops trace through ``make_fx`` /
``torch.compile`` with shape-only fake implementations, and so a model can call
them through ``torch.ops.torchinferno_amd.*``.

Ops (each a thin wrapper over ``torchinferno_amd.kernels.*`` and libti_quant.so):

* ``w4a16_mm(a, q_weight, scales, workspace, size_n, size_k) -> Tensor`` and
  ``w4a16_mm_out(out!, ...)`` -- the ``marlin_gemm`` slot (marlin.py:142-171);
* ``fp8_scaled_mm_out(out!, a, b, a_scales, b_scales)`` -- the schema of
  ``torchinferno_sgl_fp8::scaled_mm_out`` (csrc/sgl_fp8_out.cpp:75-83), with
  ``b`` the column-major ``weight.t()``;
* ``fp8_per_token_linear(x, weight_q, weight_scale) -> Tensor`` (fp8.py:208-247);
* ``act_quant(x, block_size, round_scale) -> (Tensor, Tensor)`` and
  ``fp8_block_gemm(a, a_s, b, b_s) -> Tensor`` -- DeepSeek act_quant / fp8_gemm
  (deepseek_v4_tilelang.py:147-223);
* ``moe_route_topk(logits, k, renormalize, route_scale) -> (Tensor, Tensor)`` and
  ``fused_fp8_moe(hidden, topk_weights, topk_ids, w13, w13_scale, w2, w2_scale,
  clamp_limit, round_scale=False) -> Tensor`` -- the routed-expert slot
  (deepseek_v4_marlin.py:311); ``round_scale`` is act_quant's ue8m0 scale format;
* ``rms_norm_fp8_per_token(x, weight, eps) -> (q, scale)``,
  ``add_rms_norm_fp8_per_token(x, residual, weight, eps) -> (hidden, q, scale)``,
  ``swiglu_fp8_per_token(gate, up) -> (q, scale)`` -- the fused producers of the
  per-token FP8 linear (triton_ops.py:2239-2333).
"""
from __future__ import annotations

import torch
from torch import Tensor

from .kernels import block_fp8, fp8, fused, int4, moe

_NS = "torchinferno_amd"


# --------------------------------------------------------------------------- int4


@torch.library.custom_op(f"{_NS}::w4a16_mm", mutates_args=())
def w4a16_mm(a: Tensor, q_weight: Tensor, scales: Tensor, workspace: Tensor, size_n: int,
             size_k: int) -> Tensor:
    return int4.int4_mm(a, q_weight, scales, workspace, size_n, size_k)


@w4a16_mm.register_fake
def _w4a16_mm_fake(a, q_weight, scales, workspace, size_n, size_k):
    return a.new_empty((a.size(0), size_n))


@torch.library.custom_op(f"{_NS}::w4a16_mm_out", mutates_args=("out",))
def w4a16_mm_out(out: Tensor, a: Tensor, q_weight: Tensor, scales: Tensor, workspace: Tensor,
                 size_n: int, size_k: int) -> None:
    int4.int4_mm(a, q_weight, scales, workspace, size_n, size_k, out=out)


@w4a16_mm_out.register_fake
def _w4a16_mm_out_fake(out, a, q_weight, scales, workspace, size_n, size_k):
    return None


# --------------------------------------------------------------------------- FP8


@torch.library.custom_op(f"{_NS}::fp8_scaled_mm_out", mutates_args=("out",))
def fp8_scaled_mm_out(out: Tensor, a: Tensor, b: Tensor, a_scales: Tensor, b_scales: Tensor) -> None:
    if fp8.scaled_mm_out(out, a, b, a_scales, b_scales) is None:
        raise RuntimeError("fp8_scaled_mm_out: inputs outside the supported region "
                           "(2-D e4m3 a row-major, b column-major, K and N multiples of 16, "
                           "fp32 scales [M,1] and [1,N], bf16/fp16 out)")


@fp8_scaled_mm_out.register_fake
def _fp8_scaled_mm_out_fake(out, a, b, a_scales, b_scales):
    return None


@torch.library.custom_op(f"{_NS}::fp8_per_token_linear", mutates_args=())
def fp8_per_token_linear(x: Tensor, weight_q: Tensor, weight_scale: Tensor) -> Tensor:
    return fp8.fp8_per_token_linear(x, weight_q, weight_scale)


@fp8_per_token_linear.register_fake
def _fp8_per_token_linear_fake(x, weight_q, weight_scale):
    return x.new_empty((*x.shape[:-1], fp8.weight_nk(weight_q)[0]))


@torch.library.custom_op(f"{_NS}::act_quant", mutates_args=())
def act_quant(x: Tensor, block_size: int, round_scale: bool) -> tuple[Tensor, Tensor]:
    y, s = block_fp8.act_quant(x, block_size, "ue8m0" if round_scale else None)
    return y, s


@act_quant.register_fake
def _act_quant_fake(x, block_size, round_scale):
    return (x.new_empty(x.shape, dtype=torch.float8_e4m3fn),
            x.new_empty((*x.shape[:-1], x.size(-1) // block_size), dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::fp8_block_gemm", mutates_args=())
def fp8_block_gemm(a: Tensor, a_s: Tensor, b: Tensor, b_s: Tensor) -> Tensor:
    return block_fp8.fp8_gemm(a, a_s, b, b_s)


@fp8_block_gemm.register_fake
def _fp8_block_gemm_fake(a, a_s, b, b_s):
    return a.new_empty((*a.shape[:-1], b.size(0)), dtype=torch.bfloat16)


# --------------------------------------------------------------------------- MoE


@torch.library.custom_op(f"{_NS}::moe_route_topk", mutates_args=())
def moe_route_topk(logits: Tensor, k: int, renormalize: bool, route_scale: float) -> tuple[Tensor, Tensor]:
    w, ids = moe.route_topk(logits, k, renormalize=renormalize, route_scale=route_scale)
    return w, ids


@moe_route_topk.register_fake
def _moe_route_topk_fake(logits, k, renormalize, route_scale):
    t = logits.size(0)
    return logits.new_empty((t, k), dtype=torch.float32), logits.new_empty((t, k), dtype=torch.int32)


@torch.library.custom_op(f"{_NS}::fused_fp8_moe", mutates_args=())
def fused_fp8_moe(hidden: Tensor, topk_weights: Tensor, topk_ids: Tensor, w13: Tensor, w13_scale: Tensor,
                  w2: Tensor, w2_scale: Tensor, clamp_limit: float, round_scale: bool = False) -> Tensor:
    e, two_i, h = w13.shape
    experts = moe.PreparedFp8Experts(
        w13=w13, w13_scale=w13_scale, w2=w2, w2_scale=w2_scale,
        expert_map=torch.arange(e, dtype=torch.int32, device=w13.device),
        global_num_experts=e, hidden_size=h, intermediate_size=two_i // 2)
    return moe.fused_fp8_moe(hidden, topk_weights, topk_ids, experts, clamp_limit=clamp_limit,
                             scale_fmt="ue8m0" if round_scale else None)


@fused_fp8_moe.register_fake
def _fused_fp8_moe_fake(hidden, topk_weights, topk_ids, w13, w13_scale, w2, w2_scale, clamp_limit,
                        round_scale=False):
    return torch.empty_like(hidden)


# --------------------------------------------------------------------------- fused producers


@torch.library.custom_op(f"{_NS}::rms_norm_fp8_per_token", mutates_args=())
def rms_norm_fp8_per_token(x: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    q, s = fused.rms_norm_fp8_per_token(x, weight, eps)
    return q, s


@rms_norm_fp8_per_token.register_fake
def _rms_norm_fp8_fake(x, weight, eps):
    rows = x.numel() // x.size(-1)
    return torch.empty_like(x, dtype=torch.float8_e4m3fn), x.new_empty((rows, 1), dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::add_rms_norm_fp8_per_token", mutates_args=())
def add_rms_norm_fp8_per_token(x: Tensor, residual: Tensor, weight: Tensor,
                               eps: float) -> tuple[Tensor, Tensor, Tensor]:
    h, q, s = fused.add_rms_norm_fp8_per_token(x, residual, weight, eps)
    return h, q, s


@add_rms_norm_fp8_per_token.register_fake
def _add_rms_norm_fp8_fake(x, residual, weight, eps):
    rows = x.numel() // x.size(-1)
    return (torch.empty_like(x), torch.empty_like(x, dtype=torch.float8_e4m3fn),
            x.new_empty((rows, 1), dtype=torch.float32))


@torch.library.custom_op(f"{_NS}::swiglu_fp8_per_token", mutates_args=())
def swiglu_fp8_per_token(gate: Tensor, up: Tensor) -> tuple[Tensor, Tensor]:
    q, s = fused.swiglu_fp8_per_token(gate, up)
    return q, s


@swiglu_fp8_per_token.register_fake
def _swiglu_fp8_fake(gate, up):
    rows = gate.numel() // gate.size(-1)
    return (gate.new_empty(gate.shape, dtype=torch.float8_e4m3fn),
            gate.new_empty((rows, 1), dtype=torch.float32))
