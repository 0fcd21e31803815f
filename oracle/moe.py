"""Oracle for the routed FP8 block-scaled MoE (test infrastructure only).

Reference arithmetic followed:

* Router: softmax over fp32 logits, top-k, gather the softmax scores of the
  chosen experts, renormalise to sum 1, times a route scale --
  src/torchinferno/models/deepseek_v32/model.py:692-722 (``DeepSeekMoEGate``
  with ``scoring_func="softmax"``, ``norm_topk_prob=True``, single group) and
  src/torchinferno/models/deepseek_v4/tensor_parallel.py:760-780.
  Renormalisation divides by ``sum.clamp_min(1e-20)`` (model.py:719).
* Expert: ``gate = w1(x).float()``, ``up = w3(x).float()``, with
  ``swiglu_limit > 0``: ``up = clamp(up, -limit, limit)``,
  ``gate = clamp(gate, max=limit)``; ``h = silu(gate) * up``,
  ``h = weight * h``, ``w2(h.to(bf16))`` -- deepseek_v4/tensor_parallel.py:
  792-802, where every ``wi`` is a block-FP8 ``Linear``: 1x128 activation quant
  (power-of-two scales when the module's ``scale_fmt`` is set, "ue8m0" on the
  checkpoint path, :1199-1211,1641) then the block-scaled GEMM with a bf16
  output (tensor_parallel.py:195-207).
* Combine: ``y = zeros(fp32)``; for each expert in index order,
  ``y[idx] += expert(x[idx], w[idx, slot])``; ``y.type_as(x)`` --
  deepseek_v4/tensor_parallel.py:897-914.

The gate-up weight of one expert is stored fused as ``w13 = [w1; w3]``
([2I, H]), the layout the reference's grouped path builds
(src/torchinferno/kernels/deepseek_v4_marlin.py:218-219).

Pinning (tests/test_oracle_moe.py): router vs brute-force sort on tiny inputs
and closed-form weights (k = E gives the plain softmax); all routes on one
expert reduce to that expert's dense FFN; token permutation equivariance;
linearity in the route weight through w2's input.
"""
from __future__ import annotations

import numpy as np

from .fp4 import fp4_gemm
from .fp8 import act_quant_block, fp8_gemm_block
from .numerics import bf16_round

F32 = np.float32


def route_softmax_topk(logits: np.ndarray, k: int, renormalize: bool = True,
                       route_scale: float = 1.0) -> tuple[np.ndarray, np.ndarray]:
    """logits fp32 [T,E] -> (weights fp32 [T,k], ids int32 [T,k]) in descending score order."""
    z = np.asarray(logits, dtype=F32)
    z = z - z.max(axis=1, keepdims=True)
    e = np.exp(z.astype(np.float64))
    p = (e / e.sum(axis=1, keepdims=True)).astype(F32)
    ids = np.argsort(-p, axis=1, kind="stable")[:, :k].astype(np.int32)
    w = np.take_along_axis(p, ids, axis=1)
    if renormalize:
        w = w / np.maximum(w.sum(axis=1, keepdims=True), F32(1e-20))
    return (w * F32(route_scale)).astype(F32), ids


def block_fp8_linear(x_bf16: np.ndarray, w_codes: np.ndarray, w_s: np.ndarray,
                     round_scale: bool = False) -> np.ndarray:
    """DSv4 ``linear`` for an e4m3 weight: act_quant 1x128 then fp8_gemm, bf16 out."""
    xq, xs = act_quant_block(x_bf16, round_scale=round_scale)
    return bf16_round(fp8_gemm_block(xq, xs, w_codes, w_s))


def mxfp4_linear(x_bf16: np.ndarray, w_packed: np.ndarray, w_s: np.ndarray,
                 round_scale: bool = False) -> np.ndarray:
    """DSv4 ``linear`` for an MXFP4 weight: act_quant 1x128 then fp4_gemm, bf16 out."""
    xq, xs = act_quant_block(x_bf16, round_scale=round_scale)
    return bf16_round(fp4_gemm(xq, xs, w_packed, w_s))


def ue8m0(linear):
    """The same Linear with the "ue8m0" scale format (power-of-two activation scales)."""
    return lambda x, w, s: linear(x, w, s, round_scale=True)


def expert_forward(x_bf16: np.ndarray, route_w: np.ndarray, w13: np.ndarray, s13: np.ndarray,
                   w2: np.ndarray, s2: np.ndarray, linear=block_fp8_linear,
                   clamp_limit: float = 0.0) -> np.ndarray:
    """One expert on its routed rows.  x bf16-valued [R,H], route_w [R,1];
    ``linear`` is the weight format's Linear (block FP8 or MXFP4)."""
    inter = w13.shape[0] // 2
    gu = linear(x_bf16, w13, s13)  # [R, 2I] bf16 values
    gate, up = gu[:, :inter], gu[:, inter:]
    if clamp_limit > 0:
        lim = F32(clamp_limit)
        up = np.clip(up, -lim, lim)
        gate = np.minimum(gate, lim)
    with np.errstate(over="ignore"):
        e = np.exp(-gate.astype(np.float64)).astype(F32)
    h = (gate / (F32(1.0) + e)).astype(F32) * up  # F.silu(gate) = gate / (1 + exp(-gate)), fp32
    h = (route_w.astype(F32) * h).astype(F32)
    return linear(bf16_round(h), w2, s2)


def moe_reference(x_bf16: np.ndarray, weights: np.ndarray, ids: np.ndarray,
                  experts: list[tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]],
                  linear=block_fp8_linear, clamp_limit: float = 0.0) -> np.ndarray:
    """Per-expert loop; returns fp32 values rounded to bf16, [T,H]."""
    t, h = x_bf16.shape
    y = np.zeros((t, h), dtype=F32)
    for e, (w13, s13, w2, s2) in enumerate(experts):
        tok, slot = np.nonzero(ids == e)
        if tok.size == 0:
            continue
        out = expert_forward(x_bf16[tok], weights[tok, slot][:, None], w13, s13, w2, s2, linear, clamp_limit)
        np.add.at(y, tok, out)
    return bf16_round(y)
