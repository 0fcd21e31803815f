"""Pins oracle/moe.py (CPU): router against brute force and closed forms; the
expert path against unquantized fp64 math (a swapped w1/w3 half, a transposed
weight or a dropped route weight fails it); token-permutation equivariance;
routes that do not exist contribute nothing."""
import itertools

import numpy as np

from oracle import fp8 as ofp8
from oracle import moe as omoe
from oracle.numerics import bf16_round

F32 = np.float32


def test_router_brute_force_small():
    rng = np.random.default_rng(0)
    z = rng.standard_normal((6, 5)).astype(F32)
    w, ids = omoe.route_softmax_topk(z, 2)
    for t in range(6):
        p = np.exp(z[t].astype(np.float64) - z[t].max())
        p /= p.sum()
        best = max(itertools.combinations(range(5), 2), key=lambda c: sum(p[list(c)]))
        assert set(ids[t]) == set(best)
        assert p[ids[t, 0]] >= p[ids[t, 1]]
        np.testing.assert_allclose(w[t], p[ids[t]] / p[ids[t]].sum(), rtol=1e-6)


def test_router_k_equals_e_is_softmax_and_scale():
    rng = np.random.default_rng(1)
    z = rng.standard_normal((3, 8)).astype(F32)
    w, ids = omoe.route_softmax_topk(z, 8, renormalize=False)
    p = np.exp(z - z.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    np.testing.assert_allclose(np.take_along_axis(p, ids, 1), w, rtol=1e-6)
    w2, _ = omoe.route_softmax_topk(z, 3, route_scale=2.5)
    np.testing.assert_allclose(w2.sum(1), 2.5, rtol=1e-6)


def _experts(rng, e, h, inter):
    out = []
    for _ in range(e):
        w13, s13 = ofp8.quantize_weight_block((rng.standard_normal((2 * inter, h)) * 0.05).astype(F32))
        w2, s2 = ofp8.quantize_weight_block((rng.standard_normal((h, inter)) * 0.05).astype(F32))
        out.append((w13, s13, w2, s2))
    return out


def test_expert_matches_unquantized_fp64_math():
    rng = np.random.default_rng(2)
    h, inter = 256, 128
    (w13, s13, w2, s2), = _experts(rng, 1, h, inter)
    x = bf16_round(rng.standard_normal((4, h)).astype(F32))
    rw = np.array([[1.0], [0.5], [0.25], [2.0]], F32)
    got = omoe.expert_forward(x, rw, w13, s13, w2, s2)
    W13 = ofp8.dequantize_block_fp8(w13, s13).astype(np.float64)
    W2 = ofp8.dequantize_block_fp8(w2, s2).astype(np.float64)
    gu = x.astype(np.float64) @ W13.T
    g, u = gu[:, :inter], gu[:, inter:]
    hid = rw * (g / (1 + np.exp(-g))) * u
    want = hid @ W2.T
    # activation quantization (e4m3, 3 mantissa bits) twice over K=128-256 sums: ~5%
    assert np.abs(got - want).max() <= 0.08 * np.abs(want).max()
    # swapping the w1/w3 halves is caught
    w13s = np.concatenate([w13[inter:], w13[:inter]])
    s13s = np.concatenate([s13[1:], s13[:1]])
    bad = omoe.expert_forward(x, rw, w13s, s13s, w2, s2)
    assert np.abs(bad - want).max() > 0.2 * np.abs(want).max()


def test_moe_permutation_equivariance_and_missing_routes():
    rng = np.random.default_rng(3)
    h, inter, e, t, k = 128, 128, 4, 6, 2
    experts = _experts(rng, e, h, inter)
    x = bf16_round(rng.standard_normal((t, h)).astype(F32))
    w, ids = omoe.route_softmax_topk(rng.standard_normal((t, e)).astype(F32), k)
    y = omoe.moe_reference(x, w, ids, experts)
    perm = rng.permutation(t)
    yp = omoe.moe_reference(x[perm], w[perm], ids[perm], experts)
    np.testing.assert_array_equal(yp, y[perm])
    # a route to an expert id outside [0, E) adds nothing
    ids2 = ids.copy()
    ids2[0, 1] = e + 5
    y2 = omoe.moe_reference(x, w, ids2, experts)
    only = omoe.moe_reference(x[:1], w[:1, :1], ids[:1, :1], experts)
    np.testing.assert_array_equal(y2[0], only[0])


def test_expert_clamp_limit_matches_fp64_math():
    """swiglu_limit (tensor_parallel.py:796-800): up clamped to [-l, l], gate to <= l.
    With l small the clamp is active on most elements; the fp64 restatement agrees and
    the unclamped expert does not."""
    rng = np.random.default_rng(5)
    h, inter, lim = 256, 128, 0.3
    (w13, s13, w2, s2), = _experts(rng, 1, h, inter)
    x = bf16_round(rng.standard_normal((3, h)).astype(F32))
    rw = np.ones((3, 1), F32)
    got = omoe.expert_forward(x, rw, w13, s13, w2, s2, clamp_limit=lim)
    W13 = ofp8.dequantize_block_fp8(w13, s13).astype(np.float64)
    W2 = ofp8.dequantize_block_fp8(w2, s2).astype(np.float64)
    gu = x.astype(np.float64) @ W13.T
    g, u = np.minimum(gu[:, :inter], lim), np.clip(gu[:, inter:], -lim, lim)
    want = ((g / (1 + np.exp(-g))) * u) @ W2.T
    assert np.abs(got - want).max() <= 0.08 * np.abs(want).max()
    free = omoe.expert_forward(x, rw, w13, s13, w2, s2)
    assert np.abs(free - want).max() > 0.5 * np.abs(want).max()


def test_ue8m0_linear_uses_power_of_two_activation_scales():
    """scale_fmt "ue8m0": the activation scales are 2^ceil(log2(amax/448)); the linear
    stays within quantization error of the fp64 product and differs from the plain one."""
    rng = np.random.default_rng(6)
    (w13, s13, _, _), = _experts(rng, 1, 256, 128)
    x = bf16_round(rng.standard_normal((5, 256)).astype(F32))
    pow2 = omoe.ue8m0(omoe.block_fp8_linear)(x, w13, s13)
    plain = omoe.block_fp8_linear(x, w13, s13)
    want = x.astype(np.float64) @ ofp8.dequantize_block_fp8(w13, s13).astype(np.float64).T
    assert np.abs(pow2 - want).max() <= 0.05 * np.abs(want).max()
    assert not np.array_equal(pow2, plain)
    xq, xs = ofp8.act_quant_block(x, round_scale=True)
    assert np.array_equal(pow2, bf16_round(ofp8.fp8_gemm_block(xq, xs, w13, s13)))
    assert np.all(np.log2(xs) == np.round(np.log2(xs)))
