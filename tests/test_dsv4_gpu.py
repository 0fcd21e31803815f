"""DeepSeek-V4 drop-in on the GPU against the CPU oracle, with the model's scale
settings: ``scale_fmt = "ue8m0"`` (power-of-two activation scales) and
``scale_dtype`` fp32 or ``float8_e8m0fnu``, the globals the reference's DSv4
module reads in ``linear`` and ``Expert.forward``
(src/torchinferno/models/deepseek_v4/tensor_parallel.py:195-207,792-802,
1199-1212,1641).

Bar: the patched ``linear`` within an elementwise bound of the oracle
(1 bf16 ulp + 2^-16 of the sum of |terms|, tests/_tol.py) on the same weights;
the MoE hook within 1.5e-2 of the oracle's per-expert loop (max-normalised: two
chained activation quants, where a one-ulp bf16 difference in an intermediate
can flip an e4m3 code; measured up to 1.5 bf16 ulps of the largest output), with
99% of the elements within a quarter of that.  Each
test also shows that the oracle with plain ``amax/448`` scales -- the scale
format a missed ``scale_fmt`` would give -- is NOT within that bound, so the
tests tell the two formats apart.
"""
import sys
import types

import numpy as np
import pytest
import torch

from oracle import fp4 as of4
from oracle import fp8 as ofp8
from oracle import moe as omoe
from oracle.numerics import bf16_round
from tests._tol import abs_codes, elementwise_ratio

pytestmark = pytest.mark.gpu

MOE_TOL = 1.5e-2


def _codes(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


def _rel_err(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _fake_module(name, scale_fmt, scale_dtype):
    from torchinferno_amd import hooks
    mod = types.ModuleType(name)
    mod.linear = None
    mod.scale_fmt = scale_fmt
    mod.scale_dtype = scale_dtype
    sys.modules[name] = mod
    undo = hooks.patch_deepseek_v4_module(mod)
    return mod, undo


def _fp8_weight(n, k, rng, dev, scale_dtype):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    codes, s = ofp8.quantize_weight_block(w)
    if scale_dtype == torch.float8_e8m0fnu:
        # E8M0 storage holds powers of two: round the block scales up to one
        s = (2.0 ** np.ceil(np.log2(s))).astype(np.float32)
        codes = ofp8.e4m3_encode(w / np.repeat(np.repeat(s, 128, 0), 128, 1)[:n, :k])
    wt = torch.from_numpy(codes).to(dev).view(torch.float8_e4m3fn)
    wt.scale = torch.from_numpy(s).to(dev).to(scale_dtype)
    return wt, codes, s


def _fp4_weight(n, k, rng, dev):
    packed = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    sc = rng.integers(116, 121, (n, k // 32), dtype=np.uint8)
    wt = torch.from_numpy(packed).to(dev).view(torch.float4_e2m1fn_x2)
    wt.scale = torch.from_numpy(sc).to(dev).view(torch.float8_e8m0fnu)
    return wt, packed, sc


@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.float8_e8m0fnu])
@pytest.mark.parametrize("m,k,n", [(1, 512, 256), (37, 1024, 384), (300, 7168, 512)])
def test_linear_ue8m0_fp8_matches_oracle(dev, scale_dtype, m, k, n):
    print(f"[dsv4] linear fp8 ue8m0 {scale_dtype} M={m} K={k} N={n}", flush=True)
    mod, undo = _fake_module(f"fake_dsv4_lin_{m}", "ue8m0", scale_dtype)
    try:
        rng = np.random.default_rng(m + k + n)
        wt, codes, s = _fp8_weight(n, k, rng, dev, scale_dtype)
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
        y = mod.linear(x.to(dev), wt).float().cpu().numpy()
        xh = x.float().numpy()
        xq, xs = ofp8.act_quant_block(xh, round_scale=True)
        ref = ofp8.fp8_gemm_block(xq, xs, codes, s)
        ref_abs = ofp8.fp8_gemm_block(abs_codes(xq), xs, abs_codes(codes), s)
        assert elementwise_ratio(y, ref, ref_abs) <= 1.0
        # the plain-scale oracle (scale_fmt None) is told apart
        pq, ps = ofp8.act_quant_block(xh)
        plain = ofp8.fp8_gemm_block(pq, ps, codes, s)
        assert elementwise_ratio(y, plain, ref_abs) > 1.0
    finally:
        undo()
        del sys.modules[mod.__name__]


@pytest.mark.parametrize("m,k,n", [(1, 512, 256), (45, 2048, 320)])
def test_linear_ue8m0_fp4_matches_oracle(dev, m, k, n):
    print(f"[dsv4] linear fp4 ue8m0 M={m} K={k} N={n}", flush=True)
    mod, undo = _fake_module(f"fake_dsv4_fp4_{m}", "ue8m0", torch.float32)
    try:
        rng = np.random.default_rng(m * 3 + n)
        wt, packed, sc = _fp4_weight(n, k, rng, dev)
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16)
        y = mod.linear(x.to(dev), wt).float().cpu().numpy()
        xq, xs = ofp8.act_quant_block(x.float().numpy(), round_scale=True)
        ref = of4.fp4_gemm(xq, xs, packed, sc)
        ref_abs = of4.fp4_gemm(abs_codes(xq), xs, packed & 0x77, sc)
        assert elementwise_ratio(y, ref, ref_abs) <= 1.0
        pq, ps = ofp8.act_quant_block(x.float().numpy())
        assert elementwise_ratio(y, of4.fp4_gemm(pq, ps, packed, sc), ref_abs) > 1.0
    finally:
        undo()
        del sys.modules[mod.__name__]


def test_block_api_e8m0_scale_storage(dev):
    """act_quant(scale_dtype=float8_e8m0fnu) returns the same powers of two as E8M0;
    fp8_gemm on E8M0 scales equals the power-of-two GEMM on their fp32 values bit for
    bit, and both it and the fp32-scale GEMM are within the oracle's bound."""
    from torchinferno_amd.kernels import block_fp8 as tb
    rng = np.random.default_rng(3)
    wt, codes, s = _fp8_weight(256, 1024, rng, dev, torch.float8_e8m0fnu)
    x = torch.from_numpy(rng.standard_normal((20, 1024)).astype(np.float32)).to(torch.bfloat16).to(dev)
    q8, s8 = tb.act_quant(x, 128, "ue8m0", torch.float8_e8m0fnu)
    q32, s32 = tb.act_quant(x, 128, "ue8m0")
    assert s8.dtype == torch.float8_e8m0fnu and torch.equal(s8.float(), s32)
    assert torch.equal(q8.view(torch.uint8), q32.view(torch.uint8))
    y8 = tb.fp8_gemm(q8, s8, wt, wt.scale, torch.float8_e8m0fnu)
    y32 = tb.fp8_gemm(q32, s32, wt, wt.scale.float())
    assert torch.equal(y8, tb._fp8_gemm_raw(q32, s32, 0, wt, wt.scale.float(), True))
    xq, xs = _codes(q32), s32.cpu().numpy()
    ref = ofp8.fp8_gemm_block(xq, xs, codes, s)
    ref_abs = ofp8.fp8_gemm_block(abs_codes(xq), xs, abs_codes(codes), s)
    for y in (y8, y32):
        assert elementwise_ratio(y.float().cpu().numpy(), ref, ref_abs) <= 1.0
    with pytest.raises(ValueError):
        tb.act_quant(x, 128, None, torch.float8_e8m0fnu)
    with pytest.raises(ValueError):
        tb.fp8_gemm(q32, s32, wt, wt.scale)  # E8M0 weight scales with scale_dtype fp32


def _moe_model(mod, e, h, inter, k, fmt, clamp, rng, dev):
    """A DSv4-shaped MoE object (gate, experts, shared expert) whose class lives in
    ``mod``, the module whose globals the hook reads."""
    from torchinferno_amd.kernels import moe as tmoe

    def weight(n, kk):
        if fmt == "fp8":
            return _fp8_weight(n, kk, rng, dev, torch.float32)[0]
        if fmt == "fp8e8m0":  # E8M0 weight scales: all scales powers of two
            return _fp8_weight(n, kk, rng, dev, torch.float8_e8m0fnu)[0]
        return _fp4_weight(n, kk, rng, dev)[0]

    class Lin:
        def __init__(self, n, kk):
            self.weight = weight(n, kk)
            self.scale = self.weight.scale

    class Expert:
        swiglu_limit = clamp

        def __init__(self):
            self.w1, self.w3, self.w2 = Lin(inter, h), Lin(inter, h), Lin(h, inter)

    class Shared:
        swiglu_limit = clamp

        def __call__(self, x):
            return torch.zeros_like(x)

    gw = torch.from_numpy(rng.standard_normal((e, h)).astype(np.float32)).to(dev)

    class Gate:
        def __call__(self, x, ids):
            return tmoe.route_topk(x.float() @ gw.t(), k)

    MoE = type("MoE", (), {"__module__": mod.__name__})
    m = object.__new__(MoE)
    m.dim, m.n_routed_experts, m.experts_start_idx, m.experts_end_idx = h, e, 0, e
    m.gate, m.experts, m.shared_experts = Gate(), [Expert() for _ in range(e)], Shared()
    return m


def _host_experts(m, fmt):
    out = []
    for ex in m.experts:
        w13 = np.concatenate([_codes(ex.w1.weight), _codes(ex.w3.weight)])
        w2 = _codes(ex.w2.weight)
        s13 = np.concatenate([_codes(ex.w1.scale) if fmt == "fp4" else ex.w1.scale.float().cpu().numpy(),
                              _codes(ex.w3.scale) if fmt == "fp4" else ex.w3.scale.float().cpu().numpy()])
        s2 = _codes(ex.w2.scale) if fmt == "fp4" else ex.w2.scale.float().cpu().numpy()
        out.append((w13, s13, w2, s2))
    return out


@pytest.mark.parametrize("fmt", ["fp8", "fp8e8m0", "fp4"])
@pytest.mark.parametrize("t,clamp", [(5, 0.0), (40, 0.0), (300, 0.4)])
def test_moe_hook_ue8m0_matches_oracle(dev, fmt, t, clamp):
    """MoE.forward with fused experts (prepare_fused_experts -> fused_{fp8,mxfp4}_moe)
    under scale_fmt "ue8m0": every expert Linear quantizes its input with power-of-two
    scales, as the reference's Expert -> linear -> act_quant does.  With E8M0 weight
    scales (fp8e8m0, fp4) the grouped GEMMs apply all scales inside the MFMA."""
    from torchinferno_amd import hooks
    print(f"[dsv4] moe hook {fmt} ue8m0 T={t} clamp={clamp}", flush=True)
    mod, undo = _fake_module(f"fake_dsv4_moe_{fmt}_{t}", "ue8m0", torch.float32)
    try:
        e, h, inter, k = 8, 512, 256, 3
        rng = np.random.default_rng(t + (7 if fmt == "fp4" else 0))
        m = _moe_model(mod, e, h, inter, k, fmt, clamp, rng, dev)
        assert hooks.prepare_fused_fp8_experts(m)
        x = torch.from_numpy(rng.standard_normal((t, h)).astype(np.float32)).to(torch.bfloat16).to(dev)
        y = hooks.moe_forward(m, x.view(1, t, h), torch.zeros((1, t), dtype=torch.long, device=dev))
        w, ids = m.gate(x, None)
        lin = omoe.mxfp4_linear if fmt == "fp4" else omoe.block_fp8_linear
        args = (x.float().cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy(), _host_experts(m, fmt))
        ref = omoe.moe_reference(*args, linear=omoe.ue8m0(lin), clamp_limit=clamp)
        got = y.view(t, h).float().cpu().numpy()
        plain = omoe.moe_reference(*args, linear=lin, clamp_limit=clamp)
        scale = np.abs(ref).max()
        d, dp = np.abs(got - ref) / scale, np.abs(got - plain) / scale
        # max within MOE_TOL; 99% of elements within a quarter of it; the plain-scale
        # oracle is several times further away on both measures
        assert d.max() <= MOE_TOL, d.max()
        assert np.percentile(d, 99) <= MOE_TOL / 4, np.percentile(d, 99)
        assert dp.max() > 3 * d.max() and np.percentile(dp, 99) > 3 * np.percentile(d, 99)
    finally:
        undo()
        del sys.modules[mod.__name__]
