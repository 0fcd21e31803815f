"""GPU parity of the power-of-two (E8M0) scale GEMMs -- DeepSeek-V4's "ue8m0"
format, where every scale is an exponent that the gfx950 block-scaled MFMA applies
itself (ti_fp8_gemm_block_pow2, ti_fp4_gemm_pow2, and the routed MoE with
round_scale 2) -- against the CPU oracle and against the fp32-scale GEMMs on the
same bytes.

Bar: the oracle's elementwise bound (1 bf16 ulp + 2^-16 of the sum of |terms|,
tests/_tol.py) for the block GEMM, 1e-2 max-normalised for MXFP4 (as its
fp32-scale path); every tile kind with and without split-K; and the scaled-MFMA
result within 2 bf16 ulps of the largest output of the fold path's (the two differ
only in fp32 accumulation order).
"""
import numpy as np
import pytest
import torch

from oracle import fp4 as of4
from oracle import fp8 as ofp8
from oracle import moe as omoe
from oracle.numerics import e4m3_encode
from tests._tol import abs_codes, elementwise_ratio

pytestmark = pytest.mark.gpu

E8M0 = torch.float8_e8m0fnu


def _codes(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


def _rel_err(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _near(y_pow2, y_fold):
    a, b = y_pow2.float().cpu().numpy(), y_fold.float().cpu().numpy()
    return np.abs(a - b).max() <= 2 ** -7 * np.abs(b).max()


def _block_problem(m, k, n, seed, dev):
    """W ~ N(0, 0.02) in 128x128 blocks with power-of-two scales (E8M0), x ~ N(0,1)
    through act_quant with the ue8m0 format."""
    from torchinferno_amd.kernels import block_fp8 as tb
    rng = np.random.default_rng(seed)
    # block magnitudes 2^-3..2^3 apart, so that a wrong block index changes the result
    spread = 2.0 ** rng.integers(-3, 4, (-(-n // 128), k // 128))
    w = (rng.standard_normal((n, k)) * 0.02 * np.repeat(np.repeat(spread, 128, 0), 128, 1)[:n]).astype(np.float32)
    _, s = ofp8.quantize_weight_block(w)
    s = (2.0 ** np.ceil(np.log2(s))).astype(np.float32)
    codes = ofp8.e4m3_encode(w / np.repeat(np.repeat(s, 128, 0), 128, 1)[:n, :k])
    b = torch.from_numpy(codes).to(dev).view(torch.float8_e4m3fn)
    b_s = torch.from_numpy(s).to(dev)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(torch.bfloat16).to(dev)
    x = x * (2.0 ** torch.from_numpy(rng.integers(-4, 5, (m, 1))).to(dev)).to(torch.bfloat16)
    a, a_s = tb.act_quant(x, 128, "ue8m0")
    return a, a_s, b, b_s, codes, s


def _check_block(y, a, a_s, codes, s):
    xq, xs = _codes(a), a_s.cpu().numpy()
    ref = ofp8.fp8_gemm_block(xq, xs, codes, s)
    ref_abs = ofp8.fp8_gemm_block(abs_codes(xq), xs, abs_codes(codes), s)
    return elementwise_ratio(y.float().cpu().numpy(), ref, ref_abs)


@pytest.mark.parametrize("kind", range(24))
def test_block_pow2_every_kind(dev, monkeypatch, kind):
    from torchinferno_amd.kernels import block_fp8 as tb
    a, a_s, b, b_s, codes, s = _block_problem(200, 1280, 400, 50 + kind, dev)
    for splits in ("1", "3"):
        print(f"[pow2] block kind {kind} splits={splits}", flush=True)
        monkeypatch.setenv("TI_ROCM_FP8_KIND", str(kind))
        monkeypatch.setenv("TI_ROCM_FP8_SPLITS", splits)
        y = tb._fp8_gemm_raw(a, a_s, 0, b, b_s, True)
        torch.cuda.synchronize()
        assert _check_block(y, a, a_s, codes, s) <= 1.0, (kind, splits)
        # step-major activation scales: the same exponents, the same result
        assert torch.equal(y, tb._fp8_gemm_raw(a, a_s.t().contiguous(), 1, b, b_s, True)), (kind, splits)
        assert _near(y, tb._fp8_gemm_raw(a, a_s, 0, b, b_s, False)), (kind, splits)


@pytest.mark.parametrize("m", [1, 16, 77, 256, 4096])
def test_block_pow2_public_api(dev, m):
    """fp8_gemm(scale_dtype=float8_e8m0fnu) at the config-3 K (7168) and M, sampled
    against the oracle."""
    from torchinferno_amd.kernels import block_fp8 as tb
    print(f"[pow2] block api M={m}", flush=True)
    a, a_s, b, b_s, codes, s = _block_problem(m, 7168, 1536, m, dev)
    y = tb.fp8_gemm(a, a_s.to(E8M0), b, b_s.to(E8M0), E8M0)
    assert torch.equal(y, tb._fp8_gemm_raw(a, a_s, 0, b, b_s, True))
    rows = np.unique(np.linspace(0, m - 1, min(m, 24)).astype(int))
    cols = np.unique(np.linspace(0, b.size(0) - 1, 200).astype(int))
    ri, ci = torch.as_tensor(rows, device=dev), torch.as_tensor(cols, device=dev)
    ratio = 0.0
    for blk in np.unique(cols // 128):
        sel = cols[cols // 128 == blk]
        sub = torch.as_tensor(sel, device=dev)
        xq, xs = _codes(a[ri]), a_s[ri].cpu().numpy()
        ref = ofp8.fp8_gemm_block(xq, xs, codes[sel], s[blk:blk + 1])
        ref_abs = ofp8.fp8_gemm_block(abs_codes(xq), xs, abs_codes(codes[sel]), s[blk:blk + 1])
        ratio = max(ratio, elementwise_ratio(y[ri][:, sub].float().cpu().numpy(), ref, ref_abs))
    assert ratio <= 1.0, ratio


def test_block_pow2_env_switch(dev, monkeypatch):
    from torchinferno_amd.kernels import block_fp8 as tb
    a, a_s, b, b_s, _, _ = _block_problem(64, 1024, 512, 3, dev)
    monkeypatch.setenv("TI_ROCM_POW2_MFMA", "0")
    y = tb.fp8_gemm(a, a_s.to(E8M0), b, b_s.to(E8M0), E8M0)
    assert torch.equal(y, tb.fp8_gemm(a, a_s, b, b_s))  # the fp32-scale GEMM, bit for bit


def _fp4_inputs(m, n, k, seed, dev):
    rng = np.random.default_rng(seed)
    a = e4m3_encode((rng.standard_normal((m, k)) * 60).astype(np.float32))
    a_s = (2.0 ** rng.integers(-12, -4, (m, k // 128))).astype(np.float32)
    b = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    b_s = rng.integers(118, 132, (n, k // 32), dtype=np.uint8)
    t = (torch.from_numpy(a).to(dev).view(torch.float8_e4m3fn), torch.from_numpy(a_s).to(dev),
         torch.from_numpy(b).to(dev).view(torch.float4_e2m1fn_x2),
         torch.from_numpy(b_s).to(dev).view(E8M0))
    return (a, a_s, b, b_s), t


@pytest.mark.parametrize("kind", ["1", "2", "3", "5", "6", "9", "10", "11", "12", "13", "15", "16", "17", "18", "23",
                                  "19", "20"])
def test_fp4_pow2_every_kind(dev, monkeypatch, kind):
    from torchinferno_amd.kernels import block_fp8 as tb
    host, (a, a_s, b, b_s) = _fp4_inputs(77, 400, 1536, int(kind), dev)
    ref = of4.fp4_gemm(*host)
    st = tb.fp4_scale_stepmajor(b_s.view(torch.uint8))
    for splits in ("1", "3"):
        print(f"[pow2] fp4 kind {kind} splits {splits}", flush=True)
        monkeypatch.setenv("TI_ROCM_FP8_KIND", kind)
        monkeypatch.setenv("TI_ROCM_FP8_SPLITS", splits)
        y = tb.fp4_gemm(a, a_s.to(E8M0), b, b_s, E8M0)
        assert _rel_err(y.float().cpu().numpy(), ref) <= 1e-2, (kind, splits)
        assert torch.equal(y, tb._fp4_gemm_raw(a, a_s.t().contiguous(), 1, b, st, 1, 400, True))
        assert _near(y, tb.fp4_gemm(a, a_s, b, b_s)), (kind, splits)


def _fp8_experts_pow2(e, h, inter, seed, dev):
    from torchinferno_amd.kernels import moe as tmoe
    rng = np.random.default_rng(seed)

    def w(n, k):
        f = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        _, s = ofp8.quantize_weight_block(f)
        s = (2.0 ** np.ceil(np.log2(s))).astype(np.float32)
        c = ofp8.e4m3_encode(f / np.repeat(np.repeat(s, 128, 0), 128, 1))
        return torch.from_numpy(c).to(dev).view(torch.float8_e4m3fn), torch.from_numpy(s).to(dev).to(E8M0)
    ws = [[w(inter, h), w(inter, h), w(h, inter)] for _ in range(e)]
    st = lambda i, j: torch.stack([x[i][j] for x in ws])  # noqa: E731
    return tmoe.prepare_fp8_experts(st(0, 0), st(1, 0), st(2, 0), st(0, 1), st(1, 1), st(2, 1))


@pytest.mark.parametrize("fmt", ["fp8", "fp4"])
@pytest.mark.parametrize("t,k,kind", [(9, 2, "auto"), (300, 8, "auto"), (300, 8, "17"), (300, 8, "20"),
                                      (300, 8, "11"), (600, 8, "16")])
def test_moe_pow2_matches_oracle(dev, monkeypatch, fmt, t, k, kind):
    """Routed experts under "ue8m0" with E8M0 weight scales: round_scale 2 (scales in
    the MFMA) against the per-expert oracle loop and the fold path (round_scale 1)."""
    from torchinferno_amd.kernels import moe as tmoe
    print(f"[pow2] moe {fmt} T={t} k={k} kind={kind}", flush=True)
    if kind != "auto":
        monkeypatch.setenv("TI_ROCM_MOE_KIND", kind)
    e, h, inter = 8, 512, 256
    if fmt == "fp8":
        ex = _fp8_experts_pow2(e, h, inter, t + k, dev)
        assert ex.scales_pow2
        run, lin = tmoe.fused_fp8_moe, omoe.block_fp8_linear
        experts = [(_codes(ex.w13[i]), ex.w13_scale[i].cpu().numpy(), _codes(ex.w2[i]),
                    ex.w2_scale[i].cpu().numpy()) for i in range(e)]
    else:
        from tests.test_fp4_gpu import _mxfp4_experts
        ex = _mxfp4_experts(e, h, inter, t + k, dev)
        run, lin = tmoe.fused_mxfp4_moe, omoe.mxfp4_linear

        def rows(st):  # step-major [K/128, N, 4] -> checkpoint [N, K/32]
            return st.permute(1, 0, 2).reshape(st.size(1), -1).cpu().numpy()
        experts = [(ex.w13[i].cpu().numpy(), rows(ex.w13_scale[i]), ex.w2[i].cpu().numpy(), rows(ex.w2_scale[i]))
                   for i in range(e)]
    g = torch.Generator(device=dev).manual_seed(t)
    x = torch.randn((t, h), generator=g, device=dev).to(torch.bfloat16)
    w, ids = tmoe.route_topk(torch.randn((t, e), generator=g, device=dev), k)
    y = run(x, w, ids, ex, scale_fmt="ue8m0")
    monkeypatch.setenv("TI_ROCM_POW2_MFMA", "0")
    y_fold = run(x, w, ids, ex, scale_fmt="ue8m0")
    ref = omoe.moe_reference(x.float().cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy(), experts,
                             linear=omoe.ue8m0(lin))
    got = y.float().cpu().numpy()
    assert _rel_err(got, ref) <= 1.5e-2
    assert _rel_err(got, y_fold.float().cpu().numpy()) <= 1.5e-2


@pytest.mark.parametrize("entry", ["ti_fp8_gemm_block_pow2", "ti_fp4_gemm_pow2"])
@pytest.mark.parametrize("m", [5, 300])
def test_pow2_c_abi_fp16_out(dev, entry, m):
    """The C ABI's fp16 output on the power-of-two paths: the same fp32 sums as the
    bf16 output (each output within the rounding of both formats of the other)."""
    from torchinferno_amd import _lib
    from torchinferno_amd.kernels import block_fp8 as tb
    from torchinferno_amd.kernels.fp8 import _ws_args
    if entry == "ti_fp8_gemm_block_pow2":
        a, a_s, b, b_s, _, _ = _block_problem(m, 1024, 384, 7, dev)
        n, k, extra, mode = 384, 1024, (), 3
    else:
        _, (a, a_s, b, b_s) = _fp4_inputs(m, 384, 1024, 7, dev)
        b_s = b_s.view(torch.uint8).contiguous()
        n, k, extra, mode = 384, 1024, (0,), 4
    outs = {}
    for code, dt in ((_lib.TI_DTYPE_BF16, torch.bfloat16), (_lib.TI_DTYPE_F16, torch.float16)):
        out = torch.empty((m, n), dtype=dt, device=dev)
        ws, ws_bytes = _ws_args(dev, m, n, k, mode)
        _lib.call(entry, a.data_ptr(), a_s.data_ptr(), 0, b.data_ptr(), b_s.data_ptr(), *extra, out.data_ptr(),
                  code, m, n, k, ws, ws_bytes, _lib.stream_of(a))
        outs[dt] = out.float().cpu().numpy()
    y16, yb = outs[torch.float16], outs[torch.bfloat16]
    assert np.isfinite(y16).all()
    assert np.abs(y16 - yb).max() <= 2 ** -8 * np.abs(yb).max() + 1e-6
