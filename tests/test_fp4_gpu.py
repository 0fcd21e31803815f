"""GPU parity of the MXFP4 path (FP8 activations x e2m1 weights with E8M0 scales
per 32 K) against oracle/fp4.py and oracle/moe.py.

Bar: max|y - ref| <= 1e-2 * max|ref| against the fp32-accumulated oracle on the
same bytes (bf16 output); the one-hot closed form is exact.  Every tile kind the
MXFP4 path instantiates runs with and without split-K on ragged shapes.
"""
import numpy as np
import pytest
import torch

from oracle import fp4 as of4
from oracle import moe as omoe
from oracle.numerics import e4m3_encode

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _rel_err(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def _inputs(m, n, k, seed, dev):
    rng = np.random.default_rng(seed)
    a = e4m3_encode((rng.standard_normal((m, k)) * 60).astype(np.float32))
    a_s = (rng.random((m, k // 128)) * 0.01 + 1e-3).astype(np.float32)
    b = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    b_s = rng.integers(118, 132, (n, k // 32), dtype=np.uint8)
    t = (torch.from_numpy(a).to(dev).view(torch.float8_e4m3fn), torch.from_numpy(a_s).to(dev),
         torch.from_numpy(b).to(dev).view(torch.float4_e2m1fn_x2),
         torch.from_numpy(b_s).to(dev).view(torch.float8_e8m0fnu))
    return (a, a_s, b, b_s), t


@pytest.mark.parametrize("m,n,k", [(1, 256, 128), (3, 320, 512), (16, 128, 1024), (64, 384, 256),
                                   (130, 256, 640), (512, 512, 512), (700, 1152, 256)])
def test_fp4_gemm_matches_oracle(dev, m, n, k):
    from torchinferno_amd.kernels import block_fp8 as tb
    print(f"[fp4] gemm M={m} N={n} K={k}", flush=True)
    host, (a, a_s, b, b_s) = _inputs(m, n, k, m + n + k, dev)
    y = tb.fp4_gemm(a, a_s, b, b_s)
    ref = of4.fp4_gemm(*host)
    assert y.dtype == torch.bfloat16 and y.shape == (m, n)
    assert _rel_err(y.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("kind", ["1", "2", "3", "5", "6", "9", "10", "11", "12", "13", "15", "16", "17", "18", "23",
                                  "19", "20"])
@pytest.mark.parametrize("splits", ["1", "3"])
def test_fp4_gemm_every_kind(dev, monkeypatch, kind, splits):
    """Both scale layouts: the checkpoint's [N, K/32] and the step-major copy."""
    from torchinferno_amd.kernels import block_fp8 as tb
    print(f"[fp4] kind {kind} splits {splits}", flush=True)
    monkeypatch.setenv("TI_ROCM_FP8_KIND", kind)
    monkeypatch.setenv("TI_ROCM_FP8_SPLITS", splits)
    host, (a, a_s, b, b_s) = _inputs(77, 400, 1536, int(kind) * 10 + int(splits), dev)
    ref = of4.fp4_gemm(*host)
    y = tb.fp4_gemm(a, a_s, b, b_s)
    assert _rel_err(y.float().cpu().numpy(), ref) <= TOL
    st = tb.fp4_scale_stepmajor(b_s.view(torch.uint8))
    y2 = tb._fp4_gemm_raw(a, a_s, 0, b, st, 1, 400)
    assert torch.equal(y, y2)
    y3 = tb._fp4_gemm_raw(a, a_s.t().contiguous(), 1, b, st, 1, 400)  # step-major activation scales
    assert torch.equal(y, y3)


def test_fp4_scale_stepmajor_layout(dev):
    from torchinferno_amd.kernels import block_fp8 as tb
    s = torch.randint(0, 255, (3, 40, 64), dtype=torch.uint8)
    st = tb.fp4_scale_stepmajor(s.to(dev)).cpu()
    assert st.shape == (3, 16, 40, 4)
    assert torch.equal(st, s.view(3, 40, 16, 4).permute(0, 2, 1, 3))


def test_fp4_gemm_one_hot_exact(dev):
    """A single nonzero product at (m=1, n=2, k=37) with block scale 2^3 lands exactly."""
    from torchinferno_amd.kernels import block_fp8 as tb
    m, n, k = 2, 3, 128
    a = torch.zeros((m, k), dtype=torch.uint8)
    a[1, 37] = int(e4m3_encode(np.array([3.0], np.float32))[0])
    codes = np.zeros((n, k), np.uint8)
    codes[2, 37] = 0b1111  # -6
    b_s = torch.full((n, k // 32), 127, dtype=torch.uint8)
    b_s[2, 1] = 130
    y = tb.fp4_gemm(a.to(dev).view(torch.float8_e4m3fn), torch.full((m, 1), 0.25, device=dev),
                    torch.from_numpy(of4.pack_fp4(codes)).to(dev), b_s.to(dev))
    expect = torch.zeros((m, n))
    expect[1, 2] = 3.0 * 0.25 * -6.0 * 8.0
    assert torch.equal(y.float().cpu(), expect)


def test_fp4_scales_as_fp32_powers_of_two(dev):
    from torchinferno_amd.kernels import block_fp8 as tb
    host, (a, a_s, b, b_s) = _inputs(8, 256, 256, 5, dev)
    y1 = tb.fp4_gemm(a, a_s, b, b_s)
    y2 = tb.fp4_gemm(a, a_s, b, b_s.float().contiguous())
    assert torch.equal(y1, y2)
    with pytest.raises(ValueError):
        tb.fp4_gemm(a, a_s, b, (b_s.float() * 1.5).contiguous())


def test_deepseek_linear_fp4_weight(dev):
    """DSv4 ``linear`` with an MXFP4 weight: act_quant + fp4_gemm (tensor_parallel.py:195-207)."""
    import types
    from torchinferno_amd import hooks
    from torchinferno_amd.kernels import block_fp8 as tb
    mod = types.ModuleType("fake_dsv4")
    mod.linear = None
    undo = hooks.patch_deepseek_v4_module(mod)
    try:
        _, (_, _, b, b_s) = _inputs(1, 256, 512, 9, dev)
        w = b.clone()
        w.scale = b_s
        x = torch.randn((3, 4, 512), device=dev).to(torch.bfloat16)
        y = mod.linear(x, w)
        xq, xs = tb.act_quant(x)
        assert y.shape == (3, 4, 256) and torch.equal(y, tb.fp4_gemm(xq, xs, b, b_s))
        ref = omoe.mxfp4_linear(x.float().cpu().numpy().reshape(12, 512), b.view(torch.uint8).cpu().numpy(),
                                b_s.view(torch.uint8).cpu().numpy())
        assert _rel_err(y.float().cpu().numpy().reshape(12, 256), ref) <= TOL
    finally:
        undo()


# --------------------------------------------------------------------------- MoE


def _mxfp4_experts(e, h, inter, seed, dev):
    from torchinferno_amd.kernels import moe as tmoe
    rng = np.random.default_rng(seed)

    def w(n, k):
        return (torch.from_numpy(rng.integers(0, 256, (e, n, k // 2), dtype=np.uint8)).to(dev)
                .view(torch.float4_e2m1fn_x2),
                torch.from_numpy(rng.integers(117, 122, (e, n, k // 32), dtype=np.uint8)).to(dev)
                .view(torch.float8_e8m0fnu))
    (w1, s1), (w3, s3), (w2, s2) = w(inter, h), w(inter, h), w(h, inter)
    return tmoe.prepare_mxfp4_experts(w1, w3, w2, s1, s3, s2)


@pytest.mark.parametrize("t,k", [(1, 1), (9, 2), (64, 4), (300, 8)])
@pytest.mark.parametrize("kind", ["auto", "2", "3", "4", "5", "6", "9", "10", "11", "12", "13", "15", "17", "20"])
def test_mxfp4_moe_matches_oracle(dev, monkeypatch, t, k, kind):
    from torchinferno_amd.kernels import moe as tmoe
    print(f"[fp4] moe T={t} k={k} kind={kind}", flush=True)
    if kind != "auto":
        monkeypatch.setenv("TI_ROCM_MOE_KIND", kind)
    e, h, inter = 8, 256, 256
    ex = _mxfp4_experts(e, h, inter, t * 10 + k, dev)
    g = torch.Generator(device=dev).manual_seed(t)
    x = torch.randn((t, h), generator=g, device=dev).to(torch.bfloat16)
    w, ids = tmoe.route_topk(torch.randn((t, e), generator=g, device=dev), k)
    y = tmoe.fused_mxfp4_moe(x, w, ids, ex)
    def rows(st):  # step-major [K/128, N, 4] -> checkpoint [N, K/32]
        return st.permute(1, 0, 2).reshape(st.size(1), -1).cpu().numpy()
    experts = [(ex.w13[i].cpu().numpy(), rows(ex.w13_scale[i]), ex.w2[i].cpu().numpy(), rows(ex.w2_scale[i]))
               for i in range(e)]
    ref = omoe.moe_reference(x.float().cpu().numpy(), w.cpu().numpy(), ids.cpu().numpy(), experts,
                             linear=omoe.mxfp4_linear)
    assert _rel_err(y.float().cpu().numpy(), ref) <= TOL


def test_mxfp4_moe_tile_boundaries(dev, monkeypatch):
    """MXFP4 experts whose row counts sit on the m-tile boundaries of the two-tier
    plans (128-row first tier, 192- or 256-row second tier) against the single-tier
    128x128 tile (kind 15, to a bf16-rounding bound) and the oracle."""
    from torchinferno_amd.kernels import moe as tmoe
    counts = [0, 1, 128, 129, 192, 193, 255, 256, 257, 321, 385]
    e, h, inter = len(counts), 512, 256
    ex = _mxfp4_experts(e, h, inter, 21, dev)
    ids_np = np.concatenate([np.full(c, i, dtype=np.int32) for i, c in enumerate(counts)])
    np.random.default_rng(5).shuffle(ids_np)
    t = ids_np.size
    g = torch.Generator(device=dev).manual_seed(8)
    x = torch.randn((t, h), generator=g, device=dev).to(torch.bfloat16)
    ids = torch.from_numpy(ids_np).to(dev).view(t, 1)
    w = (torch.rand((t, 1), generator=g, device=dev) + 0.5).float()
    ys = {}
    for plan in ("15", "20/19", "17/18", "17/16"):
        print(f"[fp4] moe tile boundaries plan={plan}", flush=True)
        kind, _, kind2 = plan.partition("/")
        monkeypatch.setenv("TI_ROCM_MOE_KIND", kind)
        monkeypatch.setenv("TI_ROCM_MOE_KIND2", kind2)
        ys[plan] = tmoe.fused_mxfp4_moe(x, w, ids, ex).float().cpu().numpy()

    def rows(st):  # step-major [K/128, N, 4] -> checkpoint [N, K/32]
        return st.permute(1, 0, 2).reshape(st.size(1), -1).cpu().numpy()
    experts = [(ex.w13[i].cpu().numpy(), rows(ex.w13_scale[i]), ex.w2[i].cpu().numpy(), rows(ex.w2_scale[i]))
               for i in range(e)]
    ref = omoe.moe_reference(x.float().cpu().numpy(), w.cpu().numpy(), ids_np.reshape(t, 1), experts,
                             linear=omoe.mxfp4_linear)
    for plan, y in ys.items():
        assert _rel_err(y, ref) <= TOL, plan
        for i, c in enumerate(counts):
            r = ids_np == i
            if r.any():
                assert np.abs(y[r] - ys["15"][r]).max() <= 2 ** -7 * np.abs(ys["15"][r]).max(), (plan, c)
