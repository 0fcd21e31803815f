"""GPU parity of the FP8 path (quantizers and W8A8 GEMMs) against the CPU oracle.

Bar: quantizer codes and scales bit-exact; GEMM max|y - ref| <= 1e-2 * max|ref|
against the fp64-accumulated oracle on the same e4m3 inputs (bf16 output), the
north-star tolerance.  Shapes: BASELINE config 2 (per-token x per-channel,
Llama-3-70B qkv / gate_up / down, M in {1, 64, 512, 4096}) and config 3
(DeepSeek 128x128 blocks, M in {16, 256, 4096}); at full size the oracle checks a
random sample of output rows x columns (an output element depends only on its
row of A and its column of B), fed the exact bytes the GPU used.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle.numerics import bf16_round
from tests._tol import abs_codes, elementwise_ratio

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _codes(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


def _rel_err(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


# --------------------------------------------------------------------------- quantizers


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,k", [(1, 128), (7, 136), (64, 8192), (33, 28672), (512, 28672), (600, 20000),
                                 (1024, 4096), (2048, 9000), (2100, 2056)])
def test_per_token_quant_bit_exact(dev, dtype, m, k):
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator().manual_seed(m * 7 + k)
    x = (torch.randn((m, k), generator=g) * 3).to(dtype)
    xq, xs = tf8.quantize_activation_fp8_per_token(x.to(dev))
    oq, os_ = ofp8.quantize_activation_per_token(x.float().numpy())
    assert np.array_equal(_codes(xq), oq)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), os_.view(np.uint32))


@pytest.mark.parametrize("m", [1, 300])
@pytest.mark.parametrize("amax", [672.0, 784.0, 840.0, 448.0 * 1.3, 448.0 * 0.7])
def test_per_token_quant_e4m3_midpoints(dev, m, amax):
    """Quotients on and next to e4m3 rounding midpoints, where a reciprocal product
    and the IEEE quotient can round to different codes: every e4m3 midpoint times
    the row scale, and its bf16 neighbours.  With amax 672 / 784 / 840 the scale is
    1.5 / 1.75 / 1.875, every such product is exact in bf16 and every quotient an
    exact tie; for 1.75 and 1.875, fl(x * fl(1/s)) lands one ulp above many of
    those ties, so a plain reciprocal product would round them up."""
    from torchinferno_amd.kernels import fp8 as tf8
    codes = np.arange(1, 0x7E, dtype=np.uint8)
    vals = ofp8.e4m3_decode(codes).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    amax = float(torch.tensor(amax).to(torch.bfloat16))
    sc = np.float32(np.float32(amax) / np.float32(448.0))
    base = torch.tensor(np.concatenate([mids, -mids]) * float(sc), dtype=torch.float32).to(torch.bfloat16)
    bits = base.view(torch.int16)
    row = torch.cat([base, (bits + 1).view(torch.bfloat16), (bits - 1).view(torch.bfloat16)])
    row = torch.cat([row, torch.tensor([amax], dtype=torch.bfloat16)])
    k = -(-row.numel() // 8) * 8
    x = torch.zeros((m, k), dtype=torch.bfloat16)
    x[:, :row.numel()] = row
    assert float(x.abs().max()) == float(torch.tensor(amax).to(torch.bfloat16))
    xq, xs = tf8.quantize_activation_fp8_per_token(x.to(dev))
    oq, os_ = ofp8.quantize_activation_per_token(x.float().numpy())
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(_codes(xq), oq)


@pytest.mark.parametrize("round_scale", [False, True])
@pytest.mark.parametrize("amax", [672.0, 784.0, 840.0, 448.0 * 1.3])
def test_block_act_quant_e4m3_midpoints(dev, round_scale, amax):
    """The 1x128 quant on quotients at and next to e4m3 midpoints (as the per-token
    test above): each 128-wide block holds its amax and 127 such values."""
    from torchinferno_amd.kernels import block_fp8 as tb
    codes = np.arange(1, 0x7E, dtype=np.uint8)
    vals = ofp8.e4m3_decode(codes).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    amax = float(torch.tensor(amax).to(torch.bfloat16))
    sc = np.float32(np.float32(amax) * np.float32(1.0 / 448.0))
    base = torch.tensor(np.concatenate([mids, -mids]) * float(sc), dtype=torch.float32).to(torch.bfloat16)
    bits = base.view(torch.int16)
    vals_all = torch.cat([base, (bits + 1).view(torch.bfloat16), (bits - 1).view(torch.bfloat16)])
    nblk = -(-vals_all.numel() // 127)
    x = torch.zeros((nblk, 128), dtype=torch.bfloat16)
    flat = torch.zeros(nblk * 127, dtype=torch.bfloat16)
    flat[:vals_all.numel()] = vals_all
    x[:, :127] = flat.view(nblk, 127)
    x[:, 127] = amax
    x = x.reshape(1, -1).repeat(3, 1)
    xq, xs = tb.act_quant(x.to(dev), 128, "ue8m0" if round_scale else None)
    oq, os_ = ofp8.act_quant_block(x.float().numpy(), round_scale=round_scale)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(_codes(xq), oq)


def test_per_token_quant_zero_row_uses_eps(dev):
    from torchinferno_amd.kernels import fp8 as tf8
    x = torch.zeros((2, 256), dtype=torch.bfloat16, device=dev)
    x[1, 3] = 1.0
    xq, xs = tf8.quantize_activation_fp8_per_token(x)
    assert xs[0, 0].item() == np.float32(1e-10)
    assert int(xq.view(torch.uint8)[1, 3]) == 0x7E  # the row max encodes as 448


def test_per_channel_weight_quant_bit_exact(dev):
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator().manual_seed(16)
    w = (torch.randn((300, 1024), generator=g) * 0.02).to(torch.bfloat16)
    wq, ws = tf8.quantize_weight_fp8_per_channel(w.to(dev))
    oq, os_ = ofp8.quantize_weight_fp8_per_channel(w.float().numpy())
    assert ws.shape == (1, 300)
    assert np.array_equal(_codes(wq), oq)
    assert np.array_equal(ws.cpu().numpy(), os_)


@pytest.mark.parametrize("round_scale", [False, True])
@pytest.mark.parametrize("m,k", [(1, 128), (3, 640), (5, 7168), (64, 18432)])
def test_block_act_quant_bit_exact(dev, round_scale, m, k):
    from torchinferno_amd.kernels import block_fp8 as tb
    g = torch.Generator().manual_seed(k + m)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    x[0, :128] = 0  # an all-zero block takes the 1e-4 floor
    y, s = tb.act_quant(x.to(dev), 128, "ue8m0" if round_scale else None)
    oq, os_ = ofp8.act_quant_block(x.float().numpy(), 128, round_scale)
    assert np.array_equal(_codes(y), oq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))


@pytest.mark.parametrize("shift", [2, 8])
def test_block_act_quant_unaligned_input(dev, shift):
    """An input that starts 4 bytes past a 16-byte boundary takes the 4-byte-access kernel,
    16 bytes past one the 16-byte kernel; both give the oracle's codes and scales."""
    from torchinferno_amd.kernels import block_fp8 as tb
    m, k = 7, 896
    g = torch.Generator().manual_seed(shift)
    flat = (torch.randn(m * k + shift, generator=g) * 2).to(torch.bfloat16)
    xd = flat.to(dev)[shift:].view(m, k)
    assert (xd.data_ptr() % 16 != 0) == (shift == 2)
    y, s = tb.act_quant(xd)
    oq, os_ = ofp8.act_quant_block(flat[shift:].view(m, k).float().numpy())
    assert np.array_equal(_codes(y), oq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))


@pytest.mark.parametrize("m", [1, 77, 300])
def test_block_act_quant_stepmajor_layout(dev, m):
    """Scale layout 1 writes the same scales transposed, [K/128, M], and the same codes."""
    from torchinferno_amd.kernels import block_fp8 as tb
    x = (torch.randn((m, 1024), generator=torch.Generator().manual_seed(m)) * 3).to(torch.bfloat16).to(dev)
    y, s = tb.act_quant(x)
    y_t, s_t = tb._act_quant_stepmajor(x)
    assert s_t.shape == (8, m)
    assert torch.equal(y.view(torch.uint8), y_t.view(torch.uint8))
    assert torch.equal(s.t(), s_t)


def test_block_linear_stepmajor_matches_public_path(dev):
    """The DSv4 linear (step-major scales inside) equals act_quant + fp8_gemm bit for bit."""
    from torchinferno_amd.kernels import block_fp8 as tb
    a, a_s, b, b_s = _problem_block(1, 1024, 384, 5, dev)
    x = (torch.randn((3, 70, 1024), generator=torch.Generator().manual_seed(2))).to(torch.bfloat16).to(dev)
    xq, xs = tb.act_quant(x)
    ref = tb.fp8_gemm(xq, xs, b, b_s)
    got = tb.linear(x, b, b_s)
    assert got.shape == (3, 70, 384) and torch.equal(got, ref)
    empty = tb.linear(x[:, :0], b, b_s)
    assert empty.shape == (3, 0, 384)


def test_block_act_quant_inplace_round_trip(dev):
    from torchinferno_amd.kernels import block_fp8 as tb
    g = torch.Generator().manual_seed(5)
    x = torch.randn((4, 256), generator=g).to(torch.bfloat16)
    xd = x.to(dev)
    r = tb.act_quant(xd, inplace=True)
    assert r is xd
    oq, os_ = ofp8.act_quant_block(x.float().numpy())
    deq = ofp8.dequantize_block_fp8(oq, np.ones((1, 2), np.float32)) * np.repeat(os_, 128, 1)
    assert np.array_equal(xd.float().cpu().numpy(), bf16_round(deq))


def test_tensor_quant_bit_exact(dev):
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator().manual_seed(15)
    x = torch.randn((32, 128), generator=g).to(torch.bfloat16)
    sc = np.float32(np.abs(x.float().numpy()).max() / np.float32(448.0))
    inv = np.float32(np.float32(1.0) / sc)
    xq, s = tf8.quantize_activation_fp8(x.to(dev), scale=torch.tensor(sc, device=dev),
                                        inverse_scale=torch.tensor(inv, device=dev))
    oq, _ = ofp8.quantize_activation_tensor(x.float().numpy(), sc)
    assert np.array_equal(_codes(xq), oq)


def _all_positive(dtype):
    top = 0x7F80 if dtype == torch.bfloat16 else 0x7C00
    return torch.arange(1, top, dtype=torch.int32).to(torch.int16).view(dtype)


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "fp16")])
def test_tensor_scale_rule_is_torch_on_gpu(dev, dtype, name):
    """Pins oracle.fp8.tensor_scale against torch's own evaluation of fp8.py:125 on the
    GPU (the reference runs it on its weight's / activation's device) for every finite
    positive amax of the dtype, and the per-channel rule (fp8.py:131-134, fp32) for every
    bf16 amax: torch turns division by a host scalar into a reciprocal multiply."""
    v = _all_positive(dtype).to(dev)
    gpu = (v / 448.0).clamp(min=1e-6).to(torch.float32).cpu().numpy()
    orc = np.array([ofp8.tensor_scale(a, name) for a in v.float().cpu().numpy()], np.float32)
    assert np.array_equal(gpu.view(np.uint32), orc.view(np.uint32))
    if dtype == torch.bfloat16:
        w = torch.zeros((v.numel(), 8), dtype=dtype, device=dev)
        w[:, 3] = -v
        ch = (w.abs().amax(dim=1, keepdim=True).to(torch.float32) / 448.0).clamp(min=1e-10)
        _, os_ = ofp8.quantize_weight_fp8_per_channel(w.float().cpu().numpy())
        assert np.array_equal(ch.cpu().numpy()[:, 0].view(np.uint32), os_[0].view(np.uint32))


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "fp16")])
@pytest.mark.parametrize("scale", [0.02, 1.0, 2e-6])
def test_tensorwise_weight_quant_bit_exact(dev, dtype, name, scale):
    """quantize_weight_fp8 (fp8.py:119-126): scale and codes equal the oracle."""
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator().manual_seed(int(scale * 1e6) + 3)
    w = (torch.randn((257, 384), generator=g) * scale).to(dtype)
    wq, ws = tf8.quantize_weight_fp8(w.to(dev))
    oq, os_ = ofp8.quantize_weight_fp8(w.float().numpy(), name)
    assert ws.dtype == torch.float32 and ws.item() == os_
    assert np.array_equal(_codes(wq), oq)


@pytest.mark.parametrize("dtype,name", [(torch.bfloat16, "bf16"), (torch.float16, "fp16")])
@pytest.mark.parametrize("m,k,scale", [(1, 128, 1.0), (32, 128, 1.0), (300, 1000, 7.0), (64, 8192, 1e-3)])
def test_dynamic_tensor_activation_quant_bit_exact(dev, dtype, name, m, k, scale):
    """quantize_activation_fp8(x) with scale=None (fp8.py:141-181): the dynamic scale and
    the codes equal the oracle bit for bit."""
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator().manual_seed(m + k)
    x = (torch.randn((m, k), generator=g) * scale).to(dtype)
    xq, xs = tf8.quantize_activation_fp8(x.to(dev))
    oq, os_ = ofp8.quantize_activation_tensor(x.float().numpy(), None, name)
    assert xs.item() == os_
    assert np.array_equal(_codes(xq), oq)


def test_block_act_quant_unaligned_output(dev):
    """A 16-byte aligned input with an output only 2-byte aligned (a C caller's carved
    buffer) takes the 4-byte-access kernel; codes and scales equal the oracle."""
    from torchinferno_amd import _lib
    m, k = 5, 640
    g = torch.Generator().manual_seed(11)
    x = (torch.randn((m, k), generator=g) * 2).to(torch.bfloat16)
    xd = x.to(dev)
    buf = torch.zeros(m * k + 16, dtype=torch.uint8, device=dev)
    xq = buf[2:2 + m * k]
    assert xd.data_ptr() % 16 == 0 and xq.data_ptr() % 8 == 2
    xs = torch.empty((m, k // 128), dtype=torch.float32, device=dev)
    _lib.call("ti_fp8_quant_block", xd.data_ptr(), _lib.dtype_code(xd.dtype), m, k, 128, 0,
              xq.data_ptr(), xs.data_ptr(), 0, _lib.stream_of(xd))
    oq, os_ = ofp8.act_quant_block(x.float().numpy())
    assert np.array_equal(xq.view(m, k).cpu().numpy(), oq)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    assert int(buf[:2].sum()) == 0 and int(buf[2 + m * k:].sum()) == 0


def test_static_activation_scale_reference_case(dev):
    """tests/test_conversion_and_kernels.py:186-205: a reusable static scale (4x margin)
    and its inverse; the op writes the caller's buffer, returns the caller's scale,
    and restores within atol 6e-2 / rtol 1.3e-1."""
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator(device=dev).manual_seed(15)
    values = torch.randn((32, 128), generator=g, device=dev).to(torch.bfloat16)
    scale = (values.abs().amax() / tf8.FP8_E4M3_MAX).clamp(min=1e-6).float() * 4.0
    inverse_scale = scale.reciprocal()
    output = torch.empty_like(values, dtype=torch.float8_e4m3fn)
    quantized, returned_scale = tf8.quantize_activation_fp8(values, scale=scale, inverse_scale=inverse_scale,
                                                            out=output)
    assert quantized is output
    assert returned_scale.data_ptr() == scale.data_ptr()
    restored = quantized.to(torch.bfloat16) * scale
    torch.testing.assert_close(restored, values, atol=6e-2, rtol=1.3e-1)


def test_per_token_linear_reference_case(dev):
    """tests/test_conversion_and_kernels.py:364-387: K=64 (not a multiple of 128),
    caller-owned out, within atol 1.0 / rtol 0.15 of F.linear."""
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator(device=dev).manual_seed(19)
    values = torch.randn((17, 64), generator=g, device=dev).to(torch.bfloat16)
    weight = torch.randn((32, 64), generator=g, device=dev).to(torch.bfloat16)
    weight_q, weight_scale = tf8.quantize_weight_fp8_per_channel(weight)
    output = torch.empty((17, 32), device=dev, dtype=torch.bfloat16)
    projected = tf8.fp8_per_token_linear(values, weight_q, weight_scale, out=output, use_fast_accum=True)
    assert projected is output
    reference = torch.nn.functional.linear(values, weight)
    torch.testing.assert_close(projected, reference, atol=1.0, rtol=0.15)
    xq, xs = tf8.quantize_activation_fp8_per_token(values)
    ref = ofp8.fp8_linear_rowcol(_codes(xq), xs.cpu().numpy(), _codes(weight_q), weight_scale.cpu().numpy())
    assert _rel_err(projected.float().cpu().numpy(), ref) <= TOL


# --------------------------------------------------------------------------- GEMM helpers


def _problem_rowcol(m, k, n, seed, dev):
    """Config 2 scheme on the GPU: W ~ N(0, 0.02) per-channel, x ~ N(0,1) per-token."""
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator(device=dev).manual_seed(seed)
    w = (torch.randn((n, k), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    wq, ws = tf8.quantize_weight_fp8_per_channel(w)
    del w
    xq, xs = tf8.quantize_activation_fp8_per_token(x)
    return x, xq, xs, wq, ws


def _sample(total, cap, rng):
    if total <= cap:
        return np.arange(total)
    return np.sort(rng.choice(total, cap, replace=False))


def _check_rowcol(out, xq, xs, wq, ws, rng, rows_cap=64, cols_cap=512):
    rows = _sample(out.shape[0], rows_cap, rng)
    cols = _sample(out.shape[1], cols_cap, rng)
    ri = torch.as_tensor(rows, device=out.device)
    ci = torch.as_tensor(cols, device=out.device)
    a, b = _codes(xq[ri]), _codes(wq[ci])
    sa, sb = xs[ri].cpu().numpy(), ws[:, ci].cpu().numpy()
    ref = ofp8.fp8_linear_rowcol(a, sa, b, sb)
    got = out[ri][:, ci].float().cpu().numpy()
    # elementwise: 1 ulp of the 16-bit output + 2^-16 of the sum of |terms|
    ulps = 1.0 if out.dtype == torch.bfloat16 else 1.0 / 8  # fp16 ulp = bf16 ulp / 8
    ratio = elementwise_ratio(got, ref, ofp8.fp8_linear_rowcol(abs_codes(a), sa, abs_codes(b), sb), ulps)
    assert ratio <= 1.0, ratio
    return _rel_err(got, ref)


# --------------------------------------------------------------------------- config 2


@pytest.mark.parametrize("k,n", [(8192, 10240), (8192, 57344), (28672, 8192)])
@pytest.mark.parametrize("m", [1, 64, 512, 4096])
def test_config2_per_token_linear(dev, m, k, n):
    from torchinferno_amd.kernels import fp8 as tf8
    print(f"[fp8] config2 M={m} K={k} N={n}", flush=True)
    x, xq, xs, wq, ws = _problem_rowcol(m, k, n, 2, dev)
    out = tf8.fp8_per_token_linear(x, wq, ws)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == (m, n)
    err = _check_rowcol(out, xq, xs, wq, ws, np.random.default_rng(m + n))
    assert err <= TOL, err


@pytest.mark.parametrize("m", [1, 3, 17, 40, 64, 100, 129, 300])
@pytest.mark.parametrize("n", [96, 640, 4112])
def test_rowcol_ragged(dev, m, n):
    """Ragged M and N (partial tiles in both directions, split-K at small M)."""
    from torchinferno_amd.kernels import fp8 as tf8
    print(f"[fp8] ragged M={m} N={n}", flush=True)
    x, xq, xs, wq, ws = _problem_rowcol(m, 1024, n, 50 + m, dev)
    out = tf8.fp8_per_token_linear_quantized(xq, xs, wq, ws, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    err = _check_rowcol(out, xq, xs, wq, ws, np.random.default_rng(1), rows_cap=10**9, cols_cap=10**9)
    assert err <= TOL, err


@pytest.mark.parametrize("kind", range(24))
@pytest.mark.parametrize("mode", ["rowcol", "block"])
def test_every_tile_kind(dev, monkeypatch, kind, mode):
    """Each tile configuration, forced, on a ragged problem, with and without split-K."""
    from torchinferno_amd.kernels import block_fp8 as tb
    from torchinferno_amd.kernels import fp8 as tf8
    for splits in ("1", "3"):
        print(f"[fp8] kind {kind} {mode} splits={splits}", flush=True)
        monkeypatch.setenv("TI_ROCM_FP8_KIND", str(kind))
        monkeypatch.setenv("TI_ROCM_FP8_SPLITS", splits)
        m, k, n = 200, 1280, 400
        if mode == "rowcol":
            x, xq, xs, wq, ws = _problem_rowcol(m, k, n, 7 + kind, dev)
            out = tf8.fp8_per_token_linear_quantized(xq, xs, wq, ws, out_dtype=torch.float16)
            torch.cuda.synchronize()
            assert out.dtype == torch.float16
            err = _check_rowcol(out, xq, xs, wq, ws, np.random.default_rng(0), 10**9, 10**9)
        else:
            a, a_s, b, b_s = _problem_block(m, k, n, 9 + kind, dev)
            out = tb.fp8_gemm(a, a_s, b, b_s)
            torch.cuda.synchronize()
            err = _check_block(out, a, a_s, b, b_s, np.random.default_rng(0), 10**9, 10**9)
            # step-major activation scales [K/128, M]: same products, same order
            out_t = tb._fp8_gemm_raw(a, a_s.t().contiguous(), 1, b, b_s)
            assert torch.equal(out, out_t), (kind, splits)
        assert err <= TOL, (kind, mode, splits, err)


def test_prefill_linear_tensorwise(dev):
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator(device=dev).manual_seed(19)
    w = (torch.randn((1024, 2048), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((300, 2048), generator=g, device=dev).to(torch.bfloat16)
    wq, wsc = tf8.quantize_weight_fp8(w)
    out = tf8.fp8_prefill_linear(x.view(3, 100, 2048), wq, wsc)
    assert out.shape == (3, 100, 1024) and out.dtype == torch.bfloat16
    xq, xsc = tf8.quantize_activation_fp8(x)
    ref = ofp8.fp8_linear_rowcol(_codes(xq), np.float32(xsc.item()), _codes(wq), np.float32(wsc.item()))
    assert _rel_err(out.view(300, 1024).float().cpu().numpy(), ref) <= TOL
    # and against the unquantized product, the reference test's looser bound
    # (tests/test_conversion_and_kernels.py:364-387: atol 1.0, rtol 0.15)
    torch.testing.assert_close(out.view(300, 1024).float(), (x.float() @ w.float().t()), atol=1.0, rtol=0.15)


def test_out_buffer_contract(dev):
    """Caller-owned out is written in place and returned (fp8.py:285-327)."""
    from torchinferno_amd.kernels import fp8 as tf8
    x, xq, xs, wq, ws = _problem_rowcol(48, 1024, 512, 3, dev)
    out = torch.empty((48, 512), dtype=torch.bfloat16, device=dev)
    ptr = out.data_ptr()
    r = tf8.fp8_per_token_linear(x, wq, ws, out=out)
    assert r is out and out.data_ptr() == ptr
    with pytest.raises(ValueError):
        tf8.fp8_per_token_linear(x, wq, ws, out=torch.empty((48, 512), dtype=torch.float16, device=dev))
    with pytest.raises(ValueError):
        tf8.fp8_per_token_linear(x, wq, ws[:, :10])
    # Deterministic: a second call (split-K at M=48) gives identical bits.
    r2 = tf8.fp8_per_token_linear(x, wq, ws)
    assert torch.equal(r2, out)


def test_scaled_mm_out_region(dev):
    from torchinferno_amd.kernels import fp8 as tf8
    x, xq, xs, wq, ws = _problem_rowcol(16, 1024, 256, 4, dev)
    out = torch.empty((16, 256), dtype=torch.bfloat16, device=dev)
    assert tf8.scaled_mm_out(out, xq, wq.t(), xs, ws) is out
    ref = tf8.fp8_per_token_linear_quantized(xq, xs, wq, ws, out_dtype=torch.bfloat16)
    assert torch.equal(out, ref)
    # Outside the region -> None (row-major b, K not a multiple of 128).
    assert tf8.scaled_mm_out(out, xq, wq.t().contiguous(), xs, ws) is None
    assert tf8.scaled_mm_out(out[:, :200], xq, wq[:200].t(), xs, ws[:, :200]) is None


# --------------------------------------------------------------------------- config 3


def _problem_block(m, k, n, seed, dev):
    """Config 3 scheme: W ~ N(0,0.02) -> 128x128 blocks (s = block absmax/448), x ~ N(0,1)
    -> 1x128 (act_quant).  The weight quant is the benchmark definition's formula in torch."""
    from torchinferno_amd.kernels import block_fp8 as tb
    g = torch.Generator(device=dev).manual_seed(seed)
    w = torch.randn((n, k), generator=g, device=dev) * 0.02
    nb, kb = -(-n // 128), k // 128
    wp = torch.zeros((nb * 128, k), device=dev)
    wp[:n] = w
    blocks = wp.view(nb, 128, kb, 128)
    amax = blocks.abs().amax(dim=(1, 3))
    b_s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax)).float().contiguous()
    b = (blocks / b_s[:, None, :, None]).view(nb * 128, k)[:n].to(torch.float8_e4m3fn).contiguous()
    del w, wp, blocks
    x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    a, a_s = tb.act_quant(x)
    return a, a_s, b, b_s


def _check_block(out, a, a_s, b, b_s, rng, rows_cap=32, cols_cap=384):
    rows = _sample(out.shape[0], rows_cap, rng)
    cols = _sample(out.shape[1], cols_cap, rng)
    ri = torch.as_tensor(rows, device=out.device)
    ci = torch.as_tensor(cols, device=out.device)
    # the oracle takes b_s per 128-row block: expand to the sampled columns' blocks
    bs_rows = b_s.cpu().numpy()[cols // 128]                     # [ncols, K/128]
    b_sub = _codes(b[ci])
    a_sub = _codes(a[ri])
    ref = np.zeros((len(rows), len(cols)), np.float32)
    ref_abs = np.zeros_like(ref)
    # one oracle call per distinct column block (its b_s row applies to all its columns)
    for blk in np.unique(cols // 128):
        sel = np.nonzero(cols // 128 == blk)[0]
        ref[:, sel] = ofp8.fp8_gemm_block(a_sub, a_s[ri].cpu().numpy(), b_sub[sel],
                                          bs_rows[sel[:1]].reshape(1, -1))
        ref_abs[:, sel] = ofp8.fp8_gemm_block(abs_codes(a_sub), a_s[ri].cpu().numpy(), abs_codes(b_sub[sel]),
                                              bs_rows[sel[:1]].reshape(1, -1))
    got = out[ri][:, ci].float().cpu().numpy()
    ratio = elementwise_ratio(got, ref, ref_abs)
    assert ratio <= 1.0, ratio
    return _rel_err(got, ref)


@pytest.mark.parametrize("k,n", [(7168, 18432), (18432, 7168), (7168, 24576)])
@pytest.mark.parametrize("m", [16, 256, 4096])
def test_config3_block_gemm(dev, m, k, n):
    from torchinferno_amd.kernels import block_fp8 as tb
    print(f"[fp8] config3 M={m} K={k} N={n}", flush=True)
    a, a_s, b, b_s = _problem_block(m, k, n, 3, dev)
    out = tb.fp8_gemm(a, a_s, b, b_s)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == (m, n)
    err = _check_block(out, a, a_s, b, b_s, np.random.default_rng(m + k))
    assert err <= TOL, err


@pytest.mark.parametrize("m", [1, 5, 31, 77, 200])
def test_block_gemm_ragged(dev, m):
    from torchinferno_amd.kernels import block_fp8 as tb
    print(f"[fp8] block ragged M={m}", flush=True)
    a, a_s, b, b_s = _problem_block(m, 896, 333, 40 + m, dev)  # N=333: partial last block
    out = tb.fp8_gemm(a, a_s, b, b_s)
    torch.cuda.synchronize()
    err = _check_block(out, a, a_s, b, b_s, np.random.default_rng(2), 10**9, 10**9)
    assert err <= TOL, err


def test_block_linear_3d_input(dev):
    from torchinferno_amd.kernels import block_fp8 as tb
    a, a_s, b, b_s = _problem_block(24, 512, 256, 6, dev)
    g = torch.Generator(device=dev).manual_seed(8)
    x = torch.randn((2, 12, 512), generator=g, device=dev).to(torch.bfloat16)
    y = tb.linear(x, b, b_s)
    assert y.shape == (2, 12, 256)
    xq, xs = tb.act_quant(x.view(24, 512))
    assert torch.equal(y.view(24, 256), tb.fp8_gemm(xq, xs, b, b_s))


# --------------------------------------------------------------------------- tiled weights


def test_tile_weight_layout(dev):
    """ti_fp8_tile_weight: block (n // 128, k // 128), row n % 128, byte k % 128."""
    from torchinferno_amd.kernels import fp8 as tf8
    n, k = 384, 640
    codes = torch.randint(0, 256, (n, k), dtype=torch.uint8, device=dev)
    t = tf8.tile_weight_fp8(codes.view(torch.float8_e4m3fn))
    assert t.shape == (n // 128, k // 128, 128, 128) and tf8.is_tiled_weight(t)
    assert tf8.weight_nk(t) == (n, k)
    c = codes.cpu().numpy()
    expect = c.reshape(n // 128, 128, k // 128, 128).transpose(0, 2, 1, 3)
    assert np.array_equal(t.view(torch.uint8).cpu().numpy(), expect)
    with pytest.raises(ValueError):
        tf8.tile_weight_fp8(codes[:200].view(torch.float8_e4m3fn))


@pytest.mark.parametrize("m", [1, 16, 64, 200, 512])
def test_tiled_weight_gemm_equals_row_layout(dev, m):
    """The tiled weight gives the same bits as the [N, K] weight (same tiles, same
    MFMA order), and the oracle's bound."""
    from torchinferno_amd.kernels import fp8 as tf8
    print(f"[fp8] tiled weight M={m}", flush=True)
    x, xq, xs, wq, ws = _problem_rowcol(m, 1280, 640, 60 + m, dev)
    wt = tf8.tile_weight_fp8(wq)
    y = tf8.fp8_per_token_linear_quantized(xq, xs, wq, ws, out_dtype=torch.bfloat16)
    yt = tf8.fp8_per_token_linear_quantized(xq, xs, wt, ws, out_dtype=torch.bfloat16)
    assert torch.equal(y, yt)
    assert torch.equal(tf8.fp8_per_token_linear(x, wt, ws), tf8.fp8_per_token_linear(x, wq, ws))
    err = _check_rowcol(yt, xq, xs, wq, ws, np.random.default_rng(2))
    assert err <= TOL


@pytest.mark.parametrize("kind", [k for k in range(24) if k not in (0, 7, 8)])
def test_tiled_weight_every_kind(dev, monkeypatch, kind):
    """Every 128-K-step tile kind (the 64-K-step kinds run kind 1 on tiled weights),
    with and without split-K, on a ragged M: tiled equals row layout."""
    from torchinferno_amd.kernels import fp8 as tf8
    x, xq, xs, wq, ws = _problem_rowcol(200, 1280, 512, 80 + kind, dev)
    wt = tf8.tile_weight_fp8(wq)
    for splits in ("1", "3"):
        monkeypatch.setenv("TI_ROCM_FP8_KIND", str(kind))
        monkeypatch.setenv("TI_ROCM_FP8_SPLITS", splits)
        y = tf8.fp8_per_token_linear_quantized(xq, xs, wq, ws, out_dtype=torch.bfloat16)
        yt = tf8.fp8_per_token_linear_quantized(xq, xs, wt, ws, out_dtype=torch.bfloat16)
        assert torch.equal(y, yt), (kind, splits)


def test_prefill_linear_tiled_weight(dev):
    from torchinferno_amd.kernels import fp8 as tf8
    g = torch.Generator(device=dev).manual_seed(9)
    w = (torch.randn((256, 512), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((40, 512), generator=g, device=dev).to(torch.bfloat16)
    wq, sw = tf8.quantize_weight_fp8(w)
    y = tf8.fp8_prefill_linear(x, wq, sw)
    yt = tf8.fp8_prefill_linear(x, tf8.tile_weight_fp8(wq), sw)
    assert torch.equal(y, yt)
