"""Pins oracle/fp8.py (CPU, no GPU): the reference's known answers and restore
tolerances, closed forms of the scale rules, and GEMM identities that a dropped
scale, a transposed operand or a wrong block index would break."""
import numpy as np
import torch

from oracle import fp8 as ofp8
from oracle.numerics import e4m3_decode, e4m3_encode

F32 = np.float32


def test_block_dequant_reference_known_answer():
    """tests/test_deepseek_v4.py:546-552: [[1,-2],[3,4]] e4m3 with scale 2 -> [[2,-4],[6,8]]."""
    codes = e4m3_encode(np.array([[1.0, -2.0], [3.0, 4.0]], F32))
    out = ofp8.dequantize_block_fp8(codes, np.array([[2.0]], F32))
    assert np.array_equal(out, np.array([[2.0, -4.0], [6.0, 8.0]], F32))


def test_block_dequant_uses_each_blocks_scale():
    codes = np.full((200, 300), e4m3_encode(np.array([1.0], F32))[0], np.uint8)
    scale = np.arange(1, 7, dtype=F32).reshape(2, 3)
    out = ofp8.dequantize_block_fp8(codes, scale)
    assert out[0, 0] == 1 and out[0, 128] == 2 and out[0, 299] == 3
    assert out[199, 0] == 4 and out[128, 256] == 6


def test_per_channel_weight_quant_reference_tolerance():
    """tests/test_conversion_and_kernels.py:208-220 (seed 16, [7, 13])."""
    torch.manual_seed(16)
    w = torch.randn((7, 13), dtype=torch.bfloat16).float().numpy()
    q, s = ofp8.quantize_weight_fp8_per_channel(w)
    assert q.shape == (7, 13) and s.shape == (1, 7)
    restored = e4m3_decode(q) * s.T
    np.testing.assert_allclose(restored, w, atol=1.2e-1, rtol=1.3e-1)


def test_per_channel_scale_closed_form():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((5, 64)).astype(F32)
    q, s = ofp8.quantize_weight_fp8_per_channel(w)
    amax = np.abs(w).max(1)
    # the reciprocal product lies within one ulp of the quotient
    assert np.all(np.abs(s[0].astype(np.float64) - amax / 448.0) <= np.spacing(s[0]))
    np.testing.assert_array_equal(s[0], (amax * (F32(1) / F32(448))).astype(F32))
    # each row's absmax element encodes as +-448 (code 0x7E / 0xFE)
    idx = np.abs(w).argmax(1)
    assert all((q[r, idx[r]] & 0x7F) == 0x7E for r in range(5))
    # codes: torch's own cast of w / s on the host (library cast)
    wt = torch.from_numpy(w)
    assert np.array_equal((wt / torch.from_numpy(s.T.copy())).to(torch.float8_e4m3fn).view(torch.uint8).numpy(), q)


def _all_positive(dtype):
    top = 0x7F80 if dtype == torch.bfloat16 else 0x7C00
    return torch.arange(1, top, dtype=torch.int32).to(torch.int16).view(dtype)


def test_tensor_scale_bf16_exhaustive_vs_torch():
    """fp8.py:125 evaluated by torch on every finite positive bf16 amax: the scale is
    rounded to bf16 before the clamp and the fp32 cast.  (For bf16 the quotient and
    the reciprocal product round to the same bf16 for every input, so torch's host
    division pins the oracle here exactly.)"""
    v = _all_positive(torch.bfloat16)
    want = (v / 448.0).clamp(min=1e-6).to(torch.float32).numpy()
    got = np.array([ofp8.tensor_scale(a, "bf16") for a in v.float().numpy()], F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_tensor_scale_fp16_vs_torch_host():
    """Every finite positive fp16 amax: the oracle equals torch's host expression except
    where the fp16-rounded quotient and reciprocal product differ -- there it takes the
    product, the GPU's rule (pinned on the device in tests/test_fp8_gpu.py)."""
    v = _all_positive(torch.float16)
    host = (v / 448.0).clamp(min=1e-6).to(torch.float32).numpy()
    got = np.array([ofp8.tensor_scale(a, "fp16") for a in v.float().numpy()], F32)
    f = v.float()
    quot = (f / 448.0).half()
    prod = (f * (torch.tensor(1.0) / torch.tensor(448.0))).half()
    split = (quot != prod).numpy()
    assert 0 < split.sum() < 100
    assert np.array_equal(got[~split], host[~split])
    assert np.array_equal(got[split], prod.clamp(min=1e-6).float().numpy()[split])


def test_tensor_scale_is_not_fp32_arithmetic():
    """A fp32 scale (no rounding to the input dtype) is the plausible mistake: on this
    bf16 amax it gives 0.02748326, the reference's arithmetic 0.02746582."""
    amax = F32(12.3125)  # a bf16 value
    assert ofp8.tensor_scale(amax, "bf16") == F32(0.02746582)
    assert F32(amax / F32(448)) != ofp8.tensor_scale(amax, "bf16")
    assert ofp8.tensor_scale(F32(1e-7), "bf16") == torch.tensor(1e-6, dtype=torch.bfloat16).float().item()


def test_tensorwise_weight_quant_vs_torch_host():
    """quantize_weight_fp8 (fp8.py:119-126) on seeded bf16 weights: scale and codes equal
    torch's own expression (bf16 amax/448 -> clamp -> fp32; fp32 quotient -> e4m3)."""
    g = torch.Generator().manual_seed(7)
    for scale in (0.02, 1.0, 3e-5):
        w = (torch.randn((48, 80), generator=g) * scale).to(torch.bfloat16)
        ws = (w.abs().amax() / 448.0).clamp(min=1e-6).to(torch.float32)
        wq = (w.to(torch.float32) / ws).to(torch.float8_e4m3fn)
        q, s = ofp8.quantize_weight_fp8(w.float().numpy(), "bf16")
        assert s == ws.item()
        assert np.array_equal(q, wq.view(torch.uint8).numpy())


def test_dynamic_tensor_activation_quant_vs_torch_host():
    """quantize_activation_fp8(x) with scale=None (fp8.py:154-155, cast kernel :43-51):
    bf16 and fp16 inputs, scale and codes vs torch's expression on the host."""
    g = torch.Generator().manual_seed(8)
    for dt, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16")):
        x = (torch.randn((33, 96), generator=g) * 5).to(dt)
        sc = (x.abs().amax() / 448.0).clamp(min=1e-6).to(torch.float32)
        inv = sc.reciprocal()
        want = (x.to(torch.float32) * inv).to(torch.float8_e4m3fn)
        q, s = ofp8.quantize_activation_tensor(x.float().numpy(), None, name)
        assert s == sc.item()
        assert np.array_equal(q, want.view(torch.uint8).numpy())


def test_per_token_zero_row_floor():
    x = np.zeros((2, 16), F32)
    x[1, 0] = 3.0
    q, s = ofp8.quantize_activation_per_token(x)
    assert s[0, 0] == F32(1e-10) and s[1, 0] == F32(3.0) / F32(448)
    assert q[0].max() == 0 and q[1, 0] == 0x7E


def test_static_activation_scale_reference_tolerance():
    """tests/test_conversion_and_kernels.py:186-205 (seed 15, [32,128], 4x margin)."""
    torch.manual_seed(15)
    x = torch.randn((32, 128), dtype=torch.bfloat16).float().numpy()
    sc = F32(max(np.abs(x).max() / F32(448), F32(1e-6)) * F32(4))
    q, s = ofp8.quantize_activation_tensor(x, sc)
    np.testing.assert_allclose(e4m3_decode(q) * s, x, atol=6e-2, rtol=1.3e-1)


def test_act_quant_block_closed_forms():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 256)).astype(F32)
    x[2, 128:] = 0
    q, s = ofp8.act_quant_block(x)
    np.testing.assert_array_equal(s[:2], (np.abs(x[:2]).reshape(2, 2, 128).max(2) * (F32(1) / F32(448))).astype(F32))
    assert s[2, 1] == F32(1e-4) * (F32(1) / F32(448))  # zero block: amax floor 1e-4
    qp, sp = ofp8.act_quant_block(x, round_scale=True)
    # power-of-two scales, the smallest 2^e >= amax/448
    e = np.log2(sp)
    assert np.array_equal(e, np.round(e))
    assert np.all(sp >= s * (1 - 1e-6)) and np.all(sp < 2 * s * (1 + 1e-6))


def test_rowcol_gemm_selection_matrices():
    """wq = identity-like selection codes: out = xq values * xs * ws exactly."""
    rng = np.random.default_rng(2)
    k, n = 16, 4
    xq = e4m3_encode(rng.standard_normal((3, k)).astype(F32))
    sel = np.zeros((n, k), F32)
    perm = [5, 0, 9, 3]
    for j, p in enumerate(perm):
        sel[j, p] = 1.0
    wq = e4m3_encode(sel)
    xs = np.array([[2.0], [0.5], [1.0]], F32)
    ws = np.array([[1.0, 4.0, 0.25, 8.0]], F32)
    out = ofp8.fp8_linear_rowcol(xq, xs, wq, ws)
    want = e4m3_decode(xq)[:, perm] * xs * ws
    np.testing.assert_array_equal(out, want.astype(F32))


def test_rowcol_gemm_matches_dequantized_matmul():
    rng = np.random.default_rng(3)
    xq = e4m3_encode(rng.standard_normal((5, 256)).astype(F32))
    wq = e4m3_encode(rng.standard_normal((7, 256)).astype(F32))
    xs = rng.uniform(0.01, 1, (5, 1)).astype(F32)
    ws = rng.uniform(0.01, 1, (1, 7)).astype(F32)
    out = ofp8.fp8_linear_rowcol(xq, xs, wq, ws)
    deq = (e4m3_decode(xq).astype(np.float64) * xs) @ (e4m3_decode(wq).astype(np.float64) * ws.T).T
    np.testing.assert_allclose(out, deq, rtol=1e-6, atol=1e-6)


def test_block_gemm_equals_dequantize_then_matmul():
    """Per-K-block scaling (the TileLang association) vs dequantize-then-matmul
    (ops.py:180-188 dequant + one product): same sum, different order."""
    rng = np.random.default_rng(4)
    m, k, n = 6, 384, 200
    a_codes, a_s = ofp8.act_quant_block(rng.standard_normal((m, k)).astype(F32))
    b_codes, b_s = ofp8.quantize_weight_block((rng.standard_normal((n, k)) * 0.02).astype(F32))
    out = ofp8.fp8_gemm_block(a_codes, a_s, b_codes, b_s)
    a_deq = e4m3_decode(a_codes).astype(np.float64) * np.repeat(a_s, 128, 1)
    b_deq = ofp8.dequantize_block_fp8(b_codes, b_s).astype(np.float64)
    np.testing.assert_allclose(out, a_deq @ b_deq.T, rtol=1e-5, atol=1e-6)
    # the scales matter per block: perturbing one block's weight scale moves only its columns
    b_s2 = b_s.copy()
    b_s2[1, 2] *= 2
    out2 = ofp8.fp8_gemm_block(a_codes, a_s, b_codes, b_s2)
    assert np.array_equal(out2[:, :128], out[:, :128]) and not np.allclose(out2[:, 128:], out[:, 128:])


def test_block_weight_quant_restores():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((130, 260)) * 0.02).astype(F32)
    q, s = ofp8.quantize_weight_block(w)
    assert s.shape == (2, 3)
    np.testing.assert_allclose(ofp8.dequantize_block_fp8(q, s), w, rtol=0.07, atol=1e-3)
