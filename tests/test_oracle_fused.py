"""Pins oracle/fused.py (CPU): the reference test's restore tolerances against
plain torch float math (tests/test_conversion_and_kernels.py:390-435, seed 17),
"fused == norm then per-token quant", and closed forms of the norm."""
import numpy as np
import torch

from oracle import fused as ofu
from oracle.fp8 import quantize_activation_per_token
from oracle.numerics import e4m3_decode, round_to

F32 = np.float32


def test_reference_restore_tolerances():
    torch.manual_seed(17)
    x = torch.randn((7, 64), dtype=torch.bfloat16)
    residual = torch.randn_like(x)
    weight = torch.randn((64,), dtype=torch.bfloat16)
    eps = 1e-5
    xn, rn, wn = x.float().numpy(), residual.float().numpy(), weight.float().numpy()
    expected = (x.float() * torch.rsqrt(x.float().square().mean(-1, keepdim=True) + eps) * weight.float()).numpy()
    q, s = ofu.rms_norm_fp8_per_token(xn, wn, eps, "bf16")
    np.testing.assert_allclose(e4m3_decode(q) * s, expected, atol=1.2e-1, rtol=1.3e-1)
    h = (x.float() + residual.float())
    expected2 = (h * torch.rsqrt(h.square().mean(-1, keepdim=True) + eps) * weight.float()).numpy()
    hid, q2, s2 = ofu.add_rms_norm_fp8_per_token(xn, rn, wn, eps, "bf16")
    np.testing.assert_allclose(hid, (x + residual).float().numpy(), atol=2e-2, rtol=2e-2)
    np.testing.assert_allclose(e4m3_decode(q2) * s2, expected2, atol=1.2e-1, rtol=1.3e-1)
    gate, up = torch.randn((7, 128), dtype=torch.bfloat16).split(64, dim=-1)
    exp3 = (torch.nn.functional.silu(gate.float()) * up.float()).numpy()
    q3, s3 = ofu.swiglu_fp8_per_token(gate.float().numpy(), up.float().numpy(), "bf16")
    np.testing.assert_allclose(e4m3_decode(q3) * s3, exp3, atol=1.2e-1, rtol=1.3e-1)


def test_fused_is_norm_then_quant():
    rng = np.random.default_rng(0)
    x = round_to(rng.standard_normal((5, 96)).astype(F32), "fp16")
    w = round_to(rng.standard_normal(96).astype(F32), "fp16")
    q, s = ofu.rms_norm_fp8_per_token(x, w, 1e-6, "fp16")
    q2, s2 = quantize_activation_per_token(round_to(ofu._rms(x, w, 1e-6), "fp16"))
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


def test_rms_closed_forms():
    # constant rows: rms = |c|, so normed = sign(c) * w (up to eps)
    x = np.full((2, 8), 3.0, F32)
    x[1] = -0.5
    w = np.arange(1, 9, dtype=F32)
    out = ofu._rms(x, w, 0.0)
    np.testing.assert_allclose(out[0], w, rtol=1e-6)
    np.testing.assert_allclose(out[1], -w, rtol=1e-6)
    # silu(0) * u = 0; silu(large) ~ g
    a = ofu.swiglu_activation(np.array([[0.0, 30.0]], F32), np.array([[5.0, 2.0]], F32), "fp32")
    assert a[0, 0] == 0.0 and abs(a[0, 1] - 60.0) < 1e-3


def test_exp_rounding_is_implementation_independent():
    """The SwiGLU producers evaluate exp(-g) in fp64 and round to fp32.  For every
    finite bf16 and fp16 g, exp(-g) lies at least 2^-51 (relative) from an fp32
    rounding midpoint, so any fp64 exp accurate to 1 ulp (2^-52) -- numpy's, the
    GPU math library's -- rounds to the same fp32 value: the oracle's choice is
    reproducible on the device for all inputs."""
    with np.errstate(over="ignore"):
        for vals in ((np.arange(65536, dtype=np.uint32) << 16).view(F32),
                     np.arange(65536, dtype=np.uint16).view(np.float16).astype(F32)):
            g = vals[np.isfinite(vals)].astype(np.float64)
            e = np.exp(-g)
            e = e[(e > 0) & (e < 3.0e38)]
            f = e.astype(F32)
            f64 = f.astype(np.float64)
            nxt = np.where(e >= f64, np.nextafter(f, F32(np.inf)), np.nextafter(f, F32(0))).astype(np.float64)
            mid = (f64 + nxt) / 2
            assert (np.abs(e - mid) / e).min() >= 2.0 ** -51


def test_exp_neg_closed_forms_outside_table_range():
    """The bf16 SwiGLU kernel tabulates g / (1 + exp(-g)) only for exponent fields
    102..133 (2^-25 <= |g| < 128).  Outside that range the fp64 expression,
    rounded to fp32, is exactly 1 (|g| < 2^-25), 0 (g >= 128) or inf
    (g <= -128) for every finite bf16 value."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    bits = bits[((bits >> 7) & 0xFF) != 0xFF]
    g = (bits << 16).view(np.float32)
    with np.errstate(over="ignore"):
        e = np.exp(-g.astype(np.float64)).astype(np.float32)
    field = (bits >> 7) & 0xFF
    neg = ((bits >> 15) & 1) == 1
    assert np.all(e[field < 102] == 1.0)
    assert np.all(e[(field >= 134) & ~neg] == 0.0)
    assert np.all(np.isposinf(e[(field >= 134) & neg]))
    # and inside it the values are neither all 1 nor saturated (the table is needed)
    inside = (field >= 102) & (field < 134)
    assert np.any(e[inside] != 1.0) and np.all(np.isfinite(e[inside & ~neg]))
    # so the quotient g / (1 + e) is g * 0.5, g and -0 there, bit for bit
    with np.errstate(over="ignore", invalid="ignore"):
        silu = (g / (np.float32(1.0) + e)).astype(np.float32)
    lo, hi_pos, hi_neg = field < 102, (field >= 134) & ~neg, (field >= 134) & neg
    assert np.array_equal(silu[lo].view(np.uint32), (g[lo] * np.float32(0.5)).view(np.uint32))
    assert np.array_equal(silu[hi_pos].view(np.uint32), g[hi_pos].view(np.uint32))
    assert np.all(silu[hi_neg].view(np.uint32) == np.uint32(0x80000000))
