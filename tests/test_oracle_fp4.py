"""Pins oracle/fp4.py (CPU): e2m1 against the OCP MX formula and torch's
float4_e2m1fn_x2 packing, e8m0 against torch's float8_e8m0fnu, and the GEMM
against an fp64 dequantize-then-matmul and one-hot closed forms."""
import numpy as np
import pytest
import torch

from oracle import fp4 as of4
from oracle.numerics import e4m3_encode


def test_e2m1_table_matches_formula():
    for code in range(16):
        s, e, m = code >> 3, (code >> 1) & 3, code & 1
        v = (m * 0.5) if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        assert of4.e2m1_decode(np.array([code]))[0] == (-v if s else v)


def test_nibble_order_matches_torch_packing():
    codes = np.arange(16, dtype=np.uint8)
    packed = of4.pack_fp4(codes)
    assert np.array_equal(of4.unpack_fp4(packed), codes)
    assert packed[0] == 0x10 and packed[7] == 0xFE  # element 0 in the low nibble
    t = torch.from_numpy(packed).view(torch.float4_e2m1fn_x2)
    assert t.shape == (8,) and t.view(torch.uint8)[0].item() == 0x10


def test_e8m0_matches_torch():
    b = np.arange(255, dtype=np.uint8)
    ref = torch.from_numpy(b).view(torch.float8_e8m0fnu).float().numpy()
    assert np.array_equal(of4.e8m0_decode(b), ref)
    assert np.isnan(of4.e8m0_decode(np.array([255]))[0])


def test_fp4_gemm_association_orders_agree():
    rng = np.random.default_rng(3)
    m, n, k = 5, 24, 256
    a = e4m3_encode((rng.standard_normal((m, k)) * 40).astype(np.float32))
    a_s = (rng.random((m, k // 128)) * 0.01 + 1e-3).astype(np.float32)
    b = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    b_s = rng.integers(118, 134, (n, k // 32), dtype=np.uint8)
    got = of4.fp4_gemm(a, a_s, b, b_s)
    ref = of4.fp4_gemm_f64(a, a_s, b, b_s)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5 * np.abs(ref).max())


def test_fp4_gemm_one_hot_closed_form():
    m, n, k = 2, 3, 128
    a = np.zeros((m, k), np.uint8)
    a[1, 37] = e4m3_encode(np.array([3.0], np.float32))[0]
    a_s = np.full((m, 1), 0.25, np.float32)
    codes = np.zeros((n, k), np.uint8)
    codes[2, 37] = 0b1111  # -6
    b_s = np.full((n, k // 32), 127, np.uint8)
    b_s[2, 1] = 130  # 2^3 for the block holding k=37
    out = of4.fp4_gemm(a, a_s, of4.pack_fp4(codes), b_s)
    expect = np.zeros((m, n), np.float32)
    expect[1, 2] = 3.0 * 0.25 * -6.0 * 8.0
    assert np.array_equal(out, expect)


def test_reference_known_answer():
    """tests/test_deepseek_v4.py:554-558 of the reference: byte 0x21 with a unit
    E8M0 scale dequantizes to [0.5, 1.0] (low nibble first), 32 values per row."""
    packed = np.zeros((1, 16), np.uint8)
    packed[0, 0] = 0x21
    out = of4.dequantize_fp4(packed, np.full((1, 1), 127, np.uint8))
    assert out.shape == (1, 32)
    assert out[0, 0] == 0.5 and out[0, 1] == 1.0 and not out[0, 2:].any()
