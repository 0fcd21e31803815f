"""Pins oracle/int4.py with checks that do not restate its formulas."""
import numpy as np
import torch

from oracle import int4 as o


def test_pack_hand_built_word():
    codes = np.zeros((8, 2), dtype=np.uint8)
    codes[:, 0] = np.arange(8)          # 0x76543210
    codes[:, 1] = [15, 0, 0, 0, 0, 0, 0, 1]  # 0x1000000F
    w = o.pack_int4(codes).view(np.uint32)
    assert w[0, 0] == 0x76543210 and w[0, 1] == 0x1000000F
    assert np.array_equal(o.unpack_int4(w.view(np.int32)), codes)


def test_pack_roundtrip_random():
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (256, 48), dtype=np.uint8)
    assert np.array_equal(o.unpack_int4(o.pack_int4(codes)), codes)


def test_dequant_closed_forms():
    codes = np.zeros((128, 3), dtype=np.uint8)
    codes[:, 0], codes[:, 1], codes[:, 2] = 8, 0, 15
    s = np.float32([[0.5, 0.25, 2.0]])
    d = o.dequant_int4(o.pack_int4(codes), s)
    assert np.all(d[:, 0] == 0) and np.all(d[:, 1] == -2.0) and np.all(d[:, 2] == 14.0)


def test_gemm_selection_matrix_returns_activation_columns():
    """codes = 8 + [k == perm[n]] with unit scales: out[:, n] = a[:, perm[n]] exactly.
    Catches transposed operands, wrong K/N indexing and a wrong zero point."""
    rng = np.random.default_rng(1)
    k = n = 256
    perm = rng.permutation(k)
    codes = np.full((k, n), 8, dtype=np.uint8)
    codes[perm, np.arange(n)] = 9
    a = rng.standard_normal((5, k)).astype(np.float32)
    out = o.w4a16_reference(a, o.pack_int4(codes), np.ones((k // 128, n), np.float32))
    assert np.array_equal(out, a[:, perm])


def test_gemm_group_scales_select_the_right_rows():
    """Only group 1 has a non-zero scale: out = rowsum of a's second 128 columns * 3 * s."""
    k, n = 384, 64
    codes = np.full((k, n), 11, dtype=np.uint8)  # value +3
    s = np.zeros((3, n), np.float32)
    s[1] = 0.5
    a = np.random.default_rng(2).standard_normal((3, k)).astype(np.float32)
    out = o.w4a16_reference(a, o.pack_int4(codes), s)
    expect = (a[:, 128:256].astype(np.float64).sum(1) * 1.5)[:, None]
    assert np.allclose(out, np.repeat(expect, n, 1), rtol=1e-5, atol=1e-5)


def test_gemm_brute_force_fp64_tiny():
    rng = np.random.default_rng(3)
    m, k, n = 3, 128, 16
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    s = rng.uniform(0.002, 0.02, (1, n)).astype(np.float32)
    a = rng.standard_normal((m, k)).astype(np.float32)
    out = o.w4a16_reference(a, o.pack_int4(codes), s)
    for i in range(m):
        for j in range(n):
            acc = sum(float(a[i, kk]) * (int(codes[kk, j]) - 8) * float(s[0, j]) for kk in range(k))
            assert abs(out[i, j] - acc) <= 1e-5 * max(1.0, abs(acc))


def test_rtn_quantizer_scale_rule_and_error_bound():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((256, 32)) * 0.02).astype(np.float16).astype(np.float32)
    q, s = o.quantize_int4_rtn(w, 128, "fp32")
    g = w.reshape(2, 128, 32)
    # Symmetric scale: the larger of max/7 and |min|/8.
    assert np.allclose(s, np.maximum(g.max(1) / 7, -g.min(1) / 8))
    d = o.dequant_int4(q, s)
    assert np.all(np.abs(d - w) <= np.repeat(s, 128, 0) * 0.5 + 1e-9)
    codes = o.unpack_int4(q)
    assert codes.min() >= 0 and codes.max() <= 15


def test_rtn_quantizer_matches_torch_restatement():
    """The product's torch quantizer (torchinferno_amd.kernels.int4) and the oracle agree."""
    from torchinferno_amd.kernels import int4 as ti4
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(512, 64, generator=g) * 0.02).to(torch.bfloat16)
    q, s = ti4.quantize_int4_rtn(w, 128, torch.bfloat16)
    oq, os_ = o.quantize_int4_rtn(w.to(torch.float16).float().numpy(), 128, "bf16")
    assert np.array_equal(q.numpy(), oq) and np.array_equal(s.float().numpy(), os_)


def test_torch_pack_matches_oracle_pack():
    from torchinferno_amd.kernels import int4 as ti4
    codes = torch.randint(0, 16, (64, 24), generator=torch.Generator().manual_seed(5))
    assert np.array_equal(ti4.pack_int4(codes).numpy(), o.pack_int4(codes.numpy().astype(np.uint8)))


def test_zero_point_dequant_closed_forms():
    """(q - z) * s: z = 8 is the symmetric dequant; q = z gives exact zeros; each
    group's zero point acts only on its own 128 rows and column."""
    rng = np.random.default_rng(11)
    k, n = 256, 24
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    q = o.pack_int4(codes)
    s = torch.from_numpy((rng.random((2, n)) * 0.02 + 0.002).astype(np.float32)).to(torch.bfloat16).float().numpy()
    z8 = np.full((2, n), 8, np.int32)
    assert np.array_equal(o.dequant_int4_zp(q, s, z8), o.dequant_int4(q, s))
    z = rng.integers(0, 16, (2, n)).astype(np.int32)
    deq = o.dequant_int4_zp(q, s, z)
    for g in range(2):
        rows = slice(128 * g, 128 * (g + 1))
        want = (codes[rows].astype(np.float64) - z[g]) * s[g].astype(np.float64)
        assert np.array_equal(deq[rows].astype(np.float64), want)
    z2 = z.copy()
    z2[1, 3] += 1
    diff = o.dequant_int4_zp(q, s, z2) - deq
    assert np.all(diff[128:, 3] == -s[1, 3]) and np.count_nonzero(diff) == 128
    a = rng.standard_normal((3, k)).astype(np.float32)
    np.testing.assert_allclose(o.w4a16_reference_zp(a, q, s, z),
                               a.astype(np.float64) @ deq.astype(np.float64), rtol=1e-5, atol=1e-5)
