"""Host-side checks of GPTQ / AWQ int4 ingestion (CPU): the word unpacking
against an independent per-nibble packer written from the formats' definitions,
zero-point validation and act-order regrouping."""
import numpy as np
import pytest
import torch

from tests._problems import pack_k_words as _pack_k, pack_n_words as _pack_n
from torchinferno_amd.kernels import checkpoint as ck


def test_unpack_along_k_and_n():
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, (256, 64), dtype=np.uint8)
    assert np.array_equal(ck._unpack_words_k(_pack_k(codes)).numpy(), codes)
    assert np.array_equal(ck._unpack_words_n(_pack_n(codes)).numpy(), codes)
    order = (0, 2, 4, 6, 1, 3, 5, 7)
    assert np.array_equal(ck._unpack_words_n(_pack_n(codes, order), order).numpy(), codes)


def test_zero_offset_host_side():
    """(8 - z) * s per (group, column), fp32, with s rounded to the activation dtype;
    None when every zero point is 8; GPTQ v1 storage (z - 1) and AWQ's word order
    unpack to the same zero points; bad shapes and group maps are rejected."""
    k, n = 256, 64
    rng = np.random.default_rng(3)
    z = rng.integers(0, 16, (k // 128, n)).astype(np.uint8)
    s = torch.from_numpy((rng.random((k // 128, n)) * 0.02 + 0.002).astype(np.float32))
    zo = ck._zero_offset(torch.from_numpy(z.astype(np.int64)), s, torch.bfloat16, torch.device("cpu"))
    want = (8 - z.astype(np.float64)) * s.to(torch.bfloat16).double().numpy()
    assert zo.dtype == torch.float32 and np.array_equal(zo.double().numpy(), want)
    assert ck._zero_offset(torch.full((2, n), 8), s, torch.float16, torch.device("cpu")) is None
    with pytest.raises(ValueError):
        ck._zero_offset(torch.full((2, n), 16), s, torch.float16, torch.device("cpu"))
    v1 = np.clip(z.astype(np.int64) - 1, 0, 15)
    assert np.array_equal((ck._unpack_words_n(_pack_n(v1)) + 1).numpy(), np.maximum(z, 1))
    order = (0, 2, 4, 6, 1, 3, 5, 7)
    assert np.array_equal(ck._unpack_words_n(_pack_n(z, order), order).numpy(), z)
    q = _pack_k(np.zeros((k, n), np.uint8))
    with pytest.raises(ValueError):
        ck.from_gptq(q, s, g_idx=torch.zeros(k, dtype=torch.int32))  # every row in group 0
    with pytest.raises(ValueError):
        ck.from_gptq(q, s, bits=8)


def test_act_order_regrouping_preserves_the_product():
    """Regrouping rows by g_idx and gathering the activation's columns with the
    same permutation leaves A @ W unchanged (the identity the GPU path relies on)."""
    rng = np.random.default_rng(1)
    k, n = 256, 8
    g_idx = rng.permutation(np.repeat(np.arange(k // 128), 128))
    perm = np.argsort(g_idx, kind="stable")
    w = rng.standard_normal((k, n))
    a = rng.standard_normal((3, k))
    assert np.allclose(a[:, perm] @ w[perm], a @ w)
    assert np.array_equal(np.sort(g_idx[perm]), g_idx[perm])  # groups contiguous after regrouping
