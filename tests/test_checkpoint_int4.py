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


def test_asymmetric_zero_points_rejected():
    k, n = 256, 64
    q = _pack_k(np.zeros((k, n), np.uint8))
    s = torch.ones((k // 128, n), dtype=torch.float16)
    zeros = np.full((k // 128, n), 7, np.uint8)  # v1 storage of zero point 8
    zeros[1, 5] = 3
    with pytest.raises(NotImplementedError):
        ck.from_gptq(q, s, _pack_n(zeros))
    with pytest.raises(NotImplementedError):
        ck.from_awq(_pack_n(np.zeros((k, n), np.uint8), (0, 2, 4, 6, 1, 3, 5, 7)), s,
                    _pack_n(np.full((k // 128, n), 5, np.uint8)))
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
