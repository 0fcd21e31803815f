"""Seeded synthetic problems of BASELINE.json's configs, generated on the CPU
with torch.Generator so the oracle (numpy) and the GPU see identical inputs."""
from __future__ import annotations

import numpy as np
import torch


def int4_problem(m: int, k: int, n: int, dtype: torch.dtype, seed: int):
    """Config 0/1 scheme: a ~ N(0,1), codes ~ U{0..15}, scales ~ U[0.002, 0.02]."""
    g = torch.Generator().manual_seed(seed)
    a = torch.randn((m, k), generator=g).to(dtype)
    codes = torch.randint(0, 16, (k, n), generator=g, dtype=torch.int32)
    scales = (torch.rand((k // 128, n), generator=g) * 0.018 + 0.002).to(dtype)
    return a, codes, scales


def to_np32(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy()


def pack_k_words(codes):
    """GPTQ qweight: word [r, n] holds rows 8r..8r+7 of column n, row 8r+i in bits 4i."""
    k, n = codes.shape
    out = np.zeros((k // 8, n), np.uint32)
    for r in range(k // 8):
        for i in range(8):
            out[r] |= codes[8 * r + i].astype(np.uint32) << np.uint32(4 * i)
    return torch.from_numpy(out.view(np.int32))


def pack_n_words(codes, order=None):
    """Words along N: word [r, c] holds columns 8c..8c+7; slot j holds column
    8c + order[j] (AWQ) or 8c + j (GPTQ qzeros)."""
    r_, n = codes.shape
    out = np.zeros((r_, n // 8), np.uint32)
    for c in range(n // 8):
        for j in range(8):
            col = 8 * c + (order[j] if order else j)
            out[:, c] |= codes[:, col].astype(np.uint32) << np.uint32(4 * j)
    return torch.from_numpy(out.view(np.int32))
