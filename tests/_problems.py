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
