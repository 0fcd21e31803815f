"""GPTQ / AWQ ingestion and the prepared-weight file on the GPU: the product of
an act-order GPTQ checkpoint equals the oracle's dequantize-then-matmul of the
original (un-permuted) weight; save/load round-trips bit for bit."""
import numpy as np
import pytest
import torch

from oracle import int4 as oint4
from tests._problems import pack_k_words as _pack_k, pack_n_words as _pack_n

pytestmark = pytest.mark.gpu


def _rel(y, ref):
    return float(np.abs(y - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("act_order", [False, True])
@pytest.mark.parametrize("m", [1, 24, 100])
def test_gptq_act_order_matches_oracle(dev, act_order, m):
    from torchinferno_amd.kernels import checkpoint as ck
    print(f"[ckpt] gptq act_order={act_order} M={m}", flush=True)
    rng = np.random.default_rng(m + act_order)
    k, n = 1024, 320
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)   # original row order
    scales = (rng.random((k // 128, n)) * 0.02 + 0.002).astype(np.float16)
    g_idx = rng.permutation(np.repeat(np.arange(k // 128), 128)) if act_order else np.arange(k) // 128
    # GPTQ stores row r's scale in group g_idx[r]: build the checkpoint so that the
    # dequantized weight is (codes - 8) * scales[g_idx[r]].
    zeros = np.full((k // 128, n), 7, np.uint8)  # v1: zero point 8 stored as 7
    w = ck.from_gptq(_pack_k(codes), torch.from_numpy(scales), _pack_n(zeros),
                     torch.from_numpy(g_idx.astype(np.int32)), dtype=torch.bfloat16, device=dev)
    a = torch.randn((m, k), device=dev).to(torch.bfloat16)
    y = w.mm(a)
    deq = (codes.astype(np.float64) - 8) * torch.from_numpy(scales).to(torch.bfloat16).double().numpy()[g_idx]
    ref = a.float().cpu().double().numpy() @ deq
    assert _rel(y.float().cpu().numpy(), ref) <= 1e-2


def test_awq_symmetric_matches_oracle(dev):
    from torchinferno_amd.kernels import checkpoint as ck
    rng = np.random.default_rng(5)
    k, n = 512, 128
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    scales = (rng.random((k // 128, n)) * 0.02 + 0.002).astype(np.float16)
    order = (0, 2, 4, 6, 1, 3, 5, 7)
    w = ck.from_awq(_pack_n(codes, order), torch.from_numpy(scales),
                    _pack_n(np.full((k // 128, n), 8, np.uint8), order), device=dev)
    a = torch.randn((7, k), device=dev).to(torch.float16)
    ref = oint4.w4a16_reference(a.float().cpu().numpy(), oint4.pack_int4(codes), scales.astype(np.float32))
    assert _rel(w.mm(a).float().cpu().numpy(), ref) <= 1e-2


def test_prepared_file_round_trip(dev, tmp_path):
    from torchinferno_amd.kernels import checkpoint as ck
    rng = np.random.default_rng(9)
    k, n = 256, 64
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    g_idx = rng.permutation(np.repeat(np.arange(2), 128)).astype(np.int32)
    w = ck.from_gptq(_pack_k(codes), torch.ones((2, n), dtype=torch.float16), None, torch.from_numpy(g_idx),
                     device=dev)
    path = str(tmp_path / "w.safetensors")
    ck.save_prepared(path, {"layers.0.mlp.down": w})
    back = ck.load_prepared(path, device=dev)["layers.0.mlp.down"]
    assert (back.size_k, back.size_n) == (k, n)
    assert torch.equal(back.q_weight, w.q_weight) and torch.equal(back.scales, w.scales)
    assert torch.equal(back.perm, w.perm)
    a = torch.randn((4, k), device=dev).to(torch.float16)
    assert torch.equal(back.mm(a), w.mm(a))


@pytest.mark.parametrize("fmt,act_order,m", [("gptq", False, 1), ("gptq", True, 17), ("awq", False, 5),
                                             ("awq", False, 64)])
def test_asymmetric_zero_points_match_oracle(dev, fmt, act_order, m):
    """Asymmetric checkpoints: W = (q - z) * s with per-(group, column) z in [0, 15]
    (GPTQ stores z - 1), against the oracle's dequantize-then-matmul; z = 8 columns
    and the symmetric result agree."""
    from torchinferno_amd.kernels import checkpoint as ck
    print(f"[ckpt] zero points {fmt} act_order={act_order} M={m}", flush=True)
    rng = np.random.default_rng(m * 3 + act_order)
    k, n = 1024, 192
    codes = rng.integers(0, 16, (k, n), dtype=np.uint8)
    scales = (rng.random((k // 128, n)) * 0.02 + 0.002).astype(np.float16)
    z = rng.integers(1, 16, (k // 128, n)).astype(np.uint8)
    z[:, :16] = 8  # some symmetric columns
    g_idx = rng.permutation(np.repeat(np.arange(k // 128), 128)) if act_order else np.arange(k) // 128
    if fmt == "gptq":
        w = ck.from_gptq(_pack_k(codes), torch.from_numpy(scales), _pack_n(z - 1),
                         torch.from_numpy(g_idx.astype(np.int32)), dtype=torch.float16, device=dev)
    else:
        order = (0, 2, 4, 6, 1, 3, 5, 7)
        w = ck.from_awq(_pack_n(codes, order), torch.from_numpy(scales), _pack_n(z, order), device=dev)
    assert w.zero_offset is not None
    a = torch.randn((m, k), device=dev).to(torch.float16)
    y = w.mm(a).float().cpu().numpy()
    s32 = scales.astype(np.float32)
    deq = (codes.astype(np.float64) - z.astype(np.float64)[g_idx]) * s32.astype(np.float64)[g_idx]
    ref = a.float().cpu().double().numpy() @ deq
    assert _rel(y, ref) <= 1e-2
    if not act_order:  # the oracle function itself on the canonical words
        ref2 = oint4.w4a16_reference_zp(a.float().cpu().numpy(), oint4.pack_int4(codes), s32, z.astype(np.int32))
        assert _rel(y, ref2) <= 1e-2
