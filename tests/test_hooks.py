"""Host-side behaviour of the drop-in layer (no GPU): custom-op registration and
fake (shape) implementations, the dispatch gates that fall back to None off-GPU
(tensor_parallel.py:2757-2760 returns None for CPU tensors), and patch/undo."""
import types

import torch

from torchinferno_amd import hooks, ops  # noqa: F401  (registers the ops)


def test_custom_ops_registered():
    for name in ("w4a16_mm", "w4a16_mm_out", "fp8_scaled_mm_out", "fp8_per_token_linear", "act_quant",
                 "fp8_block_gemm", "moe_route_topk", "fused_fp8_moe"):
        assert hasattr(torch.ops.torchinferno_amd, name), name


def test_fake_shapes_on_meta():
    m = torch.device("meta")
    a = torch.empty((5, 256), dtype=torch.bfloat16, device=m)
    y = torch.ops.torchinferno_amd.w4a16_mm(a, torch.empty((16, 2, 256), dtype=torch.int32, device=m),
                                            torch.empty((2, 256), dtype=torch.bfloat16, device=m),
                                            torch.empty(4, dtype=torch.int32, device=m), 256, 256)
    assert y.shape == (5, 256) and y.dtype == torch.bfloat16
    q, s = torch.ops.torchinferno_amd.act_quant(torch.empty((3, 7, 384), dtype=torch.bfloat16, device=m), 128, False)
    assert q.shape == (3, 7, 384) and q.dtype == torch.float8_e4m3fn and s.shape == (3, 7, 3)
    g = torch.ops.torchinferno_amd.fp8_block_gemm(q, s, torch.empty((200, 384), dtype=torch.float8_e4m3fn, device=m),
                                                  torch.empty((2, 3), device=m))
    assert g.shape == (3, 7, 200) and g.dtype == torch.bfloat16
    w, ids = torch.ops.torchinferno_amd.moe_route_topk(torch.empty((9, 256), device=m), 8, True, 1.0)
    assert w.shape == (9, 8) and ids.dtype == torch.int32


class _Layer:
    pass


def test_llama3_hooks_fall_back_off_gpu(monkeypatch):
    undo = hooks.patch_llama3_layer_class(_Layer)
    try:
        layer = object.__new__(_Layer)
        x = torch.randn(2, 1, 64)
        w = torch.randn(128, 64)
        assert layer._marlin_proj(x, "gu", w) is None  # CPU tensor -> bf16 fallback
        monkeypatch.setenv("TORCHINFERNO_FP8_PREFILL", "1")
        assert layer._fp8_proj(torch.randn(300, 64), "gu", w) is None
        monkeypatch.setenv("TORCHINFERNO_MARLIN_INT4_DECODE", "0")
        assert layer._marlin_proj(x, "gu", w) is None
    finally:
        undo()
    assert not hasattr(_Layer, "_marlin_proj")


def test_fp8_decode_gate():
    import os
    os.environ["TORCHINFERNO_FP8_DECODE"] = "1"
    try:
        assert hooks.fp8_decode_shape_enabled(torch.empty(4, 1, 8))
        assert not hooks.fp8_decode_shape_enabled(torch.empty(4, 2, 8))
        assert not hooks.fp8_decode_shape_enabled(torch.empty(200, 1, 8))
    finally:
        del os.environ["TORCHINFERNO_FP8_DECODE"]
    assert not hooks.fp8_decode_shape_enabled(torch.empty(4, 1, 8))


def test_deepseek_module_patch_and_bf16_passthrough():
    mod = types.ModuleType("fake_dsv4")
    mod.linear = lambda x, w, b=None: "original"
    undo = hooks.patch_deepseek_v4_module(mod)
    x, w = torch.randn(3, 8), torch.randn(4, 8)
    assert torch.allclose(mod.linear(x, w), x @ w.t())  # bf16/fp32 weights keep F.linear
    undo()
    assert mod.linear(x, w) == "original"


def test_power_of_two_scale_detection(monkeypatch):
    """Experts take the MFMA-applied scale path (round_scale 2) only when every block
    scale is a power of two in the E8M0 range and the activation scales are too."""
    from torchinferno_amd.kernels import moe as tmoe
    e8 = torch.tensor([1.0, 0.5, 2.0 ** -20]).to(torch.float8_e8m0fnu)
    assert tmoe._all_pow2(e8)
    assert tmoe._all_pow2(torch.tensor([[0.25, 4.0], [2.0 ** -127, 1.0]]))
    assert not tmoe._all_pow2(torch.tensor([0.25, 0.3]))           # not a power of two
    assert not tmoe._all_pow2(torch.tensor([2.0 ** -128]))         # below E8M0's range
    assert not tmoe._all_pow2(torch.tensor([0.0]))
    assert not tmoe._all_pow2(torch.tensor([-0.5]))
    assert tmoe._round_scale(None, True) == 0
    assert tmoe._round_scale("ue8m0", False) == 1
    assert tmoe._round_scale("ue8m0", True) == 2
    monkeypatch.setenv("TI_ROCM_POW2_MFMA", "0")
    assert tmoe._round_scale("ue8m0", True) == 1
