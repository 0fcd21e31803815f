"""The drop-in dispatch on the GPU: patched Llama3 layer methods and the DeepSeek
linear/MoE hooks run this package's kernels, keep the reference's contracts
(lazy per-key cache, caller-owned out, M gates, sticky failure -> None), and the
custom ops pass torch.library.opcheck."""

import numpy as np
import pytest
import torch

from oracle import int4 as oint4

pytestmark = pytest.mark.gpu


class _Layer:
    pass


@pytest.fixture
def layer():
    from torchinferno_amd import hooks
    undo = hooks.patch_llama3_layer_class(_Layer)
    yield object.__new__(_Layer)
    undo()


def _rel(a, b):
    a, b = a.float().cpu().numpy(), np.asarray(b, dtype=np.float32)
    return float(np.abs(a - b).max() / np.abs(b).max())


def test_marlin_proj_caches_and_matches_oracle(dev, layer):
    from torchinferno_amd.kernels import int4 as ti4
    g = torch.Generator(device=dev).manual_seed(1)
    w = (torch.randn((512, 1024), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((8, 1, 1024), generator=g, device=dev).to(torch.bfloat16)
    y = layer._marlin_proj(x, "gu", w)
    assert y.shape == (8, 1, 512) and layer._marlin_gu_n == 512 and layer._marlin_gu_k == 1024
    # against the layer's own cached int4 weight (exact dequant on the GPU)
    deq = ti4.dequantize_int4(layer._marlin_gu_q, layer._marlin_gu_s, 1024, 512).cpu().numpy()
    ref = x.view(8, 1024).float().cpu().numpy().astype(np.float64) @ deq.astype(np.float64)
    assert _rel(y.view(8, 512), ref) <= 1e-2
    out = torch.empty((8, 1, 512), dtype=torch.bfloat16, device=dev)
    r = layer._marlin_proj(x, "gu", w, out=out)
    assert torch.equal(out, y) and r.data_ptr() == out.data_ptr()
    # prefill-size M stays bf16
    assert layer._marlin_proj(torch.zeros((129, 1024), dtype=torch.bfloat16, device=dev), "gu", w) is None


@pytest.mark.parametrize("wdt,sdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16),
                                     (torch.bfloat16, torch.float16)])
def test_int4_rtn_quantizer_gpu_bit_exact(dev, wdt, sdt):
    """The lazy weight quantization (ti_int4_quantize_rtn, the quantizer of
    marlin.py:117-128) matches the oracle's codes and scales bit for bit, including
    round-half-even ties (common: fp16 weights have 11 significant bits)."""
    from oracle.numerics import round_to
    from torchinferno_amd.kernels import int4 as ti4
    g = torch.Generator(device=dev).manual_seed(1)
    w = (torch.randn((1024, 512), generator=g, device=dev) * 0.02).to(wdt)
    w[:128, 0] = 0  # all-zero group: scale floor 1e-8
    qd, sd = ti4.quantize_int4_rtn(w, 128, sdt)
    oq, os_ = oint4.quantize_int4_rtn(round_to(w.float().cpu().numpy(), "fp16"), 128,
                                      "bf16" if sdt == torch.bfloat16 else "fp16")
    assert np.array_equal(qd.cpu().numpy(), oq)
    assert np.array_equal(sd.float().cpu().numpy(), os_)


def test_marlin_proj_unsupported_shape_is_sticky(dev, layer):
    w = torch.randn((100, 256), device=dev).to(torch.bfloat16)  # N % 64 != 0
    x = torch.randn((2, 256), device=dev).to(torch.bfloat16)
    assert layer._marlin_proj(x, "o", w) is None
    assert layer._marlin_o_failed is True
    assert layer._marlin_proj(x, "o", w) is None


def test_fp8_proj_tensorwise_and_per_token(dev, layer, monkeypatch):
    g = torch.Generator(device=dev).manual_seed(2)
    w = (torch.randn((512, 1024), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((300, 1024), generator=g, device=dev).to(torch.bfloat16)
    assert layer._fp8_proj(x, "gu", w) is None  # off by default
    monkeypatch.setenv("TORCHINFERNO_FP8_PREFILL", "1")
    y = layer._fp8_proj(x, "gu", w)
    ref = x.float() @ w.float().t()
    torch.testing.assert_close(y.float(), ref, atol=1.0, rtol=0.15)
    assert layer._fp8_gu_wq.dtype == torch.float8_e4m3fn
    from torchinferno_amd.kernels import fp8 as tf8
    assert tf8.is_tiled_weight(layer._fp8_gu_wq)  # the cache holds the GEMM's tiled layout
    wq_rows, sb_rows = tf8.quantize_weight_fp8(w)
    assert torch.equal(y, tf8.fp8_prefill_linear(x, wq_rows, sb_rows))  # same bits as [N, K]
    assert layer._fp8_proj(x[:200], "gu", w) is None  # M <= 256 gate
    monkeypatch.setenv("TORCHINFERNO_FP8_PER_TOKEN_SCALE", "1")
    out = torch.empty((300, 512), dtype=torch.bfloat16, device=dev)
    y2 = layer._fp8_proj(x, "down", w, out=out)
    assert y2 is out
    torch.testing.assert_close(out.float(), ref, atol=1.0, rtol=0.15)
    assert layer._fp8_per_token_down_ws.shape == (1, 512)


def test_fp8_decode_static_scale(dev, layer, monkeypatch):
    monkeypatch.setenv("TORCHINFERNO_FP8_DECODE", "1")
    g = torch.Generator(device=dev).manual_seed(3)
    w = (torch.randn((256, 512), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn((16, 1, 512), generator=g, device=dev).to(torch.bfloat16)
    y = layer._fp8_proj(x, "gu", w)
    assert y.shape == (16, 1, 256)
    assert layer._fp8_gu_decode_activation_scale.numel() == 1  # cached static scale (margin 4)
    torch.testing.assert_close(y.float(), (x.float() @ w.float().t()), atol=1.0, rtol=0.3)


def test_custom_ops_opcheck(dev):
    from torchinferno_amd import ops  # noqa: F401
    from torchinferno_amd.kernels import fp8 as tf8
    from torchinferno_amd.kernels import int4 as ti4
    g = torch.Generator(device=dev).manual_seed(5)
    a = torch.randn((4, 256), generator=g, device=dev).to(torch.bfloat16)
    q, s = ti4.quantize_to_int4(torch.randn((256, 128), generator=g, device=dev).to(torch.bfloat16))
    ws = ti4.make_workspace(128, dev, size_k=256, max_m=4)
    torch.library.opcheck(torch.ops.torchinferno_amd.w4a16_mm, (a, q, s, ws, 128, 256),
                          test_utils=("test_schema", "test_faketensor"))
    wq, wsc = tf8.quantize_weight_fp8_per_channel(torch.randn((128, 256), generator=g, device=dev).to(torch.bfloat16))
    # torch's schema checker multiplies tensors to detect mutation, which it cannot
    # do on float8 tensors; ops with e4m3 operands get the fake-tensor check only.
    torch.library.opcheck(torch.ops.torchinferno_amd.fp8_per_token_linear, (a, wq, wsc),
                          test_utils=("test_faketensor",))
    torch.library.opcheck(torch.ops.torchinferno_amd.act_quant, (a, 128, False),
                          test_utils=("test_faketensor",))
    xq, xs = tf8.quantize_activation_fp8_per_token(a)
    out = torch.empty((4, 128), dtype=torch.bfloat16, device=dev)
    torch.ops.torchinferno_amd.fp8_scaled_mm_out(out, xq, wq.t(), xs, wsc)
    assert torch.equal(out, tf8.fp8_per_token_linear_quantized(xq, xs, wq, wsc, out_dtype=torch.bfloat16))
