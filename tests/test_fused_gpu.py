"""Fused (add +) RMSNorm / SwiGLU -> per-token FP8 producers on the GPU: codes,
scales and the summed hidden state equal oracle/fused.py bit for bit, and the
reference test's restore tolerances hold (tests/test_conversion_and_kernels.py:
390-435 of the reference, same shapes and seed)."""
import numpy as np
import pytest
import torch

from oracle import fused as ofu
from oracle.numerics import e4m3_decode

pytestmark = pytest.mark.gpu

_ACT = {torch.bfloat16: "bf16", torch.float16: "fp16"}


def _np(t):
    return t.float().cpu().numpy()


def _codes(q):
    return q.reshape(-1, q.size(-1)).view(torch.uint8).cpu().numpy()


def test_reference_restore_tolerances(dev):
    from torchinferno_amd.kernels import fused
    torch.manual_seed(17)
    x = torch.randn((7, 64), device=dev, dtype=torch.bfloat16)
    residual = torch.randn_like(x)
    weight = torch.randn((64,), device=dev, dtype=torch.bfloat16)
    eps = 1e-5
    q, s = fused.triton_rms_norm_fp8_per_token(x, weight, eps)
    exp = x.float() * torch.rsqrt(x.float().square().mean(-1, keepdim=True) + eps) * weight.float()
    torch.testing.assert_close(q.float() * s, exp, atol=1.2e-1, rtol=1.3e-1)
    h, q2, s2 = fused.triton_add_rms_norm_fp8_per_token(x, residual, weight, eps)
    hs = x.float() + residual.float()
    exp2 = hs * torch.rsqrt(hs.square().mean(-1, keepdim=True) + eps) * weight.float()
    torch.testing.assert_close(h, x + residual, atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(q2.float() * s2, exp2, atol=1.2e-1, rtol=1.3e-1)
    gate, up = torch.randn((7, 128), device=dev, dtype=torch.bfloat16).split(64, dim=-1)
    q3, s3 = fused.triton_swiglu_fp8_per_token(gate, up)
    exp3 = torch.nn.functional.silu(gate.float()) * up.float()
    torch.testing.assert_close(q3.float() * s3, exp3, atol=1.2e-1, rtol=1.3e-1)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,n", [(1, 4096), (5, 8), (33, 2056), (3, 16384), (130, 8192), (2, 65536), (4, 24576)])
def test_rmsnorm_bit_exact(dev, dt, rows, n):
    from torchinferno_amd.kernels import fused
    g = torch.Generator(device=dev).manual_seed(rows * 7 + n)
    x = (torch.randn((rows, n), generator=g, device=dev) * 3).to(dt)
    r = torch.randn((rows, n), generator=g, device=dev).to(dt)
    w = (torch.rand((n,), generator=g, device=dev) + 0.5).to(dt)
    x[0, : n // 2] = 0  # a half-zero row
    eps = 1e-6
    q, s = fused.rms_norm_fp8_per_token(x, w, eps)
    oq, os_ = ofu.rms_norm_fp8_per_token(_np(x), _np(w), eps, _ACT[dt])
    assert np.array_equal(_codes(q), oq) and np.array_equal(s.cpu().numpy(), os_)
    h, q2, s2 = fused.add_rms_norm_fp8_per_token(x, r, w, eps)
    oh, oq2, os2 = ofu.add_rms_norm_fp8_per_token(_np(x), _np(r), _np(w), eps, _ACT[dt])
    assert h.dtype == dt and np.array_equal(_np(h), oh)
    assert np.array_equal(_codes(q2), oq2) and np.array_equal(s2.cpu().numpy(), os2)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,n", [(1, 14336), (4, 8), (17, 1032), (64, 4096), (2, 40000), (3, 28672)])
def test_swiglu_bit_exact_on_split_views(dev, dt, rows, n):
    from torchinferno_amd.kernels import fused
    g = torch.Generator(device=dev).manual_seed(rows + n)
    gu = (torch.randn((rows, 1, 2 * n), generator=g, device=dev) * 4).to(dt)
    gate, up = gu.split((n, n), dim=-1)  # strided rows, as the Llama3 MLP hands them over
    q, s = fused.swiglu_fp8_per_token(gate, up)
    assert q.shape == gate.shape and s.shape == (rows, 1)
    oq, os_ = ofu.swiglu_fp8_per_token(_np(gate).reshape(rows, n), _np(up).reshape(rows, n), _ACT[dt])
    assert np.array_equal(_codes(q), oq) and np.array_equal(s.cpu().numpy(), os_)


def test_swiglu_every_bf16_gate_value(dev):
    """Every finite bf16 gate value (all 2^16 bit patterns in order, 1,024 to a
    row -- rows of like exponents -- with inf / NaN patterns replaced by 0),
    up = 1 and up = -3: the bf16 path reads g / (1 + exp(-g)) from a per-workgroup table
    covering 2^-25 <= |g| < 128 and closed forms outside, and must equal the
    fp64 expression everywhere.  More rows than workgroups, so the
    row-striding loop runs too."""
    from torchinferno_amd.kernels import fused
    bits = np.arange(1 << 16, dtype=np.uint32)
    bits[((bits >> 7) & 0xFF) == 0xFF] = 0                # inf / NaN -> +0
    gate_np = (bits << 16).view(np.float32)
    gate = torch.from_numpy(gate_np.copy()).to(torch.bfloat16).reshape(64, 1024)
    gate = gate.repeat(9, 1).to(dev)                     # 576 rows > 512 workgroups
    for u in (1.0, -3.0):
        up = torch.full_like(gate, u)
        q, s = fused.swiglu_fp8_per_token(gate, up)
        oq, os_ = ofu.swiglu_fp8_per_token(_np(gate), _np(up), "bf16")
        assert np.array_equal(_codes(q), oq) and np.array_equal(s.cpu().numpy(), os_)


def test_zero_rows_and_errors(dev):
    from torchinferno_amd.kernels import fused
    x = torch.zeros((2, 64), device=dev, dtype=torch.bfloat16)
    w = torch.ones((64,), device=dev, dtype=torch.bfloat16)
    q, s = fused.rms_norm_fp8_per_token(x, w, 1e-6)  # all-zero rows: scale floor, zero codes
    assert torch.all(s == 1e-10) and not _codes(q).any()
    e = torch.empty((0, 64), device=dev, dtype=torch.bfloat16)
    q, s = fused.rms_norm_fp8_per_token(e, w, 1e-6)
    assert q.shape == (0, 64) and s.shape == (0, 1)
    with pytest.raises(ValueError):
        fused.rms_norm_fp8_per_token(x.float(), w, 1e-6)
    with pytest.raises(ValueError):
        fused.rms_norm_fp8_per_token(x, w[:32], 1e-6)
    with pytest.raises(ValueError):
        fused.add_rms_norm_fp8_per_token(x, x[:1], w, 1e-6)
    with pytest.raises(ValueError):
        fused.swiglu_fp8_per_token(x, x.half())
    with pytest.raises(ValueError):
        fused.swiglu_fp8_per_token(x.t(), x.t())
    wide = torch.zeros((1, 65544), device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        fused.swiglu_fp8_per_token(wide, wide)


def test_feeds_per_token_linear(dev):
    """SwiGLU -> FP8 -> per-token GEMM equals the GEMM on the separately quantized
    activation (the Llama3 down-projection chain, tensor_parallel.py:3183-3200)."""
    from torchinferno_amd.kernels import fp8 as tf8
    from torchinferno_amd.kernels import fused
    g = torch.Generator(device=dev).manual_seed(9)
    gu = torch.randn((8, 2048), generator=g, device=dev).to(torch.bfloat16)
    gate, up = gu.split(1024, dim=-1)
    wq, ws = tf8.quantize_weight_fp8_per_channel(
        (torch.randn((512, 1024), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    q, s = fused.swiglu_fp8_per_token(gate, up)
    act = (torch.nn.functional.silu(gate.float()) * up.float()).to(torch.bfloat16)
    q2, s2 = tf8.quantize_activation_fp8_per_token(act)
    y1 = tf8.fp8_per_token_linear_quantized(q, s, wq, ws, out_dtype=torch.bfloat16)
    y2 = tf8.fp8_per_token_linear_quantized(q2, s2, wq, ws, out_dtype=torch.bfloat16)
    torch.testing.assert_close(y1.float(), y2.float(), atol=2e-2, rtol=5e-2)


def test_ops_and_patch(dev):
    import types
    from torchinferno_amd import hooks, ops  # noqa: F401
    from torchinferno_amd.kernels import fused
    x = torch.randn((4, 256), device=dev, dtype=torch.bfloat16)
    w = torch.rand((256,), device=dev, dtype=torch.bfloat16)
    torch.library.opcheck(torch.ops.torchinferno_amd.add_rms_norm_fp8_per_token, (x, x, w, 1e-6),
                          test_utils=("test_faketensor",))
    torch.library.opcheck(torch.ops.torchinferno_amd.swiglu_fp8_per_token, (x, x),
                          test_utils=("test_faketensor",))
    mod = types.ModuleType("fake_triton_ops")
    undo = hooks.patch_fused_producers(mod)
    assert mod.triton_swiglu_fp8_per_token is fused.swiglu_fp8_per_token
    undo()
    assert not hasattr(mod, "triton_swiglu_fp8_per_token")


def test_e4m3_hardware_encoder_matches_software_everywhere_in_range(dev):
    """The gfx950 fp32 -> e4m3 conversion the producers use agrees with the
    round-to-nearest-even software encoder (itself pinned against the oracle)
    on every finite fp32 value with |x| < 480: all 2^32 bit patterns."""
    from torchinferno_amd import _lib
    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    _lib.call("ti_fp8_e4m3_selfcheck", counts.data_ptr(), _lib.stream_of(counts))
    torch.cuda.synchronize()
    in_range, outside = (int(v) for v in counts.cpu())
    print(f"[fp8] e4m3 encoders disagree on {in_range} in-range and {outside} other inputs", flush=True)
    assert in_range == 0


def test_bf16_hardware_rounding_matches_software_on_every_number(dev):
    """Every kernel rounds fp32 to bf16 with the gfx950 conversion instruction;
    it equals the integer round-to-nearest-even (NaN -> quiet NaN) rounding on
    all 2^32 fp32 bit patterns."""
    from torchinferno_amd import _lib
    counts = torch.zeros(2, dtype=torch.int64, device=dev)
    _lib.call("ti_bf16_round_selfcheck", counts.data_ptr(), _lib.stream_of(counts))
    torch.cuda.synchronize()
    num, nan = (int(v) for v in counts.cpu())
    print(f"[bf16] roundings disagree on {num} numbers and {nan} NaNs", flush=True)
    assert num == 0 and nan == 0
