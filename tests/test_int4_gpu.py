"""GPU parity of the int4 W4A16 path against the CPU oracle (oracle/int4.py).

Bar: dequantized weights bit-exact; GEMM max|y - ref| <= 1e-2 * max|ref|
(fp32-accumulated reference, fp16/bf16 output), the north-star tolerance.
Shapes: BASELINE config 0 (fp16, M=16, K=N=4096, seed 0), config 1 (bf16,
gate_up K=4096 N=28672 and down K=14336 N=4096, M in {1, 8, 32, 128}), ragged
M, the reference test's shapes (tests/test_marlin_int4.py:52-70).
"""
import numpy as np
import pytest
import torch

from oracle import int4 as oint4
from oracle.numerics import round_to
from tests._problems import int4_problem, to_np32

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _setup(m, k, n, dtype, seed, dev):
    from torchinferno_amd.kernels import int4 as ti4
    a, codes, scales = int4_problem(m, k, n, dtype, seed)
    qweight = ti4.pack_int4(codes)
    pw, ps = ti4.repack_int4(qweight.to(dev), scales.to(dev))
    ws = ti4.make_workspace(n, dev, size_k=k, max_m=max(m, 1))
    return a, qweight, scales, pw, ps, ws


def _rel_err(y, ref):
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dequant_bit_exact(dev, dtype):
    from torchinferno_amd.kernels import int4 as ti4
    k, n = 512, 192
    _, qweight, scales, pw, ps, _ = _setup(1, k, n, dtype, 7, dev)
    got = ti4.dequantize_int4(pw, ps, k, n).cpu().numpy()
    ref = oint4.dequant_int4(qweight.numpy(), to_np32(scales))
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _run_gemm(dev, m, k, n, dtype, seed):
    from torchinferno_amd.kernels import int4 as ti4
    a, qweight, scales, pw, ps, ws = _setup(m, k, n, dtype, seed, dev)
    out = ti4.int4_mm(a.to(dev), pw, ps, ws, n, k)
    torch.cuda.synchronize()
    ref = oint4.w4a16_reference(to_np32(a), qweight.numpy(), to_np32(scales))
    return out, ref


@pytest.mark.parametrize("m", [16])
def test_config0_fp16(dev, m):
    print(f"[int4] config0 M={m}", flush=True)
    out, ref = _run_gemm(dev, m, 4096, 4096, torch.float16, 0)
    assert out.dtype == torch.float16 and out.shape == (m, 4096)
    err = _rel_err(out.float().cpu().numpy(), ref)
    assert err <= TOL, err
    # Output rounding bound: a correct kernel is within a few fp16 ulps of the
    # rounded fp32 reference.
    assert err <= 2e-3, err


@pytest.mark.parametrize("k,n", [(4096, 28672), (14336, 4096)])
@pytest.mark.parametrize("m", [1, 8, 32, 128])
def test_config1_bf16(dev, m, k, n):
    print(f"[int4] config1 M={m} K={k} N={n}", flush=True)
    out, ref = _run_gemm(dev, m, k, n, torch.bfloat16, 1)
    err = _rel_err(out.float().cpu().numpy(), ref)
    assert err <= TOL, err


@pytest.mark.parametrize("m", [1, 2, 15, 17, 33, 63, 65, 100, 129, 200])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_ragged_m(dev, m, dtype):
    print(f"[int4] ragged M={m} {dtype}", flush=True)
    out, ref = _run_gemm(dev, m, 1024, 320, dtype, 100 + m)
    err = _rel_err(out.float().cpu().numpy(), ref)
    assert err <= TOL, err


@pytest.mark.parametrize("n,k", [(7168, 8192), (8192, 3584)])
def test_reference_marlin_shapes_rtn(dev, n, k):
    """tests/test_marlin_int4.py:52-70: RTN-quantized w = randn*0.02, a = randn(48, K),
    seed 0, mean-abs relative error < 0.03 vs the dequant reference of the *original*
    weights' quantization."""
    from torchinferno_amd.kernels import int4 as ti4
    print(f"[int4] reference shape N={n} K={k}", flush=True)
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(k, n, generator=g) * 0.02).to(torch.bfloat16)
    a = torch.randn(48, k, generator=g).to(torch.bfloat16)
    q, s = ti4.quantize_int4_rtn(w, 128, torch.bfloat16)
    oq, os_ = oint4.quantize_int4_rtn(round_to(w.float().numpy(), "fp16"), 128, "bf16")
    assert np.array_equal(q.numpy(), oq)
    assert np.array_equal(s.float().numpy(), os_)
    pw, ps = ti4.repack_int4(q.to(dev), s.to(dev))
    ws = ti4.make_workspace(n, dev, size_k=k, max_m=48)
    out = ti4.marlin_int4_mm(a.to(dev), pw, ps, ws, n, k).float().cpu().numpy()
    ref = oint4.w4a16_reference(to_np32(a), oq, os_)
    rel = np.abs(out - ref).mean() / np.abs(ref).mean()
    assert rel < 0.03
    assert _rel_err(out, ref) <= TOL


def test_out_buffer_contract_and_workspace_reuse(dev):
    """Caller-owned out is written in place (tests/test_marlin_int4.py:15-37); a
    shared workspace stays valid across calls of different M (ticket reset)."""
    from torchinferno_amd.kernels import int4 as ti4
    k, n = 14336, 4096
    a, qweight, scales, pw, ps, ws = _setup(32, k, n, torch.bfloat16, 3, dev)
    ad = a.to(dev)
    out = torch.empty((32, n), dtype=torch.bfloat16, device=dev)
    ptr = out.data_ptr()
    r1 = ti4.int4_mm(ad, pw, ps, ws, n, k, out=out)
    assert r1 is out and out.data_ptr() == ptr
    first = out.clone()
    a5 = ad[:5].contiguous()
    r2 = ti4.int4_mm(a5, pw, ps, ws, n, k)
    r3 = ti4.int4_mm(ad, pw, ps, ws, n, k)
    r4 = ti4.int4_mm(a5, pw, ps, ti4.make_workspace(n, dev, size_k=k, max_m=5), n, k)
    torch.cuda.synchronize()
    assert torch.equal(first, r3), "nondeterministic or workspace not reset"
    # Same M, shared vs fresh workspace: identical bits (fixed split order).
    assert torch.equal(r2, r4)
    # Different M may take a different split plan (another fp32 summation
    # order), so rows agree to the output tolerance, not bit for bit.
    ref = first[:5].float()
    assert float((r2.float() - ref).abs().max() / ref.abs().max()) <= TOL
    with pytest.raises(ValueError):
        ti4.int4_mm(ad, pw, ps, ws, n, k, out=torch.empty((32, n), dtype=torch.float16, device=dev))


def test_unsupported_shape_raises(dev):
    from torchinferno_amd import _lib
    from torchinferno_amd.kernels import int4 as ti4
    assert not ti4.int4_supports_shape(16032, 8192)
    a = torch.zeros((4, 256), dtype=torch.bfloat16, device=dev)
    pw = torch.zeros((100 * 256 // 8,), dtype=torch.int32, device=dev)
    ps = torch.zeros((2, 100), dtype=torch.bfloat16, device=dev)
    with pytest.raises(_lib.TiUnsupported):
        ti4.int4_mm(a, pw, ps, None, 100, 256)


@pytest.mark.parametrize("k,n", [(4096, 28672), (14336, 4096)])
@pytest.mark.parametrize("m", [24, 48, 64])
def test_decode_kernel_rows(dev, m, k, n):
    """Rows 17..64 run the LDS-DMA decode kernel (int4_decode.hip)."""
    print(f"[int4] decode M={m} K={k} N={n}", flush=True)
    out, ref = _run_gemm(dev, m, k, n, torch.bfloat16, 11)
    assert _rel_err(out.float().cpu().numpy(), ref) <= TOL


# Every template variant of the decode kernel, forced through the plan override
# ("nt:wk:ring:splits"), on a ragged problem; rows 3 / 13 / 29 stage 4 / 16 / 32 rows.
_DECODE_PLANS = ["1:1:3:1", "2:1:4:3", "4:1:6:1", "1:2:3:2", "2:2:6:1", "4:2:4:2",
                 "1:4:4:1", "2:4:3:4", "4:4:3:1"]


@pytest.mark.parametrize("plan", _DECODE_PLANS)
@pytest.mark.parametrize("m", [3, 13, 29, 45])
def test_decode_kernel_plans(dev, monkeypatch, plan, m):
    print(f"[int4] decode plan {plan} M={m}", flush=True)
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MIN_M", "1")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_WAVES", "4")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_PLAN", plan)
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MR", "4" if m <= 4 else ("16" if m <= 16 else "32"))
    out, ref = _run_gemm(dev, m, 2048, 512, torch.float16 if m % 2 else torch.bfloat16, 20 + m)
    assert _rel_err(out.float().cpu().numpy(), ref) <= TOL


# Tall tiles (64 / 128 staged rows): each instantiated (nt, wk, ring) with and
# without split-K, ragged M, both activation dtypes.
_TALL_PLANS = ["2:2:2:1", "4:1:2:1", "4:1:3:2", "2:1:3:1", "2:1:4:3", "2:1:2:1", "2:1:2:2"]


@pytest.mark.parametrize("plan", _TALL_PLANS)
@pytest.mark.parametrize("mr,m", [(64, 40), (64, 100), (128, 77), (128, 128), (128, 200)])
def test_decode_kernel_tall_tiles(dev, monkeypatch, plan, mr, m):
    print(f"[int4] tall plan {plan} MR={mr} M={m}", flush=True)
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_WAVES", "4")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MIN_M", "1")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MAX_M", "4096")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MR", str(mr))
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_PLAN", plan)
    out, ref = _run_gemm(dev, m, 2048, 512, torch.float16 if m % 2 else torch.bfloat16, 30 + m)
    assert _rel_err(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("m", [5, 8, 16])
def test_decode_four_row_override_ignored_above_four_rows(dev, monkeypatch, m):
    """A forced 4-row tile (TI_ROCM_W4A16_DECODE_MR=4) stages only 4 activation
    rows, so the plan keeps it for M <= 4 only; larger M falls back to 16 rows."""
    print(f"[int4] decode MR=4 override M={m}", flush=True)
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MIN_M", "1")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MR", "4")
    out, ref = _run_gemm(dev, m, 2048, 512, torch.bfloat16, 50 + m)
    assert _rel_err(out.float().cpu().numpy(), ref) <= TOL


# 8-wave tiles (two waves per SIMD, the K range split between them): every
# instantiated (mr, nt, wk, ring), with and without split-K, ragged M, both
# dtypes, narrow and wide N.
@pytest.mark.parametrize("plan", ["64/4:2:2:1", "64/4:2:2:3", "64/2:2:2:1", "64/2:2:3:1", "64/2:2:3:2",
                                  "32/4:4:2:1", "32/4:4:2:2", "32/2:2:3:1", "32/2:4:3:2", "32/1:4:3:1",
                                  "32/1:4:3:3", "16/4:2:3:1", "16/4:2:3:2", "16/2:2:4:1", "16/2:4:4:3",
                                  "16/1:4:6:2"])
@pytest.mark.parametrize("m,n", [(40, 512), (64, 1024), (100, 768), (128, 512), (21, 256)])
def test_decode_kernel_eight_waves(dev, monkeypatch, plan, m, n):
    print(f"[int4] 8-wave plan {plan} M={m} N={n}", flush=True)
    mr, plan = plan.split("/")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MIN_M", "1")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MAX_M", "4096")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MR", mr)
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_WAVES", "8")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_PLAN", plan)
    out, ref = _run_gemm(dev, m, 2048, n, torch.float16 if m % 2 else torch.bfloat16, 60 + m)
    assert _rel_err(out.float().cpu().numpy(), ref) <= TOL


# 16-wave tiles (four waves per SIMD): every instantiated (mr, nt, wk, ring),
# with and without split-K, ragged M, both dtypes.
@pytest.mark.parametrize("plan", ["64/2:2:2:1", "64/2:2:2:3", "32/2:4:2:1", "32/2:4:2:2", "32/1:4:3:1",
                                  "32/1:4:3:3", "16/2:4:3:1", "16/2:4:3:2", "16/1:4:4:1", "16/1:4:4:3"])
@pytest.mark.parametrize("m,n", [(40, 512), (100, 1024), (21, 256), (7, 512)])
def test_decode_kernel_sixteen_waves(dev, monkeypatch, plan, m, n):
    print(f"[int4] 16-wave plan {plan} M={m} N={n}", flush=True)
    mr, plan = plan.split("/")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MIN_M", "1")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MAX_M", "4096")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_MR", mr)
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_WAVES", "16")
    monkeypatch.setenv("TI_ROCM_W4A16_DECODE_PLAN", plan)
    out, ref = _run_gemm(dev, m, 2048, n, torch.float16 if m % 2 else torch.bfloat16, 80 + m)
    assert _rel_err(out.float().cpu().numpy(), ref) <= TOL



# (nt:waves:depth:splits, M) for every instantiated streaming-kernel configuration
# (int4_stream.hip), forced through TI_ROCM_W4A16_STREAM on a small problem: ragged
# M inside the row tile, K ranges that do not divide evenly over the waves, and
# the split-K ticket reduction.
_STREAM_CASES = [("7:8:2:1", 5), ("7:8:2:1", 29), ("7:16:1:1", 11), ("2:8:4:2", 8), ("4:8:2:4", 13),
                 ("4:16:1:4", 27), ("1:8:4:1", 3), ("1:16:2:1", 1), ("2:16:1:2", 20), ("2:8:4:3", 1)]


@pytest.mark.parametrize("plan,m", _STREAM_CASES)
def test_stream_kernel_configs(dev, monkeypatch, plan, m):
    import ctypes
    from torchinferno_amd import _lib
    from torchinferno_amd.kernels import int4 as ti4
    nt = int(plan.split(":")[0])
    k, n = 128 * 19, 16 * nt * 8
    monkeypatch.setenv("TI_ROCM_W4A16_STREAM", plan)
    buf = ctypes.create_string_buffer(256)
    _lib.lib().ti_w4a16_plan_name(m, n, k, 128, buf, 256)
    print(f"[int4] stream {plan} M={m}: {buf.value.decode()}", flush=True)
    assert buf.value.startswith(b"w4a16_stream_kernel"), buf.value
    a, qweight, scales, pw, ps, ws = _setup(m, k, n, torch.bfloat16, m + nt, dev)
    out = ti4.int4_mm(a.to(dev), pw, ps, ws, n, k)
    out2 = ti4.int4_mm(a.to(dev), pw, ps, ws, n, k)
    torch.cuda.synchronize()
    ref = oint4.w4a16_reference(to_np32(a), qweight.numpy(), to_np32(scales))
    assert _rel_err(out.float().cpu().numpy(), ref) <= TOL
    assert torch.equal(out, out2)  # deterministic, tickets left at zero
