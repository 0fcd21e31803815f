"""The C ABI allocates nothing and clears nothing with memsets (split-K tickets
are left at zero by the kernels themselves), so calls can be captured into a HIP
graph.  Captured int4 (split-K), FP8 (split-K), fused-producer and MoE calls, and
the power-of-two (E8M0) block GEMM (split-K) and MoE, are
replayed several times, with eager work and synchronizations between the
replays, and every replay must equal the eager result bit for bit."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(dev, monkeypatch):
    from torchinferno_amd.kernels import fp8 as tf8
    from torchinferno_amd.kernels import fused
    from torchinferno_amd.kernels import int4 as ti4
    from torchinferno_amd.kernels import moe as tmoe
    from tests.test_moe_gpu import _make_experts
    from tests.test_pow2_gpu import _fp8_experts_pow2
    from torchinferno_amd.kernels import block_fp8 as tb

    g = torch.Generator(device=dev).manual_seed(3)
    # int4, a split-K plan (narrow N, deep K)
    k4, n4, m4 = 14336, 512, 4
    q, s = ti4.quantize_to_int4((torch.randn((k4, n4), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    ws4 = ti4.make_workspace(n4, dev, size_k=k4, max_m=m4)
    a4 = torch.randn((m4, k4), generator=g, device=dev).to(torch.bfloat16)
    assert ti4.workspace_bytes(m4, n4, k4) > 0, "the case must exercise split-K"
    # FP8 row/col, a split-K plan (M=1)
    wq, wsc = tf8.quantize_weight_fp8_per_channel(
        (torch.randn((1024, 8192), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    x8 = torch.randn((1, 8192), generator=g, device=dev).to(torch.bfloat16)
    # fused producer, MoE
    gu = torch.randn((6, 2 * 2048), generator=g, device=dev).to(torch.bfloat16)
    ex = _make_experts(8, 256, 256, 5, dev)
    xm = torch.randn((12, 256), generator=g, device=dev).to(torch.bfloat16)
    logits = torch.randn((12, 8), generator=g, device=dev)
    # power-of-two scales: a DSv4 block linear (M=3: a split-K plan) and MoE
    ex2 = _fp8_experts_pow2(8, 256, 256, 6, dev)
    # finite e4m3 codes only (0x7F and 0xFF are NaN)
    wb = (torch.randint(0, 0x7E, (512, 1024), generator=g, device=dev)
          | (torch.randint(0, 2, (512, 1024), generator=g, device=dev) << 7)).to(torch.uint8).view(torch.float8_e4m3fn)
    wbs = torch.exp2(torch.randint(-12, -8, (4, 8), generator=g, device=dev).float()).to(torch.float8_e8m0fnu)
    xb = torch.randn((3, 1024), generator=g, device=dev).to(torch.bfloat16)

    def run():
        y4 = ti4.int4_mm(a4, q, s, ws4, n4, k4)
        xq, xs = tf8.quantize_activation_fp8_per_token(x8)
        y8 = tf8.fp8_per_token_linear_quantized(xq, xs, wq, wsc, out_dtype=torch.bfloat16)
        fq, fs = fused.swiglu_fp8_per_token(*gu.split(2048, dim=-1))
        ym = tmoe.moe_forward(xm, logits, ex, 2)
        yb = tb.linear(xb, wb, wbs, "ue8m0")
        ym2 = tmoe.moe_forward(xm, logits, ex2, 2, scale_fmt="ue8m0")
        return y4, y8, fq.view(torch.uint8), fs, ym, yb, ym2

    eager = [t.clone() for t in run()]
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        run()  # warm-up on the capture stream (workspaces already sized)
    torch.cuda.current_stream(dev).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        outs = run()
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(outs, eager)):
            assert torch.equal(got, ref), f"replay {rep}: output {i} differs"
        # eager work between replays, using the same workspaces
        assert torch.equal(ti4.int4_mm(a4, q, s, ws4, n4, k4), eager[0])
        torch.cuda.synchronize()
