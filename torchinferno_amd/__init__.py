"""torchinferno_amd -- MI355X-native (gfx950) quantized-linear path for TorchInferno.

Hand-written HIP kernels (libti_quant.so, C ABI in include/ti_quant.h) behind
Python modules that mirror the reference's kernel API:

* ``kernels.int4``      -- int4 W4A16 group-128 (src/torchinferno/kernels/marlin.py)
* ``kernels.fp8``       -- FP8 W8A8 per-token/per-channel and tensorwise
                           (src/torchinferno/kernels/fp8.py, sgl_fp8_out.py)
* ``kernels.block_fp8`` -- DeepSeek 1x128 / 128x128 block FP8
                           (src/torchinferno/kernels/deepseek_v4_tilelang.py)
* ``kernels.moe``       -- softmax top-k router + routed FP8 MoE
                           (src/torchinferno/kernels/deepseek_v4_marlin.py)
* ``kernels.checkpoint`` -- GPTQ / AWQ int4 ingestion, prepared-weight files
* ``kernels.fused``     -- (add +) RMSNorm / SwiGLU -> per-token FP8 producers
                           (src/torchinferno/kernels/triton_ops.py:2127-2333)
* ``ops``               -- torch.library custom ops over the above
* ``hooks``             -- drop-in dispatch methods for the Llama3 / DeepSeek-V4 models
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
