"""torchinferno_amd -- MI355X-native (gfx950) quantized-linear path for TorchInferno.

Hand-written HIP kernels (libti_quant.so, C ABI in include/ti_quant.h) behind
Python modules that mirror the reference's kernel API:

* ``kernels.int4``      -- int4 W4A16 group-128 (src/torchinferno/kernels/marlin.py)
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
