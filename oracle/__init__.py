"""CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of TorchInferno's quantized
projections (int4 W4A16 group-128, FP8 W8A8 per-token/per-channel, DeepSeek
128x128 block-scaled FP8, routed FP8 MoE).  Each function cites the reference
file:line it follows.  It is the *checker*: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it.  The product path (``torchinferno_amd``) never imports, calls or falls back
to anything here.

Pinning status (what independently checks each function) is recorded in the
module docstrings and in tests/test_oracle_*.py.
"""
