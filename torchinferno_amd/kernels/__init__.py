"""Kernel API modules mirroring src/torchinferno/kernels/ of the reference."""
