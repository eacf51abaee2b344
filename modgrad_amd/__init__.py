"""modgrad_amd: MI355X-native (gfx950) Q4_K quantized matvec for modgrad.

The product is libmodgrad_q4k.so (C ABI in include/modgrad_q4k.h, HIP kernels
in modgrad_amd/csrc). This package holds its build script and the host-side
mirror of the reference's Q4_K device interface (modgrad_amd.q4k).
"""
__version__ = "0.1.0"
