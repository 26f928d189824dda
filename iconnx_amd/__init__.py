"""iconnx_amd — MI355X (gfx950) implementation of iconnx's dynamically-quantized linear path.

DynamicQuantizeLinear, MatMulInteger (int8 MFMA) and the dequant / bias / elementwise
epilogue, as hand-written HIP kernels behind the C ABI in include/iconnx_hip.h
(libiconnx_hip.so, built ahead of time by ``python -m iconnx_amd.build``).

``iconnx_amd.ops`` mirrors the reference's per-op ``gpu_*`` wrappers on torch device
tensors.  Importing this package does not touch the GPU; the first op call loads the
library and fails loudly if it has not been built.
"""
from ._lib import IconnxError, LIB_PATH, header_symbols, lib  # noqa: F401

__all__ = ["IconnxError", "LIB_PATH", "header_symbols", "lib"]
