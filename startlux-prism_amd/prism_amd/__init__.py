"""prism_amd: StartLux-Prism's quantized linear-layer hot path, native on MI355X (gfx950).

Modules mirror the reference's kernel ops (startlux_prism/kernels/): quant (activation producers), w8a8 (Q8_0 /
per-channel W8A8 GEMM), w4a8 (Q4_K / Q6_K W4A8 GEMM), mxfp4 (MXFP4 GEMM and its quantizers); gguf_formats holds the
weight formats, weights the load-time step from a GGUF tensor's bytes to the device layouts, dispatch the MI355X
tuning tables (measured by tune).  All compute runs in libprism_amd.so (hand-written HIP for gfx950, C ABI in
include/prism_amd.h); there is no CPU fallback.
"""
from . import _lib, dispatch, gguf_formats, mxfp4, quant, w4a8, w8a8, weights  # noqa: F401

__all__ = ["gguf_formats", "quant", "w8a8", "w4a8", "mxfp4", "weights", "dispatch"]
