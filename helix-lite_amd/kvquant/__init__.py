"""KVQuant-style nuq KV-cache quantisation on MI355X (gfx950).

Drop-in for the reference's ``kvquant`` package (src/kvquant/__init__.py:23-33):
the CPU-spec functions, the scale containers, the per-head and batched kernel
families (``kvquant.triton_kernels`` / ``kvquant.triton_batched`` keep their
module paths), the compact pool and the Quest selector -- all on hand-written
HIP kernels.
"""
from .nuq import dequantize_nuq, find_outliers, quantize_nuq  # noqa: F401
from .scales import KVScales, PerChannelScale, PerTokenScale  # noqa: F401

__all__ = [
    "quantize_nuq",
    "dequantize_nuq",
    "find_outliers",
    "KVScales",
    "PerChannelScale",
    "PerTokenScale",
]
