"""Name-compatible alias of :mod:`quest.hip_kernels` (no Triton here).

src/quest/triton_kernels.py:60-91 exposed ``page_upper_bound_triton``; this
module path keeps that import working.
"""
from .hip_kernels import page_upper_bound_triton  # noqa: F401
