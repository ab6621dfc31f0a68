"""Name-compatible alias of :mod:`kvquant.hip_kernels`.

Callers written against src/kvquant/triton_kernels.py import from this module
path unchanged; there is no Triton here -- the functions are the gfx950 HIP
kernels of :mod:`kvquant.hip_kernels`.
"""
from .hip_kernels import (  # noqa: F401
    pack_keys_per_channel,
    pack_values_per_token,
    unpack_keys_per_channel,
    unpack_values_per_token,
)
