"""Name-compatible alias of :mod:`kvquant.hip_batched`.

Callers written against src/kvquant/triton_batched.py import from this module
path unchanged; the functions are the gfx950 HIP kernels of
:mod:`kvquant.hip_batched` (no Triton).
"""
from .hip_batched import (  # noqa: F401
    pack_keys_per_channel_batched,
    pack_values_per_token_batched,
    unpack_keys_per_channel_batched,
    unpack_values_per_token_batched,
)
