"""Per-head nuq pack/unpack, (T,D) layout, on hand-written gfx950 kernels.

Drop-in for src/kvquant/triton_kernels.py:96-339 (same names, arguments,
returned tensors and assertion errors).  Storage is the reference's
byte-per-code format: codes u8, outlier_v fp16 (0 where not an outlier),
outlier_m u8.  Codes are the strict-'<' ascending nearest pole over fp32
|v - pole| (src/kvquant/triton_kernels.py:66-75); outliers are v > upper or
v < lower in fp32.
"""
from __future__ import annotations

import torch

from helix_kv.ops import NuqLayerTables, nuq_pack_dense, nuq_unpack_dense


def _flat(values: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    T, D = values.shape
    return values.contiguous().view(T, 1, D), T, D


def pack_keys_per_channel(values: torch.Tensor, poles: torch.Tensor, upper: torch.Tensor,
                          lower: torch.Tensor):
    """(T,D) fp16 keys, poles (D,L), thresholds (D,) -> (codes, outlier_v, outlier_m) (T,D)."""
    assert values.is_cuda and values.dtype == torch.float16
    v, T, D = _flat(values)
    t = NuqLayerTables(poles.reshape(1, D, -1), upper.reshape(1, D), lower.reshape(1, D),
                       per_token=False)
    c, ov, om = nuq_pack_dense(v, t)
    return c.view(T, D), ov.view(T, D), om.view(T, D)


def unpack_keys_per_channel(codes: torch.Tensor, outlier_v: torch.Tensor,
                            outlier_m: torch.Tensor, poles: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`pack_keys_per_channel` -> (T,D) fp16."""
    assert codes.is_cuda and codes.dtype == torch.uint8
    T, D = codes.shape
    zeros = torch.zeros((1, D), dtype=torch.float32, device=codes.device)
    t = NuqLayerTables(poles.reshape(1, D, -1), zeros, zeros, per_token=False)
    out = nuq_unpack_dense(codes.contiguous().view(T, 1, D), outlier_v.reshape(T, 1, D),
                           outlier_m.reshape(T, 1, D), t)
    return out.view(T, D)


def pack_values_per_token(values: torch.Tensor, poles: torch.Tensor, upper: torch.Tensor,
                          lower: torch.Tensor):
    """(T,D) fp16 values, poles (T,L), thresholds (T,) -> (codes, outlier_v, outlier_m)."""
    assert values.is_cuda and values.dtype == torch.float16
    v, T, D = _flat(values)
    t = NuqLayerTables(poles.reshape(1, T, -1), upper.reshape(1, T), lower.reshape(1, T),
                       per_token=True)
    c, ov, om = nuq_pack_dense(v, t)
    return c.view(T, D), ov.view(T, D), om.view(T, D)


def unpack_values_per_token(codes: torch.Tensor, outlier_v: torch.Tensor,
                            outlier_m: torch.Tensor, poles: torch.Tensor) -> torch.Tensor:
    assert codes.is_cuda and codes.dtype == torch.uint8
    T, D = codes.shape
    zeros = torch.zeros((1, T), dtype=torch.float32, device=codes.device)
    t = NuqLayerTables(poles.reshape(1, T, -1), zeros, zeros, per_token=True)
    out = nuq_unpack_dense(codes.contiguous().view(T, 1, D), outlier_v.reshape(T, 1, D),
                           outlier_m.reshape(T, 1, D), t)
    return out.view(T, D)


__all__ = ["pack_keys_per_channel", "unpack_keys_per_channel", "pack_values_per_token",
           "unpack_values_per_token"]
