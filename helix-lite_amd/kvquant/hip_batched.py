"""Batched-head nuq pack/unpack, (T,H,D) layout, on gfx950 kernels.

Drop-in for src/kvquant/triton_batched.py:125-326: same names, arguments,
outputs and assertions.  Keys use per-(head, channel) poles (H,D,L); values
use per-(head, token) poles (H,T,L) that the caller has already gathered with
the tail clamp (src/kvquant/vllm_backend.py:151-155).
"""
from __future__ import annotations

import torch

from helix_kv.ops import NuqLayerTables, nuq_pack_dense, nuq_unpack_dense


def pack_keys_per_channel_batched(values: torch.Tensor, poles: torch.Tensor, upper: torch.Tensor,
                                  lower: torch.Tensor):
    """(T,H,D) fp16, poles (H,D,L), thresholds (H,D) -> codes, outlier_v, outlier_m (T,H,D)."""
    assert values.is_cuda and values.dtype == torch.float16
    assert values.is_contiguous(), "values must be contiguous (T, H, D)"
    t = NuqLayerTables(poles, upper, lower, per_token=False)
    return nuq_pack_dense(values, t)


def unpack_keys_per_channel_batched(codes: torch.Tensor, outlier_v: torch.Tensor,
                                    outlier_m: torch.Tensor, poles: torch.Tensor) -> torch.Tensor:
    assert codes.is_cuda and codes.dtype == torch.uint8
    assert codes.is_contiguous()
    H, D = int(poles.shape[0]), int(poles.shape[1])
    zeros = torch.zeros((H, D), dtype=torch.float32, device=codes.device)
    return nuq_unpack_dense(codes, outlier_v, outlier_m,
                            NuqLayerTables(poles, zeros, zeros, per_token=False))


def pack_values_per_token_batched(values: torch.Tensor, poles: torch.Tensor, upper: torch.Tensor,
                                  lower: torch.Tensor):
    """(T,H,D) fp16, poles (H,T,L) (already tail-extrapolated), thresholds (H,T)."""
    assert values.is_cuda and values.dtype == torch.float16
    assert values.is_contiguous()
    T, H, D = values.shape
    L = poles.shape[-1]
    assert poles.shape == (H, T, L), f"poles shape {poles.shape} != ({H},{T},{L})"
    t = NuqLayerTables(poles, upper, lower, per_token=True)
    return nuq_pack_dense(values, t)


def unpack_values_per_token_batched(codes: torch.Tensor, outlier_v: torch.Tensor,
                                    outlier_m: torch.Tensor, poles: torch.Tensor) -> torch.Tensor:
    assert codes.is_cuda and codes.dtype == torch.uint8
    assert codes.is_contiguous()
    H, Tt = int(poles.shape[0]), int(poles.shape[1])
    zeros = torch.zeros((H, Tt), dtype=torch.float32, device=codes.device)
    return nuq_unpack_dense(codes, outlier_v, outlier_m,
                            NuqLayerTables(poles, zeros, zeros, per_token=True))


__all__ = ["pack_keys_per_channel_batched", "unpack_keys_per_channel_batched",
           "pack_values_per_token_batched", "unpack_values_per_token_batched"]
