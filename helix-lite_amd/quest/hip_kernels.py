"""Fused Quest upper bound with fp16 output.

Drop-in for ``page_upper_bound_triton`` (src/quest/triton_kernels.py:60-91):
fp32 accumulation in the canonical order of :mod:`quest.reference`, one
rounding to fp16 at the end.
"""
from __future__ import annotations

import torch

from helix_kv.ops import quest_page_bound


def page_upper_bound_triton(query: torch.Tensor, K_min: torch.Tensor,
                            K_max: torch.Tensor) -> torch.Tensor:
    if query.dim() != 2 or K_min.dim() != 3 or K_max.shape != K_min.shape:
        raise ValueError(
            f"shape mismatch: query={tuple(query.shape)}, "
            f"K_min={tuple(K_min.shape)}, K_max={tuple(K_max.shape)}")
    H, D = query.shape
    P = K_min.shape[0]
    assert K_min.shape == (P, H, D), \
        f"K_min should be (P, H, D)=({P},{H},{D}), got {tuple(K_min.shape)}"
    assert query.is_cuda and K_min.is_cuda and K_max.is_cuda
    return quest_page_bound(query.to(torch.float16), K_min.to(torch.float16),
                            K_max.to(torch.float16), out_dtype=torch.float16)


__all__ = ["page_upper_bound_triton"]
