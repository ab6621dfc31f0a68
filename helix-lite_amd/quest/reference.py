"""Quest decode-time page selection on gfx950 kernels.

Drop-in for src/quest/reference.py:38-168 (same names, arguments, shapes and
ValueError checks).  The arithmetic is fixed so that results are exactly
reproducible:

* ``compute_page_stats``: amin/amax over the page-slot axis; -0 orders below
  +0; a NaN in a page-channel yields NaN.
* ``page_upper_bound``: sum_d clamp(q,0)*K_max + clamp(q,max=0)*K_min in fp32
  with products rounded before each add, the positive and negative parts summed
  separately in the canonical chunked order (chunks of 8 channels left to right,
  chunk sums combined by a halving tree) and added last; a zero bound is +0.
  The result has the promoted dtype of the inputs (fp16 inputs: the fp32 bound
  rounded once, whereas the reference rounds every fp16 product).
* ``topk_pages_with_sinks``: ties in the bound go to the lower page index; NaN
  ranks highest (as torch.topk does).
"""
from __future__ import annotations

import torch

from helix_kv.ops import quest_page_bound, quest_page_stats, quest_topk
from helix_kv.ops import selected_attention as _selected_attention


def compute_page_stats(K_pages: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(P, page, H, D) -> (K_min, K_max), each (P, H, D)."""
    if K_pages.dim() != 4:
        raise ValueError(f"expected (P, page, H, D), got {tuple(K_pages.shape)}")
    if K_pages.dtype not in (torch.float16, torch.float32):
        kmin, kmax = quest_page_stats(K_pages.float())
        return kmin.to(K_pages.dtype), kmax.to(K_pages.dtype)
    return quest_page_stats(K_pages)


def page_upper_bound(query: torch.Tensor, K_min: torch.Tensor, K_max: torch.Tensor) -> torch.Tensor:
    """(H, D) query, (P, H, D) page bounds -> (P, H) upper bound on max_t q.K[t]."""
    if query.dim() != 2:
        raise ValueError(f"query should be (H, D), got {tuple(query.shape)}")
    if K_min.shape != K_max.shape or K_min.dim() != 3:
        raise ValueError(
            f"K_min/K_max should be (P, H, D), got {tuple(K_min.shape)} and {tuple(K_max.shape)}")
    if query.shape[0] != K_min.shape[1] or query.shape[1] != K_min.shape[2]:
        raise ValueError(f"query {tuple(query.shape)} does not match K_min {tuple(K_min.shape)}")
    out_dtype = torch.promote_types(torch.promote_types(query.dtype, K_min.dtype), K_max.dtype)
    kdt = torch.float16 if (K_min.dtype == torch.float16 and K_max.dtype == torch.float16) \
        else torch.float32
    b = quest_page_bound(query, K_min.to(kdt), K_max.to(kdt),
                         out_dtype=torch.float16 if out_dtype == torch.float16 else torch.float32)
    return b if b.dtype == out_dtype else b.to(out_dtype)


def topk_pages_with_sinks(bound: torch.Tensor, k: int, sink_pages: int = 1) -> torch.Tensor:
    """(P, H) bound -> (sinks + k_eff, H) int64 page indices, ascending per head."""
    if bound.dim() != 2:
        raise ValueError(f"bound should be (P, H), got {tuple(bound.shape)}")
    return quest_topk(bound, k, sink_pages)


def selected_attention(query: torch.Tensor, K_pages: torch.Tensor, V_pages: torch.Tensor,
                       page_indices: torch.Tensor) -> torch.Tensor:
    """Attention of each head over its selected pages (src/quest/reference.py:136-168):
    head h attends with K head h and V head h % H_v over the pages
    page_indices[:, h]; fp32 softmax, (H, D_v) output in query's dtype."""
    return _selected_attention(query, K_pages, V_pages, page_indices)


__all__ = ["compute_page_stats", "page_upper_bound", "topk_pages_with_sinks",
           "selected_attention"]
