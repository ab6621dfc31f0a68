"""Quest top-K block selection over the compact pool's block statistics.

Drop-in for src/kvquant/quest_selector.py:38-90: for one layer and one decode
query, the upper bound of every used block (from the pool's fp32
k_min / k_max), the per-head top-K with the first ``sink_blocks`` used blocks
as sinks, and the union over heads, returned as ascending block ids with
their first token positions (id * block_size).

The whole selection is one call into ``hkv_quest_select_blocks`` (bound,
top-K, union by flags over the pool's block ids, compaction).  As in the
reference, the number of selected blocks is data-dependent and the returned
tensors are sized by it, which reads one device integer (the reference's
``torch.unique`` synchronises the same way).
"""
from __future__ import annotations

import torch

from helix_kv import _native as N

from .compact_pool import CompactKVPool

_flags: dict[tuple, torch.Tensor] = {}


def _flag_buffer(nblocks: int, device) -> torch.Tensor:
    """Per-(device, stream) zeroed flags; every call leaves them zero."""
    dev = torch.device(device)
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    buf = _flags.get(key)
    if buf is None or buf.numel() < nblocks:
        buf = torch.zeros(max(nblocks, 16) + 16, dtype=torch.uint8, device=dev)
        _flags[key] = buf
    return buf


def select_top_blocks_for_layer(
    pool: CompactKVPool,
    layer_idx: int,
    query: torch.Tensor,           # (H, D) query for one decode step (head-first)
    used_block_ids: torch.Tensor,  # (NU,) int64 -- blocks holding this seq's tokens
    block_size: int,
    top_k: int,
    sink_blocks: int = 4,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Pick the union-of-heads top-K blocks the decode query attends to.

    Returns ``(selected_block_ids, block_first_positions)``, int64, ascending,
    on the query's device."""
    N.require_gpu(query, used_block_ids)
    H, D = pool.num_kv_heads, pool.head_size
    if query.dim() != 2 or tuple(query.shape) != (H, D):
        raise ValueError(f"query should be ({H}, {D}), got {tuple(query.shape)}")
    assert layer_idx < pool.num_layers
    used = used_block_ids.to(torch.int64).contiguous()
    NU = int(used.numel())
    q = query.float().contiguous()
    sinks = max(0, min(int(sink_blocks), NU))
    keep = max(0, min(int(top_k), NU - sinks))
    dev = query.device
    NB = pool.num_blocks
    scores = torch.empty((H, max(NU, 1)), dtype=torch.float32, device=dev)
    sel = torch.empty((max(sinks + keep, 1), H), dtype=torch.int64, device=dev)
    cap = max(1, min(NB, NU))
    out_ids = torch.empty(cap, dtype=torch.int64, device=dev)
    out_first = torch.empty(cap, dtype=torch.int64, device=dev)
    n_sel = torch.empty(1, dtype=torch.int64, device=dev)
    flags = _flag_buffer(NB, dev)
    kmin = pool.k_min[layer_idx]
    kmax = pool.k_max[layer_idx]
    st = N.lib().hkv_quest_select_blocks(
        N.ptr(q), N.dtype_code(q), H, N.ptr(kmin), N.ptr(kmax), N.dtype_code(kmin), NB, D,
        N.ptr(used), NU, int(top_k), int(sink_blocks), int(block_size), N.ptr(scores),
        N.ptr(sel), N.ptr(flags), N.ptr(out_ids), N.ptr(out_first), N.ptr(n_sel),
        N.stream_of(q))
    N.check(st, "hkv_quest_select_blocks", ValueError)
    n = int(n_sel.item())
    return out_ids[:n], out_first[:n]
