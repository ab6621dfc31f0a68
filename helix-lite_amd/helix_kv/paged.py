"""Tensor-level wrappers of the paged compact pool (hkv_paged_*).

One layer's K or V side of the pool (D = 128, 16 slots per block):
  codes (NB, H, 16, D*bits/8) u8 -- page-head blocks of bit-packed codes;
  ocnt (NB, H) int32, oent (NB, H, cap) int32 (u32 bit patterns: fp16 value |
  channel << 16 | slot << 24) -- each page-head's outliers;
  kmin / kmax (NB, H, D) fp16 -- K page statistics of the dequantised values;
  status (1,) int32 -- bit 0 once a page-head's outliers exceeded cap.
Calls launch on torch's current stream and read nothing back.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as N
from .ops import NuqLayerTables

PAGE = 16
HEAD_DIM = 128


def bits_for_levels(levels: int) -> int:
    if levels <= 4:
        return 2
    if levels <= 16:
        return 4
    raise ValueError(f"{levels} levels exceed nuq4")


@dataclass
class PagedSide:
    codes: torch.Tensor
    ocnt: torch.Tensor
    oent: torch.Tensor
    bits: int
    kmin: torch.Tensor | None = None
    kmax: torch.Tensor | None = None
    status: torch.Tensor | None = None

    @property
    def num_blocks(self) -> int:
        return int(self.codes.shape[0])

    @property
    def heads(self) -> int:
        return int(self.codes.shape[1])

    @property
    def cap(self) -> int:
        return int(self.oent.shape[2])

    @staticmethod
    def empty(num_blocks: int, H: int, bits: int, cap: int, device, stats: bool = False,
              status: torch.Tensor | None = None) -> "PagedSide":
        dev = torch.device(device)
        D = HEAD_DIM
        side = PagedSide(
            codes=torch.zeros((num_blocks, H, PAGE, D * bits // 8), dtype=torch.uint8, device=dev),
            ocnt=torch.zeros((num_blocks, H), dtype=torch.int32, device=dev),
            oent=torch.zeros((num_blocks, H, max(cap, 0)), dtype=torch.int32, device=dev),
            bits=bits,
            status=status if status is not None else torch.zeros(1, dtype=torch.int32, device=dev))
        if stats:
            side.kmin = torch.full((num_blocks, H, D), float("inf"), dtype=torch.float16, device=dev)
            side.kmax = torch.full((num_blocks, H, D), float("-inf"), dtype=torch.float16, device=dev)
        return side


def paged_write(side: PagedSide, values: torch.Tensor, t: NuqLayerTables, slot_mapping: torch.Tensor,
                positions: torch.Tensor | None = None) -> None:
    """Write (T, H, 128) fp16 into the side's slots (hkv_paged_write); V
    (per-token scales) uses scale row min(positions[t], rows - 1)."""
    N.require_gpu(values, slot_mapping, side.codes)
    assert values.dtype == torch.float16, "values must be fp16"
    assert values.is_contiguous(), "values must be contiguous (T, H, D)"
    T = int(values.shape[0])
    H = side.heads
    if tuple(values.shape) != (T, H, HEAD_DIM):
        raise AssertionError(f"values must be ({T}, {H}, {HEAD_DIM}), got {tuple(values.shape)}")
    if t.levels > (1 << side.bits):
        raise AssertionError(f"{t.levels} levels do not fit in {side.bits} bits")
    if t.per_token and side.kmin is not None:
        raise AssertionError("page statistics are kept for K (per-channel scales) only")
    slots = slot_mapping.to(torch.int64).contiguous()
    if slots.numel() != T:
        raise AssertionError("slot_mapping must have one entry per token")
    pos = None
    if positions is not None:
        pos = positions.to(device=values.device, dtype=torch.int64).contiguous()
        if pos.numel() != T:
            raise AssertionError("positions must have one entry per token")
    if T == 0:
        return
    s = t.struct(pos)
    st = N.lib().hkv_paged_write(
        N.ptr(values), T, H, HEAD_DIM, side.bits, s, N.ptr(slots), side.num_blocks, PAGE,
        N.ptr(side.codes), N.ptr(side.ocnt), N.ptr(side.oent), side.cap, N.ptr(side.kmin),
        N.ptr(side.kmax), N.ptr(side.status), N.stream_of(values))
    N.check(st, "hkv_paged_write", AssertionError)


def paged_gather(side: PagedSide, t: NuqLayerTables, block_ids: torch.Tensor,
                 first_pos: torch.Tensor | None = None, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Dequantise blocks block_ids into (NK, 16, H, 128) fp16 (hkv_paged_gather);
    V rows min(first_pos[k] + slot, rows - 1)."""
    N.require_gpu(block_ids, side.codes)
    ids = block_ids.to(torch.int64).contiguous()
    NK = int(ids.numel())
    H = side.heads
    if out is None:
        out = torch.empty((NK, PAGE, H, HEAD_DIM), dtype=torch.float16, device=side.codes.device)
    if tuple(out.shape) != (NK, PAGE, H, HEAD_DIM) or out.dtype != torch.float16 or not out.is_contiguous():
        raise AssertionError(f"staging must be contiguous ({NK}, {PAGE}, {H}, {HEAD_DIM}) fp16")
    fp = None
    if t.per_token:
        if first_pos is None:
            raise AssertionError("per-token scales need block first positions")
        fp = first_pos.to(device=ids.device, dtype=torch.int64).contiguous()
        if fp.numel() != NK:
            raise AssertionError("one first position per kept block")
    if NK == 0:
        return out
    st = N.lib().hkv_paged_gather(
        N.ptr(side.codes), N.ptr(side.ocnt), N.ptr(side.oent), side.cap, side.num_blocks, PAGE, H,
        HEAD_DIM, side.bits, t.struct(), N.ptr(ids), N.ptr(fp), NK, N.ptr(out), N.stream_of(out))
    N.check(st, "hkv_paged_gather", AssertionError)
    return out
