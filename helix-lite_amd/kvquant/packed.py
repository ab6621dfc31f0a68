"""The compact KV format: bit-packed nuq codes + CSR outliers, per layer.

The reference planned this format but stored one byte per code plus dense fp16
outliers plus a mask (src/kvquant/triton_kernels.py:7-18,
src/kvquant/compact_pool.py:11-12, :427-432).  Here each layer's K and V
become

* codes (T, H, D*bits/8) u8 -- nuq2 for layers whose scales have <= 4 levels,
  nuq4 for <= 16 (mixed files splice both, benchmarks/pr1c/mix_scales.py:59-68);
* CSR outliers over rows t*H + h: row_ptr (T*H+1) int32, col u8, val fp16.

Codes and outlier masks are bit-identical to the reference kernels' byte
format (src/kvquant/triton_batched.py:28-82 for K, the pool's clamped V rows
src/kvquant/compact_pool.py:160-218 for V).  Scales are prepared once per
device (:func:`device_tables`): poles and thresholds are copied and the
nearest-pole decision tables are built on the GPU.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from helix_kv.ops import CompactCodes, NuqLayerTables, nuq_pack_compact, nuq_unpack_compact

from .scales import KVScales


def bits_for_levels(levels: int) -> int:
    if levels <= 4:
        return 2
    if levels <= 16:
        return 4
    raise ValueError(f"{levels} levels exceed nuq4")


@dataclass
class LayerTables:
    k: NuqLayerTables
    v: NuqLayerTables

    @property
    def k_bits(self) -> int:
        return bits_for_levels(self.k.levels)

    @property
    def v_bits(self) -> int:
        return bits_for_levels(self.v.levels)


def device_tables(scales: KVScales, device) -> list[LayerTables]:
    """Per-layer device scales + decision tables for a KVScales."""
    out = []
    for ks, vs in zip(scales.per_layer_keys, scales.per_layer_values):
        k = NuqLayerTables(ks.poles.to(device), ks.upper_threshold.to(device),
                           ks.lower_threshold.to(device), per_token=False)
        v = NuqLayerTables(vs.poles.to(device), vs.upper_threshold.to(device),
                           vs.lower_threshold.to(device), per_token=True)
        k.ensure_tables()
        v.ensure_tables()
        out.append(LayerTables(k, v))
    return out


def pack_layer(key: torch.Tensor, value: torch.Tensor, lt: LayerTables, *, positions=None,
               pos_offset: int = 0, out: tuple[CompactCodes, CompactCodes] | None = None,
               capacity: int | None = None, sync: bool = True):
    """Quantise one layer's K and V (T,H,D) fp16 into the compact format.

    V uses scale row min(position, T_cal-1) with position = positions[t] or
    pos_offset + t.  Returns (K codes, V codes)."""
    ok, ov = out if out is not None else (None, None)
    ck = nuq_pack_compact(key, lt.k, lt.k_bits, capacity=capacity, out=ok, sync=sync)
    cv = nuq_pack_compact(value, lt.v, lt.v_bits, capacity=capacity, positions=positions,
                          pos_offset=pos_offset, out=ov, sync=sync)
    return ck, cv


def unpack_layer(ck: CompactCodes, cv: CompactCodes, lt: LayerTables, *, positions=None,
                 pos_offset: int = 0, out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """Inverse of :func:`pack_layer` -> (K, V) fp16 (T,H,D)."""
    ok, ov = out if out is not None else (None, None)
    k = nuq_unpack_compact(ck, lt.k, out=ok)
    v = nuq_unpack_compact(cv, lt.v, positions=positions, pos_offset=pos_offset, out=ov)
    return k, v


__all__ = ["LayerTables", "device_tables", "pack_layer", "unpack_layer", "bits_for_levels",
           "CompactCodes"]
