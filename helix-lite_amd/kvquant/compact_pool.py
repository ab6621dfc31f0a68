"""The paged compact KV pool, on gfx950 kernels.

Drop-in for src/kvquant/compact_pool.py:398-537 (``CompactKVPool``): the same
constructor, the same public tensors -- ``k_codes, v_codes`` u8,
``k_outv, v_outv`` fp16 (0 where not an outlier), ``k_outm, v_outm`` u8, each
(L, NB, BS, H, D), and ``k_min, k_max`` (L, NB, H, D) fp32 initialised to
+inf / -inf -- and the same two methods:

* ``write_kv(layer_idx, key, value, slot_mapping, abs_positions)`` packs a
  (T,H,D) batch into the slots of the pool (slot < 0 skipped), V with scale
  row min(abs_position, T_cal - 1), and folds the reconstructed K into each
  touched block's min / max (``hkv_pool_write``);
* ``unpack_to_staging(layer_idx, block_id_list, block_first_position,
  staging_k, staging_v)`` dequantises the kept blocks into the caller's
  (NK,BS,H,D) fp16 staging (``hkv_pool_gather``).

Each call is one kernel launch per tensor on torch's current stream, with no
host synchronisation.  Codes, masks and outlier values are bit-identical to
the reference's K10-K13 (fp32 compares, strict '<' ascending nearest pole).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from helix_kv import _native as N
from helix_kv.ops import NuqLayerTables

from .scales import KVScales


@dataclass
class CompactKVPool:
    """A paged KV cache holding nuq codes + dense outliers, per layer."""

    num_layers: int
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_size: int
    scales: KVScales
    device: str = "cuda:0"
    _k_levels: list[int] = field(default_factory=list)
    _v_levels: list[int] = field(default_factory=list)

    def __post_init__(self) -> None:
        L, NB, BS = self.num_layers, self.num_blocks, self.block_size
        H, D = self.num_kv_heads, self.head_size
        dev = torch.device(self.device)
        if dev.type != "cuda":
            raise AssertionError("CompactKVPool lives on the GPU")
        if len(self.scales.per_layer_keys) < L or len(self.scales.per_layer_values) < L:
            raise AssertionError("scales cover fewer layers than the pool")
        shape = (L, NB, BS, H, D)
        self.k_codes = torch.zeros(shape, dtype=torch.uint8, device=dev)
        self.v_codes = torch.zeros(shape, dtype=torch.uint8, device=dev)
        self.k_outv = torch.zeros(shape, dtype=torch.float16, device=dev)
        self.v_outv = torch.zeros(shape, dtype=torch.float16, device=dev)
        self.k_outm = torch.zeros(shape, dtype=torch.uint8, device=dev)
        self.v_outm = torch.zeros(shape, dtype=torch.uint8, device=dev)
        self.k_min = torch.full((L, NB, H, D), float("inf"), dtype=torch.float32, device=dev)
        self.k_max = torch.full((L, NB, H, D), float("-inf"), dtype=torch.float32, device=dev)
        self._k_levels = [int(s.poles.shape[-1]) for s in self.scales.per_layer_keys[:L]]
        self._v_levels = [int(s.poles.shape[-1]) for s in self.scales.per_layer_values[:L]]
        # device scales + nearest-pole decision tables, built once per layer
        self._kt: list[NuqLayerTables] = []
        self._vt: list[NuqLayerTables] = []
        for ks, vs in zip(self.scales.per_layer_keys[:L], self.scales.per_layer_values[:L]):
            if tuple(ks.poles.shape[:2]) != (H, D) or int(vs.poles.shape[0]) != H:
                raise AssertionError("scales do not match the pool's heads / head size")
            kt = NuqLayerTables(ks.poles.to(dev), ks.upper_threshold.to(dev),
                                ks.lower_threshold.to(dev), per_token=False)
            vt = NuqLayerTables(vs.poles.to(dev), vs.upper_threshold.to(dev),
                                vs.lower_threshold.to(dev), per_token=True)
            kt.ensure_tables()
            vt.ensure_tables()
            self._kt.append(kt)
            self._vt.append(vt)

    # -- write side --
    def write_kv(self, layer_idx: int, key: torch.Tensor, value: torch.Tensor,
                 slot_mapping: torch.Tensor, abs_positions: torch.Tensor) -> None:
        """Pack one layer's K/V (T,H,D) fp16 into the pool via slot_mapping."""
        assert layer_idx < self.num_layers
        assert key.is_contiguous(), "key must be contiguous (T, H, D)"
        assert value.is_contiguous()
        N.require_gpu(key, value, slot_mapping, abs_positions)
        H, D = self.num_kv_heads, self.head_size
        T = int(key.shape[0])
        if tuple(key.shape) != (T, H, D) or tuple(value.shape) != (T, H, D):
            raise AssertionError(f"key/value must be ({T}, {H}, {D})")
        assert key.dtype == torch.float16 and value.dtype == torch.float16, "K/V must be fp16"
        if T == 0:
            return
        slots = slot_mapping.to(torch.int64).contiguous()
        pos = abs_positions.to(torch.int64).contiguous()
        if slots.numel() != T or pos.numel() != T:
            raise AssertionError("slot_mapping / abs_positions must have one entry per token")
        L = layer_idx
        stream = N.stream_of(key)
        ks = self._kt[L].struct()
        st = N.lib().hkv_pool_write(
            N.ptr(key), T, H, D, ks, N.ptr(slots), self.num_blocks, self.block_size,
            N.ptr(self.k_codes[L]), N.ptr(self.k_outv[L]), N.ptr(self.k_outm[L]),
            N.ptr(self.k_min[L]), N.ptr(self.k_max[L]), stream)
        N.check(st, "hkv_pool_write (K)", AssertionError)
        vs = self._vt[L].struct(positions=pos)
        st = N.lib().hkv_pool_write(
            N.ptr(value), T, H, D, vs, N.ptr(slots), self.num_blocks, self.block_size,
            N.ptr(self.v_codes[L]), N.ptr(self.v_outv[L]), N.ptr(self.v_outm[L]),
            None, None, stream)
        N.check(st, "hkv_pool_write (V)", AssertionError)

    # -- read side --
    def unpack_to_staging(self, layer_idx: int, block_id_list: torch.Tensor,
                          block_first_position: torch.Tensor, staging_k: torch.Tensor,
                          staging_v: torch.Tensor) -> None:
        """Dequantise the selected blocks for one layer into ``staging_*``
        (NK,BS,H,D) fp16 (caller-owned)."""
        assert layer_idx < self.num_layers
        NK = int(block_id_list.shape[0])
        BS, H, D = self.block_size, self.num_kv_heads, self.head_size
        assert staging_k.shape == (NK, BS, H, D), \
            f"staging_k shape {staging_k.shape} != ({NK},{BS},{H},{D})"
        assert staging_v.shape == staging_k.shape
        assert staging_k.dtype == torch.float16 and staging_v.dtype == torch.float16
        assert staging_k.is_contiguous() and staging_v.is_contiguous()
        N.require_gpu(block_id_list, block_first_position, staging_k, staging_v)
        if NK == 0:
            return
        ids = block_id_list.to(torch.int64).contiguous()
        first = block_first_position.to(torch.int64).contiguous()
        assert first.numel() == NK, "one first position per kept block"
        L = layer_idx
        stream = N.stream_of(staging_k)
        st = N.lib().hkv_pool_gather(
            N.ptr(self.k_codes[L]), N.ptr(self.k_outv[L]), N.ptr(self.k_outm[L]),
            self.num_blocks, BS, H, D, self._kt[L].struct(with_tables=False), N.ptr(ids), None,
            NK, N.ptr(staging_k), stream)
        N.check(st, "hkv_pool_gather (K)", AssertionError)
        st = N.lib().hkv_pool_gather(
            N.ptr(self.v_codes[L]), N.ptr(self.v_outv[L]), N.ptr(self.v_outm[L]),
            self.num_blocks, BS, H, D, self._vt[L].struct(with_tables=False), N.ptr(ids),
            N.ptr(first), NK, N.ptr(staging_v), stream)
        N.check(st, "hkv_pool_gather (V)", AssertionError)
