"""Calibrated nuq parameters and their on-disk format.

Drop-in for src/kvquant/scales.py:13-140: the same three dataclasses with the
same fields, and the same ``torch.save`` dictionary (keys ``per_layer_keys``,
``per_layer_values`` -- lists of ``{poles, upper_threshold, lower_threshold,
num_bits}`` -- plus ``first_few_fp16`` and ``num_bits``), so files written by
either implementation load in the other.  Loading never unpickles code
(``weights_only=True``).

Per-layer level counts come from ``poles.shape[-1]`` (mixed nuq2/nuq4 files
splice layers, benchmarks/pr1c/mix_scales.py:59-68); ``num_bits`` on the
container is nominal.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


def _move(t: torch.Tensor, device) -> torch.Tensor:
    return t.to(device)


@dataclass
class PerChannelScale:
    """Key scales, per (KV head, channel): poles (H,D,L), thresholds (H,D)."""

    poles: torch.Tensor
    upper_threshold: torch.Tensor
    lower_threshold: torch.Tensor
    num_bits: int = 2

    def to(self, device: torch.device | str) -> "PerChannelScale":
        return PerChannelScale(_move(self.poles, device), _move(self.upper_threshold, device),
                               _move(self.lower_threshold, device), self.num_bits)


@dataclass
class PerTokenScale:
    """Value scales, per (KV head, calibrated position): poles (H,T_cal,L),
    thresholds (H,T_cal).  Positions >= T_cal use row T_cal-1."""

    poles: torch.Tensor
    upper_threshold: torch.Tensor
    lower_threshold: torch.Tensor
    num_bits: int = 2

    def to(self, device: torch.device | str) -> "PerTokenScale":
        return PerTokenScale(_move(self.poles, device), _move(self.upper_threshold, device),
                             _move(self.lower_threshold, device), self.num_bits)


def _as_dict(s) -> dict:
    return {"poles": s.poles, "upper_threshold": s.upper_threshold,
            "lower_threshold": s.lower_threshold, "num_bits": s.num_bits}


@dataclass
class KVScales:
    """Scales for every layer; ``first_few_fp16`` is the attention-sink count
    kept in fp16 by the reference's CPU spec (its GPU kernels ignore it)."""

    per_layer_keys: list[PerChannelScale] = field(default_factory=list)
    per_layer_values: list[PerTokenScale] = field(default_factory=list)
    first_few_fp16: int = 4
    num_bits: int = 2

    def __post_init__(self) -> None:
        if self.per_layer_keys and self.per_layer_values:
            assert len(self.per_layer_keys) == len(self.per_layer_values), (
                "key and value scales must cover the same number of layers")

    @property
    def num_layers(self) -> int:
        return len(self.per_layer_keys)

    def levels(self, layer: int) -> tuple[int, int]:
        """(K levels, V levels) of one layer."""
        return (int(self.per_layer_keys[layer].poles.shape[-1]),
                int(self.per_layer_values[layer].poles.shape[-1]))

    def to(self, device: torch.device | str) -> "KVScales":
        return KVScales([s.to(device) for s in self.per_layer_keys],
                        [s.to(device) for s in self.per_layer_values],
                        self.first_few_fp16, self.num_bits)

    def save(self, path: str) -> None:
        torch.save({
            "per_layer_keys": [_as_dict(s) for s in self.per_layer_keys],
            "per_layer_values": [_as_dict(s) for s in self.per_layer_values],
            "first_few_fp16": self.first_few_fp16,
            "num_bits": self.num_bits,
        }, path)

    @classmethod
    def load(cls, path: str, map_location: str | torch.device = "cpu") -> "KVScales":
        d = torch.load(path, map_location=map_location, weights_only=True)
        return cls([PerChannelScale(**s) for s in d["per_layer_keys"]],
                   [PerTokenScale(**s) for s in d["per_layer_values"]],
                   d["first_few_fp16"], d["num_bits"])

    @classmethod
    def splice(cls, shallow: "KVScales", deep: "KVScales", cut: int) -> "KVScales":
        """Layers [0, cut) from ``shallow``, [cut, L) from ``deep``
        (benchmarks/pr1c/mix_scales.py:59-70)."""
        assert shallow.num_layers == deep.num_layers, "layer count mismatch"
        assert 0 < cut < shallow.num_layers, f"cut must be in (0, {shallow.num_layers})"
        return cls(shallow.per_layer_keys[:cut] + deep.per_layer_keys[cut:],
                   shallow.per_layer_values[:cut] + deep.per_layer_values[cut:],
                   shallow.first_few_fp16, shallow.num_bits)
