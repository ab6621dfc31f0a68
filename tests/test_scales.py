"""The scales container and its .pt format (src/kvquant/scales.py:13-140;
mixed nuq2/nuq4 files by splicing, benchmarks/pr1c/mix_scales.py:59-70), on
the CPU: save / load keeps every tensor bit for bit (loaded without
unpickling code), splice takes layers [0, cut) from one file and the rest
from the other, and the level count of each layer comes from its poles."""
from __future__ import annotations

import pytest
import torch

from kvquant.scales import KVScales, PerChannelScale, PerTokenScale


def _scales(L, levels, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    H, D, Tc = 2, 8, 16
    keys = [PerChannelScale(torch.randn(H, D, levels, generator=g).sort(-1).values.to(dtype),
                            torch.rand(H, D, generator=g).to(dtype),
                            -torch.rand(H, D, generator=g).to(dtype), 2 if levels <= 4 else 4)
            for _ in range(L)]
    vals = [PerTokenScale(torch.randn(H, Tc, levels, generator=g).sort(-1).values.to(dtype),
                          torch.rand(H, Tc, generator=g).to(dtype),
                          -torch.rand(H, Tc, generator=g).to(dtype), 2 if levels <= 4 else 4)
            for _ in range(L)]
    return KVScales(keys, vals, first_few_fp16=4, num_bits=2 if levels <= 4 else 4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_save_load_round_trip(tmp_path, dtype):
    s = _scales(3, 16, dtype, 0)
    p = tmp_path / "scales.pt"
    s.save(str(p))
    r = KVScales.load(str(p))
    assert r.num_layers == 3 and r.first_few_fp16 == 4 and r.num_bits == 4
    for a, b in zip(s.per_layer_keys + s.per_layer_values, r.per_layer_keys + r.per_layer_values):
        for x, y in ((a.poles, b.poles), (a.upper_threshold, b.upper_threshold),
                     (a.lower_threshold, b.lower_threshold)):
            assert x.dtype == y.dtype and torch.equal(x, y)
        assert a.num_bits == b.num_bits


def test_splice_mixed_levels(tmp_path):
    shallow, deep = _scales(4, 4, torch.float32, 1), _scales(4, 16, torch.float32, 2)
    m = KVScales.splice(shallow, deep, 2)
    assert [m.levels(i) for i in range(4)] == [(4, 4), (4, 4), (16, 16), (16, 16)]
    assert torch.equal(m.per_layer_keys[1].poles, shallow.per_layer_keys[1].poles)
    assert torch.equal(m.per_layer_values[3].poles, deep.per_layer_values[3].poles)
    p = tmp_path / "mixed.pt"
    m.save(str(p))
    assert [KVScales.load(str(p)).levels(i) for i in range(4)] == [(4, 4), (4, 4), (16, 16), (16, 16)]
    with pytest.raises(AssertionError):
        KVScales.splice(shallow, deep, 0)
