"""The GPU path reproduces the frozen vectors of tests/golden/: bit-exact for
codes, packed bytes, CSR, page stats, bound scores and selections; within
1e-3 relative (per head, L2 and max-abs) for the decode attention."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

G = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(G / f"{name}.npz")


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _compact(dev, z):
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact

    x = _t(z["x"], dev)
    ku = _t(z["k_upper"], dev)
    vu = _t(z["v_upper"], dev)
    kt = NuqLayerTables(_t(z["k_poles"], dev), ku, -ku, per_token=False)
    vt = NuqLayerTables(_t(z["v_poles"], dev), vu, -vu, per_token=True)
    return nuq_pack_compact(x, kt, 4), kt, nuq_pack_compact(x, vt, 2), vt


def test_golden_nuq_on_gpu(dev):
    from kvquant.triton_batched import pack_keys_per_channel_batched

    z = _load("nuq")
    ku = _t(z["k_upper"], dev)
    c, v, m = pack_keys_per_channel_batched(_t(z["x"], dev), _t(z["k_poles"], dev), ku, -ku)
    assert np.array_equal(c.cpu().numpy(), z["k_codes"])
    assert np.array_equal(v.cpu().view(torch.int16).numpy().view(np.uint16), z["k_outv"])
    assert np.array_equal(m.cpu().numpy(), z["k_outm"])
    ck, _, cv, _ = _compact(dev, z)
    for cc, p in ((ck, "k"), (cv, "v")):
        assert np.array_equal(cc.packed.cpu().numpy(), z[f"{p}_packed"])
        assert np.array_equal(cc.row_ptr.cpu().numpy(), z[f"{p}_row_ptr"])
        assert np.array_equal(cc.col.cpu().numpy(), z[f"{p}_col"])
        assert np.array_equal(cc.val.cpu().view(torch.int16).numpy().view(np.uint16), z[f"{p}_val"])


def test_golden_quest_on_gpu(dev):
    from helix_kv.ops import quest_page_stats, quest_select

    z = _load("quest")
    mn, mx = quest_page_stats(_t(z["K"], dev))
    assert np.array_equal(mn.cpu().numpy(), z["k_min"]) and np.array_equal(mx.cpu().numpy(), z["k_max"])
    sel, scores = quest_select(_t(z["q"], dev), mn, mx, int(z["k"]), int(z["sinks"]))
    assert np.array_equal(scores.cpu().numpy().T, z["bound"])
    assert np.array_equal(sel.cpu().numpy(), z["sel"])


def test_golden_decode_on_gpu(dev):
    from helix_kv.ops import decode_attention

    z, n = _load("decode"), _load("nuq")
    ck, kt, cv, vt = _compact(dev, n)
    out = decode_attention(_t(z["q"], dev), ck, kt, cv, vt, _t(z["sel"], dev),
                           out_dtype=torch.float32).double().cpu().numpy()
    want = z["out"]
    for h in range(want.shape[0]):
        err = out[h] - want[h]
        assert np.linalg.norm(err) <= 1e-3 * np.linalg.norm(want[h])
        assert np.abs(err).max() <= 1e-3 * np.abs(want[h]).max()
