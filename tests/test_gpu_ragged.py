"""GPU parity of the ragged batched Quest selection and the per-head
gather + dequant of selected compact pages, against the oracle (bit-exact)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(404)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("lens,H,group,D,ks,sinks", [
    ([6, 0, 9, 300, 1], 2, 7, 128, [1, 3, 2, 75, 5], 4),
    ([2048, 5000, 777], 4, 7, 128, [512, 1250, 194], 4),
    ([100, 17000], 4, 1, 64, [25, 4250], 2),
    ([1], 1, 1, 8, [0], 0),
])
def test_select_ragged_vs_oracle(dev, lens, H, group, D, ks, sinks):
    from helix_kv.ops import quest_select_ragged

    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    Ptot = int(offs[-1])
    mn = RNG.standard_normal((Ptot, H, D)).astype(np.float16)
    mx = (mn.astype(np.float32) + np.abs(RNG.standard_normal((Ptot, H, D)))).astype(np.float16)
    mx = np.maximum(mx, mn)
    q = RNG.standard_normal((len(lens), H * group, D)).astype(np.float16)
    sel, outs, scores = quest_select_ragged(_t(q, dev), _t(mn, dev), _t(mx, dev), offs, ks, sinks)
    wsel, wouts, wscores = O.select_ragged(q.astype(np.float32), mn.astype(np.float32),
                                           mx.astype(np.float32), offs, ks, sinks)
    assert outs == wouts.tolist()
    assert np.array_equal(scores.cpu().numpy(), wscores)
    assert np.array_equal(sel.cpu().numpy(), wsel)


@pytest.mark.parametrize("bits,L,thr", [(4, 16, 1.5), (2, 4, 1.2), (4, 16, np.inf),
                                        (2, 4, 0.3)])  # ~80 outliers per row: most slots heavy
def test_gather_pages_vs_oracle(dev, bits, L, thr):
    from helix_kv.ops import NuqLayerTables, nuq_gather_pages, nuq_pack_compact

    lens = [5, 12, 1, 9]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, H, D, rows_cal = int(offs[-1]) * 16, 4, 128, 100
    x = (RNG.standard_t(3, (T, H, D)) * 0.6).astype(np.float16)
    pos = np.concatenate([np.arange(n * 16) for n in lens]).astype(np.int64)  # position in sequence
    kp = np.sort(RNG.standard_normal((H, D, L)), -1).astype(np.float16)
    vp = np.sort(RNG.standard_normal((H, rows_cal, L)), -1).astype(np.float16)
    ku = np.full((H, D), thr, np.float16)
    vu = np.full((H, rows_cal), thr, np.float16)
    kt = NuqLayerTables(_t(kp, dev), _t(ku, dev), -_t(ku, dev), per_token=False)
    vt = NuqLayerTables(_t(vp, dev), _t(vu, dev), -_t(vu, dev), per_token=True)
    ck = nuq_pack_compact(_t(x, dev), kt, bits)
    cv = nuq_pack_compact(_t(x, dev), vt, bits, positions=_t(pos, dev))
    # a selection with repeated, out-of-range and negative page ids
    outs = [0, 3, 9, 10, 14]
    sel = np.stack([RNG.integers(-1, 14, size=14) for _ in range(H)], 1).astype(np.int64)
    f = lambda a: a.astype(np.float32)  # noqa: E731
    kd = O.unpack(*O.pack_k(x, f(kp), f(ku), -f(ku)), f(kp), "k")
    vd = O.unpack(*O.pack_v(x, f(vp), f(vu), -f(vu), positions=pos), f(vp), "v", positions=pos)
    for cc, tabs, deq in ((ck, kt, kd), (cv, vt, vd)):
        got = nuq_gather_pages(cc, tabs, _t(sel, dev), offs, outs)
        want = O.gather_pages(deq, sel, offs, outs)
        assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), want)


def test_ragged_end_to_end_select_then_gather(dev):
    """Selection feeds the gather directly: every gathered (row, head) page is
    the selected page of that head in that sequence."""
    from helix_kv.ops import (NuqLayerTables, nuq_gather_pages, nuq_pack_compact,
                              quest_page_stats, quest_select_ragged)

    lens = [40, 7, 64]
    offs = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T, H, D = int(offs[-1]) * 16, 4, 128
    x = RNG.standard_normal((T, H, D)).astype(np.float16)
    kp = np.sort(RNG.standard_normal((H, D, 16)), -1).astype(np.float16)
    ku = np.full((H, D), np.inf, np.float16)
    kt = NuqLayerTables(_t(kp, dev), _t(ku, dev), -_t(ku, dev), per_token=False)
    ck = nuq_pack_compact(_t(x, dev), kt, 4)
    mn, mx = quest_page_stats(_t(x, dev).view(-1, 16, H, D))
    q = _t(RNG.standard_normal((3, H * 7, D)).astype(np.float16), dev)
    sel, outs, _ = quest_select_ragged(q, mn, mx, offs, [10, 2, 16], 4)
    st = nuq_gather_pages(ck, kt, sel, offs, outs)
    full = O.unpack(O.bitunpack(ck.packed.cpu().numpy(), 4, D), np.zeros((T, H, D), np.uint16),
                    np.zeros((T, H, D), np.uint8), kp.astype(np.float32), "k")
    want = O.gather_pages(full, sel.cpu().numpy(), offs, outs)
    assert np.array_equal(st.cpu().view(torch.int16).numpy().view(np.uint16), want)
    assert outs == [0, 14, 20, 40]
