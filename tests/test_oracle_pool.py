"""Pins of the pool oracle (oracle.pool_write / pool_gather / select_union).

The pool functions compose the already-pinned pack/unpack with a slot scatter
and per-block statistics; these tests pin what the composition adds:

* block statistics characterised independently of ordered_min_max: every
  statistic is attained by a reconstructed value of the block and bounds all
  of them (np.min / np.max by value), plus the -0 / +0 order on planted zeros;
* skipped slots (< 0, past the pool), the V scale-row clamp at T_cal - 1 via the
  scalar nearest_code, decode-style appends that merge with existing stats;
* the reference selector's known answers (src/kvquant/tests/
  test_quest_selector.py:41-95: the planted block wins, sinks are kept).
"""
from __future__ import annotations

import numpy as np

import oracle as O

RNG = np.random.default_rng(1234)


def _empty_pool(NB, BS, H, D):
    z = lambda dt: np.zeros((NB, BS, H, D), dt)  # noqa: E731
    return {"k_codes": z(np.uint8), "k_outv": z(np.uint16), "k_outm": z(np.uint8),
            "v_codes": z(np.uint8), "v_outv": z(np.uint16), "v_outm": z(np.uint8),
            "k_min": np.full((NB, H, D), np.inf, np.float32),
            "k_max": np.full((NB, H, D), -np.inf, np.float32)}


def _scales(H, D, Tcal, LK=16, LV=4, thr=1.5):
    kp = np.sort(RNG.standard_normal((H, D, LK)), -1).astype(np.float16).astype(np.float32)
    vp = np.sort(RNG.standard_normal((H, Tcal, LV)), -1).astype(np.float16).astype(np.float32)
    ku = np.full((H, D), thr, np.float32)
    vu = np.full((H, Tcal), thr, np.float32)
    return (kp, ku, -ku), (vp, vu, -vu)


def test_stats_attained_and_bounding():
    NB, BS, H, D, Tcal = 6, 4, 2, 16, 32
    ks, vs = _scales(H, D, Tcal)
    pool = _empty_pool(NB, BS, H, D)
    T = 20
    key = RNG.standard_t(3, (T, H, D)).astype(np.float16)
    slots = RNG.permutation(NB * BS)[:T]
    O.pool_write(pool, key, key, slots, np.arange(T), ks, vs, BS)
    for b in range(NB):
        mine = [t for t in range(T) if slots[t] // BS == b]
        if not mine:
            assert np.all(np.isinf(pool["k_min"][b])) and np.all(pool["k_min"][b] > 0)
            continue
        rec = []
        for t in mine:
            for h in range(H):
                for d in range(D):
                    x = np.float32(key[t, h, d])
                    if x > ks[1][h, d] or x < ks[2][h, d]:
                        rec.append((h, d, x))
                    else:
                        rec.append((h, d, ks[0][h, d, O.nearest_code(x, ks[0][h, d])]))
        vals = np.zeros((len(mine), H, D), np.float32)
        cnt = np.zeros((H, D), int)
        for h, d, x in rec:
            vals[cnt[h, d], h, d] = x
            cnt[h, d] += 1
        assert np.array_equal(pool["k_min"][b], vals.min(0))
        assert np.array_equal(pool["k_max"][b], vals.max(0))


def test_signed_zero_order_in_stats():
    NB, BS, H, D, Tcal = 2, 2, 1, 8, 4
    ks, vs = _scales(H, D, Tcal)
    ks = (np.zeros((H, D, 16), np.float32), np.full((H, D), 0.5, np.float32),
          np.full((H, D), -0.5, np.float32))  # every pole 0: non-outliers reconstruct to +0
    pool = _empty_pool(NB, BS, H, D)
    key = np.zeros((2, H, D), np.float16)
    key[0] = -0.0  # not an outlier -> pole +0
    key[1, 0, :] = np.float16(-0.0)
    O.pool_write(pool, key, key, [0, 1], [0, 1], ks, vs, BS)
    assert np.all(pool["k_min"][0] == 0) and np.all(~np.signbit(pool["k_max"][0]))
    # now an outlier -0 cannot exist (|-0| is inside the band); plant -0 poles
    ks2 = (np.full((H, D, 16), -0.0, np.float32), ks[1], ks[2])
    pool2 = _empty_pool(NB, BS, H, D)
    O.pool_write(pool2, key[:1], key[:1], [0], [0], ks2, vs, BS)
    O.pool_write(pool2, key[:1], key[:1], [1], [1], ks, vs, BS)
    assert np.all(np.signbit(pool2["k_min"][0])) and not np.any(np.signbit(pool2["k_max"][0]))


def test_skipped_slots_and_v_clamp():
    NB, BS, H, D, Tcal = 3, 4, 2, 16, 8
    ks, vs = _scales(H, D, Tcal)
    pool = _empty_pool(NB, BS, H, D)
    T = 6
    val = RNG.standard_normal((T, H, D)).astype(np.float16)
    slots = np.array([0, -1, 5, NB * BS, 11, -7])
    pos = np.array([0, 1, 100, 3, 9, 2])  # 100 and 9 clamp to row Tcal-1
    O.pool_write(pool, val, val, slots, pos, ks, vs, BS)
    written = {0: 0, 5: 2, 11: 4}
    for s in range(NB * BS):
        b, o = divmod(s, BS)
        if s not in written:
            assert not pool["v_codes"][b, o].any() and not pool["v_outm"][b, o].any()
            continue
        t = written[s]
        row = min(pos[t], Tcal - 1)
        for h in range(H):
            for d in range(D):
                x = np.float32(val[t, h, d])
                outl = x > vs[1][h, row] or x < vs[2][h, row]
                assert pool["v_outm"][b, o, h, d] == outl
                assert pool["v_codes"][b, o, h, d] == O.nearest_code(x, vs[0][h, row])
    # gather: a kept block's V rows use min(first_pos + p, Tcal - 1)
    sk, sv = O.pool_gather(pool, [2, 1], [2 * BS, 100], ks, vs)
    p, h, d = 3, 1, 5
    c = pool["v_codes"][2, p, h, d]
    want = np.float16(vs[0][h, min(2 * BS + p, Tcal - 1), c]).view(np.uint16)
    if pool["v_outm"][2, p, h, d]:
        want = pool["v_outv"][2, p, h, d]
    assert sv[0, p, h, d] == want


def test_append_merges_with_existing_stats():
    NB, BS, H, D, Tcal = 2, 8, 2, 8, 16
    ks, vs = _scales(H, D, Tcal, thr=0.8)
    key = RNG.standard_t(3, (8, H, D)).astype(np.float16)
    once = _empty_pool(NB, BS, H, D)
    O.pool_write(once, key, key, np.arange(8), np.arange(8), ks, vs, BS)
    step = _empty_pool(NB, BS, H, D)
    for t in range(8):  # decode: one token at a time into block 0
        O.pool_write(step, key[t:t + 1], key[t:t + 1], [t], [t], ks, vs, BS)
    for name in once:
        assert np.array_equal(once[name], step[name]), name


def test_reference_selector_known_answers():
    """src/kvquant/tests/test_quest_selector.py:41-95 on the oracle pool."""
    H, D, BS, NB, Tcal = 2, 8, 4, 6, 32
    poles = np.broadcast_to(np.linspace(-1.5, 1.5, 16, dtype=np.float16).astype(np.float32),
                            (H, D, 16)).copy()
    vpoles = np.broadcast_to(np.linspace(-1.5, 1.5, 4, dtype=np.float16).astype(np.float32),
                             (H, Tcal, 4)).copy()
    ks = (poles, np.full((H, D), 2.0, np.float32), np.full((H, D), -2.0, np.float32))
    vs = (vpoles, np.full((H, Tcal), 2.0, np.float32), np.full((H, Tcal), -2.0, np.float32))
    pool = _empty_pool(NB, BS, H, D)
    T = 5 * BS
    key = np.zeros((T, H, D), np.float16)
    key[3 * BS:4 * BS] = 1.0
    O.pool_write(pool, key, np.zeros_like(key), np.arange(T), np.arange(T), ks, vs, BS)
    used = np.arange(5)
    q = np.ones((H, D), np.float32)
    bound = O.page_bound(q, pool["k_min"][used], pool["k_max"][used])
    ids, first = O.select_union(bound, used, top_k=1, sink_blocks=0, block_size=BS)
    assert ids.tolist() == [3] and first.tolist() == [3 * BS]
    pool0 = _empty_pool(NB, BS, H, D)
    O.pool_write(pool0, np.zeros_like(key), np.zeros_like(key), np.arange(T), np.arange(T),
                 ks, vs, BS)
    bound0 = O.page_bound(q, pool0["k_min"][used], pool0["k_max"][used])
    ids0, _ = O.select_union(bound0, used, top_k=1, sink_blocks=2, block_size=BS)
    assert 0 in ids0.tolist() and 1 in ids0.tolist()
