"""Pins of the CPU oracle's Quest functions (no GPU).

Checked against the reference's known-answer tests (src/quest/tests/
test_reference.py, src/kvquant/tests/test_quest_selector.py), numpy/torch
reductions, torch.topk on distinct keys, and closed forms.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

RNG = np.random.default_rng(7)


def test_page_stats_match_numpy_and_spot_check():
    # src/quest/tests/test_reference.py:34-42
    K = RNG.standard_normal((4, 16, 2, 8)).astype(np.float32)
    mn, mx = O.page_stats(K)
    assert np.array_equal(mn, K.min(axis=1)) and np.array_equal(mx, K.max(axis=1))
    assert mn[1, 0, 3] == K[1, :, 0, 3].min() and mx[1, 0, 3] == K[1, :, 0, 3].max()
    Kh = K.astype(np.float16)
    mn16, mx16 = O.page_stats(Kh)
    assert mn16.dtype == np.float16
    assert np.array_equal(mn16, Kh.min(axis=1)) and np.array_equal(mx16, Kh.max(axis=1))


def test_page_stats_signed_zero_and_nan_rules():
    K = np.zeros((2, 4, 1, 2), np.float32)
    K[0, :, 0, 0] = [0.0, -0.0, 0.0, 1.0]
    K[0, :, 0, 1] = [-0.0, 0.0, -1.0, -0.0]
    K[1, 2, 0, 0] = np.nan
    mn, mx = O.page_stats(K)
    assert np.signbit(mn[0, 0, 0]) and mn[0, 0, 0] == 0.0 and mx[0, 0, 0] == 1.0
    assert mn[0, 0, 1] == -1.0 and not np.signbit(mx[0, 0, 1]) and mx[0, 0, 1] == 0.0
    assert np.isnan(mn[1, 0, 0]) and np.isnan(mx[1, 0, 0]) and mn[1, 0, 1] == 0.0


def test_bound_is_an_upper_bound():
    # src/quest/tests/test_reference.py:45-63
    P, page, H, D = 8, 16, 4, 32
    K = RNG.standard_normal((P, page, H, D)).astype(np.float32)
    q = RNG.standard_normal((H, D)).astype(np.float32)
    mn, mx = O.page_stats(K)
    bound = O.page_bound(q, mn, mx)
    true_max = np.einsum("pthd,hd->pth", K, q).max(axis=1)
    assert (bound - true_max >= -1e-4).all()


def test_bound_matches_torch_formula():
    """Same value as the reference's torch expression up to summation order."""
    P, H, D = 64, 4, 128
    q = torch.randn(H, D)
    kmin = torch.randn(P, H, D)
    kmax = kmin + torch.rand(P, H, D)
    ref = (q.clamp(min=0) * kmax).sum(-1) + (q.clamp(max=0) * kmin).sum(-1)  # reference.py:88-92
    got = O.page_bound(q.numpy(), kmin.numpy(), kmax.numpy())
    mag = (q.abs().unsqueeze(0) * torch.maximum(kmin.abs(), kmax.abs())).sum(-1)
    assert np.all(np.abs(got - ref.numpy()) <= 4 * np.finfo(np.float32).eps * mag.numpy())


def test_bound_exact_for_one_hot_query():
    P, H, D = 16, 2, 40
    mn = RNG.standard_normal((P, H, D)).astype(np.float16).astype(np.float32)
    mx = mn + RNG.random((P, H, D)).astype(np.float16).astype(np.float32)
    for d, c in [(0, 2.5), (17, -3.0), (39, 0.125)]:
        q = np.zeros((H, D), np.float32)
        q[:, d] = c
        want = c * (mx[:, :, d] if c > 0 else mn[:, :, d])
        assert np.array_equal(O.page_bound(q, mn, mx), want.astype(np.float32))


def test_group_bound_is_sum_of_head_bounds():
    P, Hkv, g, D = 32, 4, 7, 128
    q = RNG.standard_normal((Hkv * g, D)).astype(np.float16).astype(np.float32)
    mn = RNG.standard_normal((P, Hkv, D)).astype(np.float16).astype(np.float32)
    mx = mn + RNG.random((P, Hkv, D)).astype(np.float16).astype(np.float32)
    got = O.page_bound_group(q, mn, mx, g).astype(np.float64)
    per_head = np.stack([O.page_bound(q[h:h + 1], mn[:, h // g:h // g + 1],
                                      mx[:, h // g:h // g + 1])[:, 0] for h in range(Hkv * g)], 1)
    want = per_head.astype(np.float64).reshape(P, Hkv, g).sum(-1)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-4)
    assert np.array_equal(O.page_bound_group(q[:Hkv], mn, mx, 1), O.page_bound(q[:Hkv], mn, mx))


def test_topk_known_answers():
    # src/quest/tests/test_reference.py:66-92
    bound = RNG.standard_normal((16, 4)).astype(np.float32)
    bound[0, :] = -100.0
    sel = O.topk_sinks(bound, 4, 2)
    assert sel.shape == (6, 4)
    for h in range(4):
        assert {0, 1} <= set(sel[:, h].tolist())
        assert np.all(np.diff(sel[:, h]) > 0)
    assert O.topk_sinks(RNG.standard_normal((3, 2)).astype(np.float32), 10, 1).shape == (3, 2)


@pytest.mark.parametrize("P,k,s", [(1000, 250, 4), (257, 1, 0), (64, 60, 4), (5, 0, 2), (3, 1, 7)])
def test_topk_equals_torch_topk_on_distinct_keys(P, k, s):
    H = 3
    b = torch.randperm(P * H).float().reshape(P, H) * 0.25 - 100.0
    sel = O.topk_sinks(b.numpy(), k, s)
    sp = max(0, min(s, P))
    keff = max(0, min(k, P - sp))
    masked = b.clone()
    masked[:sp] = float("-inf")
    top = torch.topk(masked, keff, dim=0).indices if keff else torch.empty(0, H, dtype=torch.long)
    want = torch.cat([torch.arange(sp).unsqueeze(1).expand(-1, H), top], 0).sort(0).values
    assert np.array_equal(sel, want.numpy())


def test_topk_ties_go_to_lower_pages_and_nan_ranks_highest():
    b = np.zeros((20, 2), np.float32)
    sel = O.topk_sinks(b, 5, 2)
    assert sel[:, 0].tolist() == [0, 1, 2, 3, 4, 5, 6]
    b[15, 1] = np.nan
    b[9, 1] = 1.0
    b[3, 1] = -0.0
    sel = O.topk_sinks(b, 3, 0)
    assert sel[:, 1].tolist() == [0, 9, 15]


def _pool_stats(key, poles, up, lo, BS):
    """Reconstructed-K page stats as the reference pool keeps them (compact_pool.py:258-287)."""
    c, v, m = O.pack_k(key, poles, up, lo)
    rec = O.h2f(O.unpack(c, v, m, poles, "k"))
    T, H, D = rec.shape
    return O.page_stats(rec.reshape(T // BS, BS, H, D))


def test_select_union_known_answers():
    # src/kvquant/tests/test_quest_selector.py:41-95
    H, D, BS = 2, 8, 4
    poles = np.broadcast_to(np.linspace(-1.5, 1.5, 16, dtype=np.float16).astype(np.float32),
                            (H, D, 16)).copy()
    up, lo = np.full((H, D), 2.0), np.full((H, D), -2.0)
    key = np.zeros((5 * BS, H, D), np.float16)
    key[3 * BS:4 * BS] = 1.0
    mn, mx = _pool_stats(key, poles, up, lo, BS)
    q = np.ones((H, D), np.float32)
    ids, first = O.select_union(O.page_bound(q, mn, mx), np.arange(5), 1, 0, BS)
    assert ids.tolist() == [3] and first.tolist() == [12]
    key0 = np.zeros((5 * BS, H, D), np.float16)
    mn, mx = _pool_stats(key0, poles, up, lo, BS)
    ids, _ = O.select_union(O.page_bound(q, mn, mx), np.arange(5), 1, 2, BS)
    assert {0, 1} <= set(ids.tolist())


def test_attention_all_pages_equals_dense():
    # src/quest/tests/test_reference.py:95-117 (float64 oracle vs torch fp32 dense)
    P, page, H, D = 4, 8, 2, 16
    K = RNG.standard_normal((P, page, H, D))
    V = RNG.standard_normal((P, page, H, D))
    q = RNG.standard_normal((H, D))
    out = O.selected_attention(q, K, V, np.arange(P)[:, None].repeat(H, 1), lambda h: h)
    Kf, Vf = torch.tensor(K).reshape(P * page, H, D), torch.tensor(V).reshape(P * page, H, D)
    for h in range(H):
        a = torch.softmax(Kf[:, h] @ torch.tensor(q[h]) / np.sqrt(D), 0)
        assert np.allclose(out[h], (a @ Vf[:, h]).numpy(), atol=1e-9)


def test_attention_gqa_mask_matches_sdpa():
    """GQA (query head h -> KV head h // group), partial last page and page
    subsets against torch's own scaled_dot_product_attention in float64 over
    the gathered keys (a library routine, independent of the oracle's loop)."""
    P, S, H, group, D = 6, 16, 2, 7, 32
    T = 5 * S + 3  # last valid page holds 3 tokens, page 5 none
    K = RNG.standard_normal((P, S, H, D))
    V = RNG.standard_normal((P, S, H, D))
    q = RNG.standard_normal((H * group, D))
    sel = np.array([[0, 1], [4, 2], [5, 4], [2, 0]])  # page 5 is past T: masked
    out = O.selected_attention(q, K, V, sel, lambda h: h // group, num_tokens=T, scale=0.3)
    for hq in range(H * group):
        g = hq // group
        toks = [p * S + s for p in sel[:, g] for s in range(S) if p * S + s < T]
        Kg = torch.tensor(K.reshape(P * S, H, D)[toks, g])
        Vg = torch.tensor(V.reshape(P * S, H, D)[toks, g])
        want = torch.nn.functional.scaled_dot_product_attention(
            torch.tensor(q[hq])[None, None, None], Kg[None, None], Vg[None, None], scale=0.3)
        assert np.allclose(out[hq], want.reshape(-1).numpy(), rtol=1e-12, atol=1e-12)


def test_attention_exclusion_and_invalid_ids():
    # src/quest/tests/test_reference.py:120-139: an unselected page cannot move
    # the output, however large its keys; ids outside [0, P) select nothing.
    P, S, H, D = 5, 4, 1, 8
    K = RNG.standard_normal((P, S, H, D))
    V = RNG.standard_normal((P, S, H, D))
    q = RNG.standard_normal((H, D))
    sel = np.array([[0], [2], [4]])
    a = O.selected_attention(q, K, V, sel, lambda h: 0)
    K2, V2 = K.copy(), V.copy()
    K2[1], V2[1], K2[3] = 1e3 * q[0], 1e3, -1e3 * q[0]
    assert np.array_equal(a, O.selected_attention(q, K2, V2, sel, lambda h: 0))
    b = O.selected_attention(q, K, V, np.array([[0], [-1], [2], [P], [4], [99]]), lambda h: 0)
    assert np.array_equal(a, b)
    # a selection with no valid token leaves the head at zero
    assert not O.selected_attention(q, K, V, np.array([[3]]), lambda h: 0, num_tokens=12).any()


def test_select_ragged_known_answers():
    """Each sequence of a ragged batch selects from its own pages only, with
    local indices: a page planted with large keys in each sequence is chosen
    there and nowhere else; sinks are each sequence's first pages; an empty
    sequence contributes no rows."""
    H, D, group = 2, 16, 3
    lens = [6, 0, 9, 4]
    offs = np.concatenate([[0], np.cumsum(lens)])
    Ptot = offs[-1]
    mn = np.zeros((Ptot, H, D), np.float32)
    mx = np.zeros((Ptot, H, D), np.float32)
    planted = [4, None, 7, 2]
    for b, p in enumerate(planted):
        if p is not None:
            mx[offs[b] + p] = 5.0
            mn[offs[b] + p] = 4.0
    q = np.ones((len(lens), H * group, D), np.float32)
    sel, outs, scores = O.select_ragged(q, mn, mx, offs, [1, 1, 1, 1], 2)
    assert outs.tolist() == [0, 3, 3, 6, 9]
    assert sel[0:3, 0].tolist() == [0, 1, 4] and sel[3:6, 1].tolist() == [0, 1, 7]
    assert sel[6:9, 0].tolist() == [0, 1, 2]
    assert scores.shape == (H, Ptot) and scores[0, offs[2] + 7] == 5.0 * D * group


def test_select_ragged_single_sequence_is_plain_select():
    P, H, D, group = 300, 4, 32, 7
    mn = RNG.standard_normal((P, H, D)).astype(np.float16).astype(np.float32)
    mx = mn + np.abs(RNG.standard_normal((P, H, D))).astype(np.float16).astype(np.float32)
    q = RNG.standard_normal((1, H * group, D)).astype(np.float32)
    sel, outs, scores = O.select_ragged(q, mn, mx, [0, P], [70], 4)
    b = O.page_bound_group(q[0], mn, mx, group)
    assert np.array_equal(scores, b.T) and np.array_equal(sel, O.topk_sinks(b, 70, 4))


def test_gather_pages_known_answer():
    """Tokens carry their own index, so the gathered staging spells out which
    token of which head landed where; ids outside a sequence give zeros."""
    H, D, S = 2, 8, 16
    lens = [3, 2]
    offs = [0, 3, 5]
    T = 5 * S
    deq = np.zeros((T, H, D), np.uint16)
    for t in range(T):
        for h in range(H):
            deq[t, h] = t * 10 + h
    sel = np.array([[0, 2], [2, -1], [1, 0], [5, 1]], np.int64)  # seq 0: rows 0-1, seq 1: rows 2-3
    st = O.gather_pages(deq, sel, offs, [0, 2, 4], S)
    assert st[0, 3, 1, 0] == (2 * S + 3) * 10 + 1          # seq 0, page 2, slot 3, head 1
    assert not st[1, :, 1].any()                            # id -1
    assert st[2, 0, 0, 0] == ((3 + 1) * S) * 10             # seq 1 page 1 = global page 4
    assert not st[3, :, 0].any() and st[3, 5, 1, 0] == ((3 + 1) * S + 5) * 10 + 1


def _all_finite_f16(lo=-np.inf, hi=np.inf):
    v = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = v[np.isfinite(v)]
    return v[(v >= lo) & (v <= hi)]


@pytest.mark.parametrize("lo,hi", [(-np.inf, np.inf), (-4.0, 4.0), (0.5, 0.75), (-1e-3, 2e-3),
                                   (1000.0, 1024.0)])
def test_page_stats_u8_brackets_every_fp16_value(lo, hi):
    """Every finite fp16 statistic in a channel's range: deq(qmin) <= v <= deq(qmax)."""
    v = _all_finite_f16(lo, hi)
    P = v.shape[0]
    mn = v.reshape(P, 1, 1)
    qmin, qmax, l, st = O.page_stats_u8(mn, mn)
    dmn, dmx = O.page_stats_u8_deq(qmin, qmax, l, st)
    x = mn.astype(np.float32)
    assert (dmn <= x).all() and (dmx >= x).all()
    assert l[0, 0] == x.min() and O.page_stats_u8_deq(255, 255, l, st)[0][0, 0] >= x.max()
    # the codes are tight to within a couple of steps (the rounding loop stops early)
    assert ((x - dmn) <= 2 * st).all() and ((dmx - x) <= 2 * st).all()


def test_page_stats_u8_degenerate_and_non_finite():
    mn = np.full((5, 2, 3), 1.5, np.float16)
    qmin, qmax, lo, st = O.page_stats_u8(mn, mn)
    assert (qmin == 0).all() and (qmax == 0).all() and (lo == 1.5).all() and (st == 1.0).all()
    mn = np.array([[[np.nan, -np.inf]], [[1.0, 2.0]]], np.float16)   # (P=2, H=1, D=2)
    mx = np.array([[[np.inf, 3.0]], [[np.nan, 2.0]]], np.float16)
    qmin, qmax, lo, st = O.page_stats_u8(mn, mx)
    assert qmin[0, 0, 0] == 0 and qmin[0, 0, 1] == 0 and qmax[0, 0, 0] == 255 and qmax[1, 0, 0] == 255
    assert lo[0, 0] == 1.0 and lo[0, 1] == 2.0  # ranges over the finite statistics only
    dmn, dmx = O.page_stats_u8_deq(qmin, qmax, lo, st)
    assert dmn[1, 0, 0] <= 1.0 and dmx[0, 0, 1] >= 3.0 and dmx[1, 0, 1] >= 2.0


def test_page_bound_u8_never_below_fp16_bound():
    """Dequantised statistics bracket the originals, products and sums round
    monotonically, and the order is the same: no page's bound drops."""
    rng = np.random.default_rng(11)
    P, H, D, g = 2000, 4, 128, 7
    mn = (rng.standard_t(3, (P, H, D)) * 0.7).astype(np.float16)
    mx = (mn.astype(np.float32) + np.abs(rng.standard_t(3, (P, H, D)))).astype(np.float16)
    q = rng.standard_normal((H * g, D)).astype(np.float16)
    dmn, dmx = O.page_stats_u8_deq(*O.page_stats_u8(mn, mx))
    b16 = O.page_bound_group(q, mn, mx, g)
    b8 = O.page_bound_group(q, dmn, dmx, g)
    assert (b8 >= b16).all()
    assert np.median((b8 - b16) / np.abs(b16).max()) < 0.05  # still a useful bound
