"""GPU parity of the Quest kernels against the CPU oracle (bit-exact).

Page statistics, the canonical-order bound (fp32 and fp16 out), top-K with
sinks, and the fused score+select at the full 1M-token shape (65,536 pages).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(5)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dt", [np.float16, np.float32])
@pytest.mark.parametrize("P,S,H,D", [(64, 16, 4, 128), (9, 4, 2, 8), (5, 3, 3, 20)])
def test_page_stats_vs_oracle(dev, dt, P, S, H, D):
    from quest import compute_page_stats

    K = RNG.standard_normal((P, S, H, D)).astype(dt)
    K[0, :, 0, 0] = [0.0, -0.0] * (S // 2) + [0.0] * (S % 2)
    K[1 % P, 1 % S, 0, 1 % D] = np.nan
    mn, mx = compute_page_stats(_t(K, dev))
    wmn, wmx = O.page_stats(K)
    if dt == np.float16:
        assert np.array_equal(_u16(mn), wmn.view(np.uint16))
        assert np.array_equal(_u16(mx), wmx.view(np.uint16))
    else:
        assert np.array_equal(mn.cpu().numpy().view(np.uint32), wmn.view(np.uint32))
        assert np.array_equal(mx.cpu().numpy().view(np.uint32), wmx.view(np.uint32))


@pytest.mark.parametrize("kdt", [np.float16, np.float32])
@pytest.mark.parametrize("P,H,D,g", [(512, 4, 128, 1), (300, 4, 128, 7), (77, 2, 32, 1),
                                     (50, 3, 128, 2), (33, 5, 64, 1),
                                     (40, 1, 20, 3), (16, 2, 8, 1),
                                     (200, 8, 128, 2), (101, 16, 128, 1)])
def test_bound_bit_exact_vs_oracle(dev, kdt, P, H, D, g):
    from helix_kv.ops import quest_page_bound

    q = RNG.standard_normal((H * g, D)).astype(np.float16)
    mn = RNG.standard_normal((P, H, D)).astype(kdt)
    mx = (mn + RNG.random((P, H, D))).astype(kdt)
    got = quest_page_bound(_t(q, dev), _t(mn, dev), _t(mx, dev)).cpu().numpy()
    want = O.page_bound_group(q, mn, mx, g) if g > 1 else O.page_bound(q, mn, mx)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    got16 = quest_page_bound(_t(q, dev), _t(mn, dev), _t(mx, dev), out_dtype=torch.float16)
    assert np.array_equal(_u16(got16), O.f2h(want))


def test_reference_bound_api(dev):
    # src/quest/tests/test_triton.py:22-51 and test_reference.py:45-63 through the drop-in names
    from quest import compute_page_stats, page_upper_bound
    from quest.triton_kernels import page_upper_bound_triton

    P, H, D = 256, 4, 128
    q = torch.randn(H, D, dtype=torch.float16, device=dev)
    kmin = torch.randn(P, H, D, dtype=torch.float16, device=dev)
    kmax = kmin + torch.rand(P, H, D, dtype=torch.float16, device=dev)
    ref = (q.float().clamp(min=0) * kmax.float()).sum(-1) + (q.float().clamp(max=0) * kmin.float()).sum(-1)
    tri = page_upper_bound_triton(q, kmin, kmax)
    assert tri.dtype == torch.float16 and (tri.float() - ref).abs().max().item() < 0.5
    K = torch.randn(8, 16, 4, 32, device=dev)
    qq = torch.randn(4, 32, device=dev)
    mn, mx = compute_page_stats(K)
    b = page_upper_bound(qq, mn, mx)
    true_max = (K * qq[None, None]).sum(-1).amax(1)
    assert ((b - true_max) >= -1e-4).all()
    with pytest.raises(ValueError):
        page_upper_bound(qq[0], mn, mx)


@pytest.mark.parametrize("P,H,k,s", [(65536, 4, 16384, 4), (1000, 3, 250, 4), (257, 2, 1, 0),
                                     (64, 4, 60, 4), (5, 2, 0, 2), (3, 2, 1, 7), (4097, 1, 4000, 1)])
def test_topk_vs_oracle(dev, P, H, k, s):
    from quest import topk_pages_with_sinks

    b = RNG.standard_normal((P, H)).astype(np.float32)
    b[RNG.integers(0, P, P // 10)] = 0.5  # heavy ties
    b[RNG.integers(0, P, 3), 0] = np.nan
    got = topk_pages_with_sinks(_t(b, dev), k, s).cpu().numpy()
    assert np.array_equal(got, O.topk_sinks(b, k, s))
    got16 = topk_pages_with_sinks(_t(b.astype(np.float16), dev), k, s).cpu().numpy()
    assert np.array_equal(got16, O.topk_sinks(b.astype(np.float16).astype(np.float32), k, s))


def test_topk_all_equal_and_reference_shapes(dev):
    from quest import topk_pages_with_sinks

    b = torch.zeros(100, 4, device=dev)
    sel = topk_pages_with_sinks(b, 10, 4)
    assert torch.equal(sel[:, 0].cpu(), torch.arange(14))
    bound = torch.randn(16, 4, device=dev)
    bound[0, :] = -100.0
    sel = topk_pages_with_sinks(bound, 4, 2)  # src/quest/tests/test_reference.py:66-84
    assert sel.shape == (6, 4)
    assert (sel[:2] == torch.tensor([[0], [1]], device=dev)).all()
    assert (sel[1:] > sel[:-1]).all()
    assert topk_pages_with_sinks(torch.randn(3, 2, device=dev), 10, 1).shape == (3, 2)


@pytest.mark.parametrize("kdt", [np.float16, np.float32])
def test_fused_select_full_size_vs_oracle(dev, kdt):
    """1M tokens: 65,536 pages x 4 KV heads x 128, 28 query heads (7:1), top 25% + 4 sinks."""
    from helix_kv.ops import quest_select

    P, H, D, g = 65536, 4, 128, 7
    K = RNG.standard_normal((P, H, D)).astype(np.float16)
    mn = K.astype(kdt)
    mx = (K + np.abs(RNG.standard_normal((P, H, D))).astype(np.float16)).astype(kdt)
    q = RNG.standard_normal((H * g, D)).astype(np.float16)
    idx, scores = quest_select(_t(q, dev), _t(mn, dev), _t(mx, dev), P // 4, 4)
    want_b = O.page_bound_group(q, mn, mx, g)
    assert np.array_equal(scores.cpu().numpy().T.view(np.uint32), want_b.view(np.uint32))
    got = idx.cpu().numpy()
    assert got.shape == (P // 4 + 4, H)
    assert np.array_equal(got, O.topk_sinks(want_b, P // 4, 4))
    # repeat: the per-head completion counters reset themselves
    idx2, _ = quest_select(_t(q, dev), _t(mn, dev), _t(mx, dev), P // 4, 4)
    assert torch.equal(idx2, idx)


def test_fused_select_small_and_per_kv_head(dev):
    from helix_kv.ops import quest_select

    for P, H, D, g, k, s in [(100, 2, 32, 1, 30, 4), (10, 4, 128, 1, 20, 2), (1, 1, 8, 2, 1, 0)]:
        q = RNG.standard_normal((H * g, D)).astype(np.float16)
        mn = RNG.standard_normal((P, H, D)).astype(np.float16)
        mx = (mn + 1).astype(np.float16)
        idx, sc = quest_select(_t(q, dev), _t(mn, dev), _t(mx, dev), k, s)
        wb = O.page_bound_group(q, mn, mx, g) if g > 1 else O.page_bound(q, mn, mx)
        assert np.array_equal(sc.cpu().numpy().T, wb)
        assert np.array_equal(idx.cpu().numpy(), O.topk_sinks(wb, k, s))


@pytest.mark.parametrize("P,H,g,k,s,mode,D", [(*c, 128) if len(c) == 6 else c for c in [
    (40000, 4, 7, 10000, 4, "normal"),     # five slices, the last one partial
    (65536, 2, 7, 1, 0, "normal"),         # a single page besides no sinks
    (65536, 4, 1, 65532, 4, "normal"),     # every candidate
    (50000, 1, 3, 12345, 7, "ties"),       # few distinct scores: big equal runs
    (70000, 4, 7, 17500, 4, "equal"),      # all scores equal: the huge-bin fallback
    (131072, 2, 7, 32768, 4, "normal"),    # 16 slices: per-slice counts from reloaded groups
    (600000, 2, 7, 150000, 4, "normal"),   # many slices (KPT 32)
    (65536, 2, 7, 100, 4, "nan"),          # NaN ranks highest: the threshold in the top bin
    (65536, 2, 7, 5000, 1, "nan"),         # NaN present (coarse bins), one sink: unaligned column
    # more slice blocks than CUs: the two-kernel form (threshold by the last block, then a write kernel)
    (40960, 64, 1, 10240, 4, "normal", 8),     # 5 slices x 64 heads
    (540000, 16, 2, 135000, 4, "normal", 32),  # 17 slices of 32768 x 16 heads (KPT 32)
    # 8 and 16 KV heads at head dim 128: a bound lane keeps its head (the heads divide a block's rows)
    (65536, 8, 4, 16384, 4, "normal"),
    (20000, 16, 2, 5000, 4, "normal"),
    # a few bounds of the other sign (2^31 ordered keys below the rest): bins over the top 2^27 keys,
    # the threshold inside them, or (nearly every page kept) in bin 0, open below
    (65536, 4, 4, 16384, 4, "signs"),
    (65536, 4, 4, 65530, 4, "signs"),
    (65536, 2, 7, 30000, 0, "signs"),
]])
def test_multiblock_select_vs_oracle(dev, P, H, g, k, s, mode, D):
    """The multi-block top-K (fp16 statistics, large columns) against the
    oracle, including repeated calls on the same workspace.  Up to one slice
    block per CU every block of a head computes the threshold and writes its
    own slice (fused form); beyond that the two-kernel form runs."""
    from helix_kv.ops import quest_select

    if mode == "equal":
        mn = np.zeros((P, H, D), np.float16)
        mx = np.ones((P, H, D), np.float16)
    elif mode == "ties":
        levels = RNG.integers(0, 5, size=(P, 1, 1)).astype(np.float16)
        mn = np.broadcast_to(levels - 1, (P, H, D)).astype(np.float16)
        mx = np.broadcast_to(levels, (P, H, D)).astype(np.float16)
    else:
        mn = RNG.standard_normal((P, H, D)).astype(np.float16)
        mx = (mn + np.abs(RNG.standard_normal((P, H, D))).astype(np.float16)).astype(np.float16)
    if mode == "signs":  # pages whose bound is +-8 x the group's query sum: bounds of both signs
        mn[100:102] = mx[100:102] = -8.0
        mn[102:104] = mx[102:104] = 8.0
    if mode == "nan":  # 300 pages whose bound is NaN
        bad = RNG.choice(P, 300, replace=False)
        mn[bad, :, 5] = np.nan
        mx[bad, :, 5] = np.nan
    q = RNG.standard_normal((H * g, D)).astype(np.float16)
    want_b = O.page_bound_group(q, mn.astype(np.float32), mx.astype(np.float32), g)
    want = O.topk_sinks(want_b, k, s)
    nan = np.isnan(want_b)
    for _ in range(2):
        idx, scores = quest_select(_t(q, dev), _t(mn, dev), _t(mx, dev), k, s)
        got_b = scores.cpu().numpy().T
        assert np.array_equal(np.isnan(got_b), nan)  # NaN payloads are not compared
        assert np.array_equal(got_b[~nan].view(np.uint32), want_b[~nan].view(np.uint32))
        assert np.array_equal(idx.cpu().numpy(), want)


@pytest.mark.parametrize("P,H,g,k,s,mode,dt", [
    (65536, 4, 7, 16384, 4, "normal", np.float16),   # 1M tokens
    (1000, 2, 7, 250, 4, "normal", np.float32),      # fp32 statistics
    (40000, 4, 1, 100, 0, "heavy", np.float16),      # Student-t tails: wide ranges, dense bins
    (300, 1, 3, 50, 2, "const", np.float16),         # constant channels (step 1, codes 0)
    (5000, 4, 7, 1000, 4, "nonfinite", np.float16),  # NaN / inf statistics code as the full range
    (20000, 8, 4, 5000, 4, "normal", np.float16),    # 8 KV heads
])
def test_u8_metadata_select_vs_oracle(dev, P, H, g, k, s, mode, dt):
    """Compact u8 page metadata: the conversion bit-exact against the oracle,
    the select's scores bit-exact against the oracle bound over the
    dequantised statistics, its pages against the oracle top-K, and no score
    below the fp16 select's for the same page."""
    from helix_kv.ops import quest_page_stats_u8, quest_select, quest_select_u8

    D = 128
    if mode == "const":
        mn = np.broadcast_to(RNG.standard_normal((1, H, D)), (P, H, D)).astype(dt)
        mx = (mn.astype(np.float32) + 1).astype(dt)
    else:
        gen = RNG.standard_t(3, (P, H, D)) if mode == "heavy" else RNG.standard_normal((P, H, D))
        mn = gen.astype(dt)
        mx = (mn.astype(np.float32) + np.abs(RNG.standard_normal((P, H, D)))).astype(dt)
    if mode == "nonfinite":
        bad = RNG.choice(P, 40, replace=False)
        mn[bad[:20], :, 3] = np.nan
        mx[bad[20:], :, 7] = np.inf
    q = RNG.standard_normal((H * g, D)).astype(np.float16)
    qmin, qmax, lo, st = O.page_stats_u8(mn, mx)
    got = quest_page_stats_u8(_t(mn, dev), _t(mx, dev))
    assert np.array_equal(got.qmin.cpu().numpy(), qmin) and np.array_equal(got.qmax.cpu().numpy(), qmax)
    assert np.array_equal(got.lo.cpu().numpy().view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(got.step.cpu().numpy().view(np.uint32), st.view(np.uint32))
    dmn, dmx = O.page_stats_u8_deq(qmin, qmax, lo, st)
    want_b = O.page_bound_group(q, dmn, dmx, g)
    for _ in range(2):  # the workspace is reused
        idx, sc = quest_select_u8(_t(q, dev), got, k, s)
        b = sc.cpu().numpy().T
        assert np.array_equal(b.view(np.uint32), want_b.view(np.uint32))
        assert np.array_equal(idx.cpu().numpy(), O.topk_sinks(want_b, k, s))
    if dt == np.float16:
        _, sc16 = quest_select(_t(q, dev), _t(mn, dev), _t(mx, dev), k, s)
        b16 = sc16.cpu().numpy().T
        fin = np.isfinite(b16)
        assert (b[fin] >= b16[fin]).all()
