"""GPU parity of Quest selection and fused decode attention over the paged
compact pool (a block table scattering a sequence's pages over the pool):
the selection bit-exact against the oracle's bound + top-K over the logical
pages' statistics, the attention against the oracle's float64
selected_attention (h // group head map) over pages the oracle gathers from
the pool bytes.  Tolerance: per query head, relative L2 error and max-abs
error over max |ref| both <= 1e-3."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(2602)
H, D, PS, TOL = 4, 128, 16, 1e-3


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _scales(n, L, thr=1.2):
    poles = np.sort(RNG.standard_normal((H, n, L)), axis=-1).astype(np.float16)
    up = np.full((H, n), thr, np.float16)
    return poles, up, (-up).astype(np.float16)


def _sequence(dev, T, Lk, Lv, NB, rows=2048, cap=256):
    """A T-token sequence written into a pool of NB blocks through a random
    block table: returns the device sides and tables, the block table, and
    the oracle's pools."""
    from helix_kv.ops import NuqLayerTables
    from helix_kv.paged import PagedSide, paged_write

    P = -(-T // PS)
    bt = RNG.permutation(NB)[:P].astype(np.int64)
    slots = bt[np.arange(T) // PS] * PS + np.arange(T) % PS
    k = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
    v = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
    ks, vs = _scales(D, Lk), _scales(rows, Lv)
    kt = NuqLayerTables(*(_t(a, dev) for a in ks), per_token=False)
    vt = NuqLayerTables(*(_t(a, dev) for a in vs), per_token=True)
    kb, vb = (2 if Lk <= 4 else 4), (2 if Lv <= 4 else 4)
    kside = PagedSide.empty(NB, H, kb, cap, dev, stats=True, n_chunks=NB * H)
    vside = PagedSide.empty(NB, H, vb, cap, dev, n_chunks=NB * H)
    pos = np.arange(T)
    paged_write(kside, _t(k, dev), kt, _t(slots, dev))
    paged_write(vside, _t(v, dev), vt, _t(slots, dev), _t(pos, dev))
    kp = O.paged_empty(NB, H, D, kb, cap, stats=True)
    vp = O.paged_empty(NB, H, D, vb, cap, stats=False)
    O.paged_write(kp, k, slots, [a.astype(np.float32) for a in ks], False)
    O.paged_write(vp, v, slots, [a.astype(np.float32) for a in vs], True, positions=pos)
    first = np.arange(P) * PS
    kpages = O.h2f(O.paged_gather(kp, bt, first, ks[0].astype(np.float32), False))
    vpages = O.h2f(O.paged_gather(vp, bt, first, vs[0].astype(np.float32), True))
    return dict(kside=kside, vside=vside, kt=kt, vt=vt, bt=bt, btd=_t(bt, dev), kp=kp, T=T, P=P,
                kpages=kpages, vpages=vpages)


def _stats(S):
    """The logical pages' K statistics from the oracle pool, as float32."""
    return O.h2f(S["kp"]["kmin"][S["bt"]]), O.h2f(S["kp"]["kmax"][S["bt"]])


def _check(got, want):
    got = got.float().cpu().numpy().astype(np.float64)
    for h in range(want.shape[0]):
        ref = want[h]
        err = got[h] - ref
        assert np.linalg.norm(err) <= TOL * np.linalg.norm(ref), h
        assert np.abs(err).max() <= TOL * np.abs(ref).max(), h


@pytest.mark.parametrize("T,group,k,s", [(3000, 7, 40, 4), (16 * 2600, 7, 650, 4), (100, 1, 3, 2)])
def test_paged_select_vs_oracle(dev, T, group, k, s):
    from helix_kv.paged import paged_select

    S = _sequence(dev, T, 16, 4, NB=-(-T // PS) + 37)
    mn, mx = _stats(S)
    q = RNG.standard_normal((H * group, D)).astype(np.float16)
    sel, scores = paged_select(_t(q, dev), S["kside"], S["btd"], T, k, s)
    want = O.page_bound_group(q, mn, mx, group)
    assert np.array_equal(scores.cpu().numpy(), want.T)
    assert np.array_equal(sel.cpu().numpy(), O.topk_sinks(want, k, s))


def test_paged_select_invalid_block_is_never_chosen(dev):
    from helix_kv.paged import paged_select

    S = _sequence(dev, 1600, 16, 4, NB=120)
    bt = S["bt"].copy()
    bt[[7, 50]] = [-1, 10**6]
    q = RNG.standard_normal((H, D)).astype(np.float16)
    sel, scores = paged_select(_t(q, dev), S["kside"], _t(bt, dev), S["T"], 30, 4)
    sc = scores.cpu().numpy()
    assert np.isneginf(sc[:, [7, 50]]).all()
    assert not np.isin(sel.cpu().numpy(), [7, 50]).any()


@pytest.mark.parametrize("T,group,Lk,Lv,frac,pps", [
    (3000, 7, 16, 4, 0.3, 8),      # partial last page, nuq4 K / nuq2 V
    (4096, 7, 4, 16, 0.25, 88),    # nuq2 K / nuq4 V, one split per head
    (257, 1, 16, 16, 1.0, 1),      # group 1, every page
    (2000, 16, 4, 4, 0.5, 12),     # group 16
])
def test_paged_decode_vs_oracle(dev, T, group, Lk, Lv, frac, pps):
    from helix_kv.paged import paged_decode_attention

    S = _sequence(dev, T, Lk, Lv, NB=-(-T // PS) + 11)
    P = S["P"]
    n = P if frac >= 1 else max(min(P, 4) + 1, int(frac * P))
    cols = [np.sort(np.concatenate([np.arange(min(4, P)),
                                    RNG.permutation(np.arange(min(4, P), P))[: n - min(4, P)]]))
            for _ in range(H)]
    sel = np.stack(cols, 1).astype(np.int64)
    bad = np.concatenate([sel, [[-1] * H, [P] * H]]).astype(np.int64)   # skipped ids
    q = RNG.standard_normal((H * group, D)).astype(np.float16)
    want = O.selected_attention(q.astype(np.float64), S["kpages"], S["vpages"], sel,
                                lambda h: h // group, num_tokens=T)
    got = paged_decode_attention(_t(q, dev), S["kside"], S["kt"], S["vside"], S["vt"], S["btd"], T,
                                 _t(bad, dev), pages_per_split=pps, out_dtype=torch.float32)
    _check(got, want)


@pytest.mark.parametrize("cap", [24, 300])
def test_paged_decode_overflow_chunks(dev, cap):
    """Page-heads whose outliers pass the inline capacity keep the rest in
    overflow chunks (cap 24: nearly every page-head; 300: beyond the 256
    entries held in registers), and the decode patches them all."""
    from helix_kv.paged import paged_decode_attention

    T, group = 2500, 7
    S = _sequence(dev, T, 16, 16, NB=200, cap=cap)
    assert int(S["kside"].ovf_next.item()) > 0 or cap > 256
    P = S["P"]
    sel = np.stack([np.sort(RNG.permutation(P)[: P // 2]) for _ in range(H)], 1).astype(np.int64)
    q = RNG.standard_normal((H * group, D)).astype(np.float16)
    want = O.selected_attention(q.astype(np.float64), S["kpages"], S["vpages"], sel,
                                lambda h: h // group, num_tokens=T)
    got = paged_decode_attention(_t(q, dev), S["kside"], S["kt"], S["vside"], S["vt"], S["btd"], T,
                                 _t(sel, dev), pages_per_split=12, out_dtype=torch.float32)
    _check(got, want)


@pytest.mark.parametrize("gqa,select", [("mean", "union"), ("sum", "per_head")])
def test_paged_decode_step_vs_oracle(dev, gqa, select):
    from helix_kv.paged import paged_decode_step

    T, group, top_k, sinks = 5000, 7, 60, 4
    S = _sequence(dev, T, 16, 4, NB=400)
    P = S["P"]
    mn, mx = _stats(S)
    q = RNG.standard_normal((H * group, D)).astype(np.float16)
    qd = _t(q, dev)
    if gqa == "mean":
        qs = qd.reshape(H, group, D).mean(dim=1).to(torch.float16).cpu().numpy()  # the reference's op
        bound = O.page_bound(qs, mn, mx)
    else:
        bound = O.page_bound_group(q, mn, mx, group)
    sel = O.topk_sinks(bound, top_k, sinks)
    if select == "union":
        ids = np.unique(sel.reshape(-1))
        assert sinks + top_k < ids.size < P
        sel = np.repeat(ids[:, None], H, axis=1)
    want = O.selected_attention(q.astype(np.float64), S["kpages"], S["vpages"], sel,
                                lambda h: h // group, num_tokens=T)
    got = paged_decode_step(qd, S["kside"], S["kt"], S["vside"], S["vt"], S["btd"], T, top_k, sinks,
                            gqa=gqa, select=select, out_dtype=torch.float32)
    _check(got, want)


def test_paged_decode_step_graph_replay(dev):
    """The paged step reads nothing back, so it records into a HIP graph:
    three replays, with eager work between them, equal the eager result."""
    from helix_kv.paged import paged_decode_step

    T, group = 3300, 7
    S = _sequence(dev, T, 4, 16, NB=300)
    q = _t(RNG.standard_normal((H * group, D)).astype(np.float16), dev)
    args = (q, S["kside"], S["kt"], S["vside"], S["vt"], S["btd"], T, 50, 4)
    eager = paged_decode_step(*args).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        paged_decode_step(*args)
    torch.cuda.current_stream().wait_stream(side)
    out = torch.empty_like(eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_step(*args, out=out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        other = paged_decode_step(*args, select="per_head")
        torch.cuda.synchronize()
        assert not torch.equal(other, eager)


def _batch_pool(dev, lens, Lk, Lv, spare=23, cap=256):
    """Sequences of the given lengths written into one pool, each through its
    own random blocks; returns the sides, tables and the (B, M) block table
    (entries past a sequence's pages are -1)."""
    from helix_kv.ops import NuqLayerTables
    from helix_kv.paged import PagedSide, paged_write

    pages = [-(-n // PS) for n in lens]
    NB = sum(pages) + spare
    perm = RNG.permutation(NB).astype(np.int64)
    M = max(pages) + 3
    bt = np.full((len(lens), M), -1, np.int64)
    ks, vs = _scales(D, Lk), _scales(max(lens), Lv)
    kt = NuqLayerTables(*(_t(a, dev) for a in ks), per_token=False)
    vt = NuqLayerTables(*(_t(a, dev) for a in vs), per_token=True)
    kb, vb = (2 if Lk <= 4 else 4), (2 if Lv <= 4 else 4)
    kside = PagedSide.empty(NB, H, kb, cap, dev, stats=True, n_chunks=NB * H)
    vside = PagedSide.empty(NB, H, vb, cap, dev, n_chunks=NB * H)
    kp = O.paged_empty(NB, H, D, kb, cap, stats=True)
    vp = O.paged_empty(NB, H, D, vb, cap, stats=False)
    o = 0
    for b, (T, P) in enumerate(zip(lens, pages)):
        bt[b, :P] = perm[o:o + P]
        o += P
        slots = bt[b, np.arange(T) // PS] * PS + np.arange(T) % PS
        k = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
        v = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
        paged_write(kside, _t(k, dev), kt, _t(slots, dev))
        paged_write(vside, _t(v, dev), vt, _t(slots, dev), _t(np.arange(T), dev))
        O.paged_write(kp, k, slots, [a.astype(np.float32) for a in ks], False)
        O.paged_write(vp, v, slots, [a.astype(np.float32) for a in vs], True, positions=np.arange(T))
    oracle_pages, stats = [], []
    for b, P in enumerate(pages):
        first = np.arange(P) * PS
        oracle_pages.append((O.h2f(O.paged_gather(kp, bt[b, :P], first, ks[0].astype(np.float32), False)),
                             O.h2f(O.paged_gather(vp, bt[b, :P], first, vs[0].astype(np.float32), True))))
        stats.append((O.h2f(kp["kmin"][bt[b, :P]]), O.h2f(kp["kmax"][bt[b, :P]])))
    return kside, vside, kt, vt, _t(bt, dev), oracle_pages, stats


@pytest.mark.parametrize("gqa,select", [("mean", "union"), ("sum", "per_head"), ("mean", "per_head")])
def test_paged_decode_step_batch_equals_single_steps(dev, gqa, select):
    """One batched paged step over sequences of one pool equals paged_decode_step
    per sequence (same pages_per_split) bit for bit, with per-sequence top_k
    and a sequence shorter than its sinks + top_k; the step records into a
    HIP graph whose replays give the eager result."""
    from helix_kv.paged import paged_decode_step, paged_decode_step_batch

    lens = [3000, 700, 16 * 97, 33, 2100]
    top_k = [40, 12, 30, 50, 25]
    group, sinks, pps = 7, 4, 9
    kside, vside, kt, vt, btd, _, _ = _batch_pool(dev, lens, 16, 4)
    q = _t(RNG.standard_normal((len(lens), H * group, D)).astype(np.float16), dev)
    got = paged_decode_step_batch(q, kside, kt, vside, vt, btd, lens, top_k, sinks, gqa=gqa,
                                  select=select, pages_per_split=pps)
    for b, T in enumerate(lens):
        P = -(-T // PS)
        want = paged_decode_step(q[b], kside, kt, vside, vt, btd[b, :P], T, top_k[b], sinks,
                                 gqa=gqa, select=select, pages_per_split=pps)
        assert torch.equal(got[b], want), b
    out = torch.empty_like(got)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        paged_decode_step_batch(q, kside, kt, vside, vt, btd, lens, top_k, sinks, gqa=gqa,
                                select=select, pages_per_split=pps)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        paged_decode_step_batch(q, kside, kt, vside, vt, btd, lens, top_k, sinks, gqa=gqa,
                                select=select, pages_per_split=pps, out=out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, got)
        paged_decode_step(q[0], kside, kt, vside, vt, btd[0], lens[0], 5, 1)
        torch.cuda.synchronize()


def test_paged_decode_step_batch_above_64_sequences(dev):
    """70 sequences run as batches of 64 and 6: each result equals
    paged_decode_step on its own, bit for bit, in both select modes."""
    from helix_kv.paged import paged_decode_step, paged_decode_step_batch

    lens = [int(n) for n in np.random.default_rng(71).integers(1, 200, 70)]
    kside, vside, kt, vt, btd, _, _ = _batch_pool(dev, lens, 4, 16)
    q = _t(RNG.standard_normal((len(lens), H * 2, D)).astype(np.float16), dev)
    for select in ("union", "per_head"):
        got = paged_decode_step_batch(q, kside, kt, vside, vt, btd, lens, 3, 2, select=select,
                                      pages_per_split=2)
        for b, T in enumerate(lens):
            P = -(-T // PS)
            want = paged_decode_step(q[b], kside, kt, vside, vt, btd[b, :P], T, 3, 2, select=select,
                                     pages_per_split=2)
            assert torch.equal(got[b], want), (select, b)


def test_paged_decode_attention_batch_vs_oracle(dev):
    """The batched paged decode (hkv_paged_decode_attn_batch) over given
    selections, nuq2 K / nuq4 V, against the oracle's float64 attention over
    each sequence's pages gathered from the pool bytes."""
    import ctypes

    from helix_kv import _native as N

    lens, group, pps = [900, 1601, 40], 4, 5
    B = len(lens)
    kside, vside, kt, vt, btd, opages, _ = _batch_pool(dev, lens, 4, 16, spare=5)
    q = RNG.standard_normal((B, H * group, D)).astype(np.float16)
    sels, offs = [], [0]
    for T in lens:
        P = -(-T // PS)
        n = max(1, P // 3)
        sels.append(np.stack([np.sort(RNG.permutation(P)[:n]) for _ in range(H)], 1).astype(np.int64))
        offs.append(offs[-1] + n)
    sel = np.concatenate(sels)
    qd, seld = _t(q, dev), _t(sel, dev)
    out = torch.empty((B, H * group, D), dtype=torch.float32, device=dev)
    c_sel = (ctypes.c_int64 * (B + 1))(*offs)
    M = int(btd.shape[1])
    ws = torch.empty(int(N.lib().hkv_decode_batch_workspace_bytes(B, c_sel, H * group, pps)),
                     dtype=torch.uint8, device=dev)
    st = N.lib().hkv_paged_decode_attn_batch(
        N.ptr(qd), B, H * group, (ctypes.c_int64 * B)(*lens), N.ptr(btd),
        (ctypes.c_int64 * B)(*[b * M for b in range(B)]), kside.desc(), N.ptr(kt.ensure_tables()),
        vside.desc(), N.ptr(vt.ensure_tables()), vt.rows, N.ptr(seld), c_sel, pps, D ** -0.5,
        N.ptr(out), N.dtype_code(out), N.ptr(ws), ws.numel(), N.stream_of(qd))
    assert st == 0
    torch.cuda.synchronize()
    for b, T in enumerate(lens):
        want = O.selected_attention(q[b].astype(np.float64), *opages[b], sels[b], lambda h: h // group,
                                    num_tokens=T)
        _check(out[b], want)


@pytest.mark.parametrize("group", [7, 1])
def test_paged_select_ragged_vs_oracle(dev, group):
    """The ragged paged selection (one bound and one top-K launch for the
    batch) against the oracle's group-summed bound and top-K with sinks over
    each sequence's logical pages, bit for bit, scores included; a block-table
    entry outside the pool scores -inf and is not chosen."""
    from helix_kv.paged import paged_select_ragged

    lens = [1000, 16 * 300, 50, 16 * 41 + 3]
    top_k, sinks = [20, 100, 9, 30], 4
    kside, _, _, _, btd, _, stats = _batch_pool(dev, lens, 16, 4)
    bt = btd.cpu().numpy()
    bt[1, 17] = -1
    bt[3, 30] = 10**7
    q = RNG.standard_normal((len(lens), H * group, D)).astype(np.float16)
    sel, rows, scores = paged_select_ragged(_t(q, dev), kside, _t(bt, dev), lens, top_k, sinks)
    sel, scores = sel.cpu().numpy(), scores.cpu().numpy()
    p0 = 0
    for b, T in enumerate(lens):
        P = -(-T // PS)
        want = O.page_bound_group(q[b], *stats[b], group)
        bad = bt[b, :P] < 0
        bad |= bt[b, :P] >= kside.num_blocks
        want[bad] = -np.inf
        assert np.array_equal(scores[:, p0:p0 + P], want.T), b
        got = sel[rows[b]:rows[b + 1]]
        assert np.array_equal(got, O.topk_sinks(want, top_k[b], sinks)), b
        assert not np.isin(got, np.flatnonzero(bad)).any(), b
        p0 += P


@pytest.mark.parametrize("H8", [8, 16])
def test_paged_select_ragged_and_batch_step_more_heads(dev, H8):
    """Pools with 8 and 16 KV heads: the ragged paged selection (a bound lane
    still holds one head: the heads divide a block's 16 rows) against the
    oracle's group-summed bound and top-K with sinks, bit for bit; the
    batched paged step equal to paged_decode_step per sequence."""
    from helix_kv.ops import NuqLayerTables
    from helix_kv.paged import (PagedSide, paged_decode_step, paged_decode_step_batch, paged_select_ragged,
                                paged_write)

    lens, top_k, sinks, group = [700, 1300, 90], [30, 60, 5], 4, 2
    pages = [-(-n // PS) for n in lens]
    NB = sum(pages) + 9
    perm = RNG.permutation(NB).astype(np.int64)
    bt = np.full((len(lens), max(pages) + 1), -1, np.int64)
    kpol = np.sort(RNG.standard_normal((H8, D, 16)), axis=-1).astype(np.float16)
    kup = np.full((H8, D), 1.2, np.float16)
    vpol = np.sort(RNG.standard_normal((H8, 2048, 4)), axis=-1).astype(np.float16)
    vup = np.full((H8, 2048), 1.2, np.float16)
    kt = NuqLayerTables(_t(kpol, dev), _t(kup, dev), _t(-kup, dev), per_token=False)
    vt = NuqLayerTables(_t(vpol, dev), _t(vup, dev), _t(-vup, dev), per_token=True)
    kside = PagedSide.empty(NB, H8, 4, 256, dev, stats=True, n_chunks=NB * H8)
    vside = PagedSide.empty(NB, H8, 2, 256, dev, n_chunks=NB * H8)
    kp = O.paged_empty(NB, H8, D, 4, 256, stats=True)
    o = 0
    for b, (T, P) in enumerate(zip(lens, pages)):
        bt[b, :P] = perm[o:o + P]
        o += P
        slots = bt[b, np.arange(T) // PS] * PS + np.arange(T) % PS
        k = (RNG.standard_t(3, (T, H8, D)) * 0.7).astype(np.float16)
        v = (RNG.standard_t(3, (T, H8, D)) * 0.7).astype(np.float16)
        paged_write(kside, _t(k, dev), kt, _t(slots, dev))
        paged_write(vside, _t(v, dev), vt, _t(slots, dev), _t(np.arange(T), dev))
        O.paged_write(kp, k, slots, [kpol.astype(np.float32), kup.astype(np.float32),
                                     (-kup).astype(np.float32)], False)
    q = RNG.standard_normal((len(lens), H8 * group, D)).astype(np.float16)
    qd, btd = _t(q, dev), _t(bt, dev)
    sel, rows, scores = paged_select_ragged(qd, kside, btd, lens, top_k, sinks)
    sel, scores = sel.cpu().numpy(), scores.cpu().numpy()
    p0 = 0
    for b, P in enumerate(pages):
        mn, mx = O.h2f(kp["kmin"][bt[b, :P]]), O.h2f(kp["kmax"][bt[b, :P]])
        want = O.page_bound_group(q[b], mn, mx, group)
        assert np.array_equal(scores[:, p0:p0 + P], want.T), b
        assert np.array_equal(sel[rows[b]:rows[b + 1]], O.topk_sinks(want, top_k[b], sinks)), b
        p0 += P
    for select in ("union", "per_head"):
        got = paged_decode_step_batch(qd, kside, kt, vside, vt, btd, lens, top_k, sinks, gqa="sum",
                                      select=select, pages_per_split=7)
        for b, (T, P) in enumerate(zip(lens, pages)):
            want = paged_decode_step(qd[b], kside, kt, vside, vt, btd[b, :P], T, top_k[b], sinks, gqa="sum",
                                     select=select, pages_per_split=7)
            assert torch.equal(got[b], want), (select, b)
