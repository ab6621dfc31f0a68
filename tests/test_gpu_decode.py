"""GPU parity of the fused dequant + Quest-sparse decode attention.

The kernel reads K/V in the compact format written by the GPU pack; the
expected output is the oracle's float64 attention (selected_attention, the
restatement of src/quest/reference.py:136-168 with the h // group GQA map)
over K/V that the oracle itself decodes from the same compact bytes
(bitunpack + csr_decode + unpack).  Tolerance, written per test: the
per-head relative L2 error and the per-head max abs error over max |ref| are
both <= 1e-3 (P is rounded to fp16 for the PV product: relative error about
2^-12 per term).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(55)
PS = 16
TOL = 1e-3


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _scales(H, n, L, thr):
    poles = np.sort(RNG.standard_normal((H, n, L)), axis=-1).astype(np.float16)
    up = np.full((H, n), thr, np.float16)
    return poles, up, (-up).astype(np.float16)


def _side(dev, x, poles, up, lo, per_token, bits):
    """GPU compact pack, then the oracle's decode of the packed bytes."""
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact

    T, H, D = x.shape
    lt = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(lo, dev), per_token=per_token)
    cc = nuq_pack_compact(_t(x, dev), lt, bits)
    codes = O.bitunpack(cc.packed.cpu().numpy(), bits, D)
    m, v = O.csr_decode(cc.row_ptr.cpu().numpy(), cc.col.cpu().numpy(),
                        cc.val.cpu().numpy().view(np.uint16), T * H, D)
    deq = O.unpack(codes, v.reshape(T, H, D), m.reshape(T, H, D), poles.astype(np.float32),
                   "v" if per_token else "k")
    return cc, lt, O.h2f(deq)


def _problem(dev, T, H, Lk, Lv, rows, thr=1.2):
    D = 128
    k = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
    v = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
    kp, ku, kl = _scales(H, D, Lk, thr)
    vp, vu, vl = _scales(H, rows, Lv, thr)
    kc, kt, kd = _side(dev, k, kp, ku, kl, False, 4 if Lk > 4 else 2)
    vc, vt, vd = _side(dev, v, vp, vu, vl, True, 4 if Lv > 4 else 2)
    P = -(-T // PS)
    pad = P * PS - T
    kd = np.concatenate([kd, np.zeros((pad, H, D))]).reshape(P, PS, H, D)
    vd = np.concatenate([vd, np.zeros((pad, H, D))]).reshape(P, PS, H, D)
    return kc, kt, kd, vc, vt, vd


def _select(P, H, n, sinks=4):
    cols = []
    for _ in range(H):
        rest = RNG.permutation(np.arange(sinks, P))[: n - sinks]
        cols.append(np.sort(np.concatenate([np.arange(sinks), rest])))
    return np.stack(cols, 1).astype(np.int64)


def _check(got, want):
    got = got.float().cpu().numpy().astype(np.float64)
    for h in range(want.shape[0]):
        ref = want[h]
        err = got[h] - ref
        assert np.linalg.norm(err) <= TOL * np.linalg.norm(ref), h
        assert np.abs(err).max() <= TOL * np.abs(ref).max(), h


@pytest.mark.parametrize("T,H,group,Lk,Lv,rows,frac,pps", [
    (1000, 2, 7, 16, 4, 512, 0.5, 4),     # partial last page, V row clamp
    (4096, 4, 7, 16, 16, 4096, 0.25, 8),  # nuq4 both, cfg5 GQA 7:1
    (4096, 4, 7, 4, 4, 4096, 0.25, 88),   # nuq2 both, one split per head
    (257, 1, 1, 4, 16, 300, 1.0, 1),      # group 1, idle waves in each split
    (2048, 2, 16, 16, 4, 64, 0.3, 12),    # group 16, split not a multiple of 4
])
def test_decode_vs_oracle(dev, T, H, group, Lk, Lv, rows, frac, pps):
    from helix_kv.ops import decode_attention

    kc, kt, kd, vc, vt, vd = _problem(dev, T, H, Lk, Lv, rows)
    P = kd.shape[0]
    n = max(min(P, 4) + 1, int(frac * P)) if frac < 1 else P
    sel = _select(P, H, min(n, P), sinks=min(4, P))
    q = RNG.standard_normal((H * group, 128)).astype(np.float16)
    want = O.selected_attention(q.astype(np.float64), kd, vd, sel, lambda h: h // group,
                                num_tokens=T)
    out = decode_attention(_t(q, dev), kc, kt, vc, vt, _t(sel, dev), pages_per_split=pps,
                           out_dtype=torch.float32)
    _check(out, want)
    out16 = decode_attention(_t(q, dev), kc, kt, vc, vt, _t(sel, dev), out_dtype=torch.float16)
    assert out16.dtype == torch.float16
    _check(out16, want)


def test_decode_invalid_ids_and_scale(dev):
    from helix_kv.ops import decode_attention

    T, H, group = 700, 2, 3
    kc, kt, kd, vc, vt, vd = _problem(dev, T, H, 16, 16, 1024)
    P = kd.shape[0]
    sel = _select(P, H, 12)
    bad = np.concatenate([sel, [[-1, P], [P + 5, -7]]]).astype(np.int64)
    q = RNG.standard_normal((H * group, 128)).astype(np.float16)
    want = O.selected_attention(q.astype(np.float64), kd, vd, sel, lambda h: h // group,
                                num_tokens=T, scale=0.05)
    out = decode_attention(_t(q, dev), kc, kt, vc, vt, _t(bad, dev), scale=0.05,
                           pages_per_split=4, out_dtype=torch.float32)
    _check(out, want)


def test_decode_all_pages_equals_dense_sdpa(dev):
    """Every page selected == dense attention over all T tokens (torch's fp32
    scaled_dot_product_attention on the CPU over the oracle-decoded K/V);
    src/quest/tests/test_reference.py:95-117."""
    from helix_kv.ops import decode_attention

    T, H, group = 1500, 2, 7
    kc, kt, kd, vc, vt, vd = _problem(dev, T, H, 16, 4, 2048)
    P = kd.shape[0]
    sel = np.stack([np.arange(P)] * H, 1).astype(np.int64)
    q = RNG.standard_normal((H * group, 128)).astype(np.float16)
    out = decode_attention(_t(q, dev), kc, kt, vc, vt, _t(sel, dev), out_dtype=torch.float32)
    K = torch.tensor(kd.reshape(-1, H, 128)[:T], dtype=torch.float32).permute(1, 0, 2)
    V = torch.tensor(vd.reshape(-1, H, 128)[:T], dtype=torch.float32).permute(1, 0, 2)
    Q = torch.tensor(q, dtype=torch.float32).reshape(H, group, 128)
    want = torch.nn.functional.scaled_dot_product_attention(Q, K, V).reshape(H * group, 128)
    _check(out, want.double().numpy())


def test_decode_errors(dev):
    from helix_kv.ops import decode_attention

    kc, kt, kd, vc, vt, vd = _problem(dev, 64, 2, 16, 16, 64)
    sel = torch.zeros((2, 2), dtype=torch.int64, device=dev)
    q = torch.zeros((6, 128), dtype=torch.float16, device=dev)
    with pytest.raises(ValueError):
        decode_attention(q[:5], kc, kt, vc, vt, sel)         # Hq not a multiple of H
    with pytest.raises(ValueError):
        decode_attention(q, kc, kt, vc, vt, sel[:, :1])      # sel columns != H
    with pytest.raises(AssertionError):
        decode_attention(q.float(), kc, kt, vc, vt, sel)     # query dtype
    with pytest.raises(AssertionError):
        decode_attention(q, kc, vt, vc, vt, sel)             # K tables must be per-channel
    q34 = torch.zeros((34, 128), dtype=torch.float16, device=dev)
    with pytest.raises(AssertionError):
        decode_attention(q34, kc, kt, vc, vt, sel)           # group 17 > 16


@pytest.mark.parametrize("dt,S,H,D,gqa", [(torch.float32, 8, 4, 64, False),
                                          (torch.float16, 16, 3, 128, False),
                                          (torch.bfloat16, 4, 2, 32, False),
                                          (torch.float16, 16, 4, 128, True)])
def test_dense_selected_attention_vs_oracle(dev, dt, S, H, D, gqa):
    """quest.selected_attention (src/quest/reference.py:136-168) on dense
    pages; with gqa the query heads map to KV head h // group."""
    from helix_kv.ops import selected_attention
    from quest import selected_attention as ref_api

    P, n = 50, 9
    Hq = H * 7 if gqa else H
    K = torch.randn((P, S, H, D), dtype=torch.float32).to(dt)
    V = torch.randn((P, S, H, D), dtype=torch.float32).to(dt)
    q = torch.randn((Hq, D), dtype=torch.float32).to(dt)
    cols = H if gqa else Hq
    sel = torch.stack([torch.randperm(P)[:n].sort().values for _ in range(cols)], 1)
    kv = (lambda h: h // 7) if gqa else (lambda h: h)
    want = O.selected_attention(q.double().numpy(), K.double().numpy(), V.double().numpy(),
                                sel.numpy(), kv)
    if gqa:
        got = selected_attention(q.to(dev), K.to(dev), V.to(dev), sel.to(dev), gqa=True)
    else:
        got = ref_api(q.to(dev), K.to(dev), V.to(dev), sel.to(dev))
    assert got.dtype == dt and tuple(got.shape) == (Hq, D)
    tol = {torch.float32: 1e-5, torch.float16: 1e-3, torch.bfloat16: 8e-3}[dt]
    g = got.double().cpu().numpy()
    for h in range(Hq):
        assert np.linalg.norm(g[h] - want[h]) <= tol * np.linalg.norm(want[h]), h


def _stats(k, T, H):
    """Page min/max of the fp16 K over valid tokens (a partial last page is
    padded with its last token, so padding changes nothing)."""
    P = -(-T // PS)
    pad = np.repeat(k[-1:], P * PS - T, axis=0)
    return O.page_stats(np.concatenate([k, pad]).reshape(P, PS, H, 128))


@pytest.mark.parametrize("gqa,select", [("mean", "union"), ("mean", "per_head"),
                                        ("sum", "union"), ("sum", "per_head")])
def test_decode_step_vs_oracle(dev, gqa, select):
    """decode_step (src/kvquant/compact_backend.py:194-299 without host reads):
    the selection restated by the oracle (mean-q per KV head, or the
    group-summed bound; top-K with the first pages as sinks; union over KV
    heads, src/kvquant/quest_selector.py:80) and the attention over the
    selected pages with the partial last page masked."""
    from helix_kv.ops import decode_step

    T, H, group, top_k, sinks = 3000, 4, 7, 40, 4   # 188 pages, the last one 8 tokens
    kc, kt, kd, vc, vt, vd = _problem(dev, T, H, 16, 4, 2048)
    P = kd.shape[0]
    k16 = kd.reshape(-1, H, 128)[:T].astype(np.float16)
    kmin, kmax = _stats(k16, T, H)
    q = RNG.standard_normal((H * group, 128)).astype(np.float16)
    qd = _t(q, dev)
    if gqa == "mean":
        # the reference's own torch op (fp16 mean), evaluated where the step runs
        qs = qd.reshape(H, group, 128).mean(dim=1).to(torch.float16).cpu().numpy()
        bound = O.page_bound(qs, kmin, kmax)
    else:
        bound = O.page_bound_group(q, kmin, kmax, group)
    sel = O.topk_sinks(bound, min(top_k, P - sinks), sinks)
    if select == "union":
        ids = np.unique(sel.reshape(-1))
        assert sinks + top_k < ids.size < P
        sel = np.repeat(ids[:, None], H, axis=1)
    want = O.selected_attention(q.astype(np.float64), kd, vd, sel, lambda h: h // group,
                                num_tokens=T)
    got = decode_step(qd, kc, kt, vc, vt, _t(kmin, dev), _t(kmax, dev), top_k, sinks, gqa=gqa,
                      select=select, out_dtype=torch.float32)
    _check(got, want)


@pytest.mark.parametrize("gqa,select", [("mean", "union"), ("sum", "per_head")])
def test_decode_step_u8_metadata_vs_oracle(dev, gqa, select):
    """decode_step over the compact u8 page metadata: the selection is the
    oracle's top-K over the bound of the dequantised u8 statistics (every
    bound at least the fp16 one), the attention as in the fp16 case."""
    from helix_kv.ops import decode_step, quest_page_stats_u8

    T, H, group, top_k, sinks = 3000, 4, 7, 40, 4
    kc, kt, kd, vc, vt, vd = _problem(dev, T, H, 16, 4, 2048)
    P = kd.shape[0]
    k16 = kd.reshape(-1, H, 128)[:T].astype(np.float16)
    kmin, kmax = _stats(k16, T, H)
    qmin, qmax, lo, st = O.page_stats_u8(kmin, kmax)
    dmn, dmx = O.page_stats_u8_deq(qmin, qmax, lo, st)
    q = RNG.standard_normal((H * group, 128)).astype(np.float16)
    qd = _t(q, dev)
    if gqa == "mean":
        qs = qd.reshape(H, group, 128).mean(dim=1).to(torch.float16).cpu().numpy()
        bound = O.page_bound(qs, dmn, dmx)
    else:
        bound = O.page_bound_group(q, dmn, dmx, group)
    sel = O.topk_sinks(bound, min(top_k, P - sinks), sinks)
    if select == "union":
        ids = np.unique(sel.reshape(-1))
        sel = np.repeat(ids[:, None], H, axis=1)
    want = O.selected_attention(q.astype(np.float64), kd, vd, sel, lambda h: h // group,
                                num_tokens=T)
    u8 = quest_page_stats_u8(_t(kmin, dev), _t(kmax, dev))
    got = decode_step(qd, kc, kt, vc, vt, None, None, top_k, sinks, gqa=gqa, select=select,
                      out_dtype=torch.float32, stats_u8=u8)
    _check(got, want)


def test_decode_step_graph_replay(dev):
    """The step reads nothing back to the host, so it records into a HIP graph;
    three replays, with eager steps between them, equal the eager result."""
    from helix_kv.ops import decode_step

    T, H, group = 2500, 4, 7
    kc, kt, kd, vc, vt, vd = _problem(dev, T, H, 4, 16, 1024)
    k16 = kd.reshape(-1, H, 128)[:T].astype(np.float16)
    kmin, kmax = (_t(a, dev) for a in _stats(k16, T, H))
    q = _t(RNG.standard_normal((H * group, 128)).astype(np.float16), dev)
    eager = decode_step(q, kc, kt, vc, vt, kmin, kmax, 30, 4).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        decode_step(q, kc, kt, vc, vt, kmin, kmax, 30, 4)
    torch.cuda.current_stream().wait_stream(side)
    out = torch.empty_like(eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        decode_step(q, kc, kt, vc, vt, kmin, kmax, 30, 4, out=out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        other = decode_step(q, kc, kt, vc, vt, kmin, kmax, 30, 4, select="per_head")
        torch.cuda.synchronize()
        assert not torch.equal(other, eager)


def test_graph_survives_workspace_growth(dev):
    """A graph captured while the step's workspaces were small keeps working
    after an eager step on the same stream has grown them: the superseded
    buffers stay allocated, so replays write only where they did at capture
    (tensors allocated afterwards are untouched) and equal the eager result."""
    from helix_kv.ops import decode_step

    H, group = 4, 7
    small = _problem(dev, 700, H, 16, 4, 1024)
    large = _problem(dev, 9000, H, 16, 4, 1024)

    def stats(prob):
        kd = prob[2]
        T = kd.shape[0] * PS
        return tuple(_t(a, dev) for a in _stats(kd.reshape(-1, H, 128)[:T].astype(np.float16), T, H))

    st_small, st_large = stats(small), stats(large)   # uploaded before the capture

    def step(prob, st, q, **kw):
        kc, kt, kd, vc, vt, vd = prob
        return decode_step(q, kc, kt, vc, vt, st[0], st[1], kd.shape[0] // 3, 4, **kw)

    q = _t(RNG.standard_normal((H * group, 128)).astype(np.float16), dev)
    side = torch.cuda.Stream()   # workspaces are per stream: this one starts empty
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        eager = step(small, st_small, q).clone()
        torch.cuda.synchronize()
        out = torch.empty_like(eager)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            step(small, st_small, q, out=out)
        step(large, st_large, q)      # grows the workspaces of this stream
        torch.cuda.synchronize()
    fillers = [torch.full((1 << 18,), 7, dtype=torch.int32, device=dev) for _ in range(64)]
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    assert all(bool((f == 7).all()) for f in fillers)


@pytest.mark.parametrize("select,gqa", [("union", "mean"), ("per_head", "sum"), ("per_head", "mean"),
                                        ("union", "sum")])
def test_decode_step_batch_vs_oracle(dev, select, gqa):
    """Three sequences in one compact tensor (page-aligned starts, V packed with
    positions from each sequence's start): decode_step_batch (one ragged
    selection, the per-sequence union, one batched decode) equals the oracle
    pipeline per sequence; union and mean-q are the reference forward's."""
    from helix_kv.ops import NuqLayerTables, decode_step_batch, nuq_pack_compact

    H, group, D, top_k, sinks = 4, 7, 128, 12, 4
    lens = [1000, 2500, 333]
    starts = [0]
    for n in lens[:-1]:
        starts.append(starts[-1] + -(-n // PS) * PS)
    T = starts[-1] + -(-lens[-1] // PS) * PS
    pos = np.zeros(T, np.int64)
    for s0, n in zip(starts, lens):
        pos[s0:s0 + -(-n // PS) * PS] = np.arange(-(-n // PS) * PS)
    k = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
    v = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
    kp, ku, kl = _scales(H, D, 16, 1.2)
    vp, vu, vl = _scales(H, 1024, 4, 1.2)
    kt = NuqLayerTables(_t(kp, dev), _t(ku, dev), _t(kl, dev), per_token=False)
    vt = NuqLayerTables(_t(vp, dev), _t(vu, dev), _t(vl, dev), per_token=True)
    kc = nuq_pack_compact(_t(k, dev), kt, 4)
    vc = nuq_pack_compact(_t(v, dev), vt, 2, positions=torch.from_numpy(pos))

    def deq(cc, poles, bits, kind, positions=None):
        codes = O.bitunpack(cc.packed.cpu().numpy(), bits, D)
        m, val = O.csr_decode(cc.row_ptr.cpu().numpy(), cc.col.cpu().numpy(),
                              cc.val.cpu().numpy().view(np.uint16), T * H, D)
        return O.h2f(O.unpack(codes, val.reshape(T, H, D), m.reshape(T, H, D),
                              poles.astype(np.float32), kind, positions=positions))

    kd = deq(kc, kp, 4, "k")
    vd = deq(vc, vp, 2, "v", positions=pos)
    stats = [_stats(k[s0:s0 + n], n, H) for s0, n in zip(starts, lens)]
    kmin = np.concatenate([s[0] for s in stats])
    kmax = np.concatenate([s[1] for s in stats])
    assert kmin.shape[0] == T // PS
    q = RNG.standard_normal((len(lens), H * group, D)).astype(np.float16)
    qd = _t(q, dev)
    got = decode_step_batch(qd, kc, kt, vc, vt, _t(kmin, dev), _t(kmax, dev), starts, lens,
                            top_k, sinks, gqa=gqa, select=select, out_dtype=torch.float32)
    for b, (s0, n) in enumerate(zip(starts, lens)):
        P = -(-n // PS)
        pad = P * PS - n
        kb = np.concatenate([kd[s0:s0 + n], np.zeros((pad, H, D))]).reshape(P, PS, H, D)
        vb = np.concatenate([vd[s0:s0 + n], np.zeros((pad, H, D))]).reshape(P, PS, H, D)
        if gqa == "mean":
            qs = qd[b].reshape(H, group, D).mean(dim=1).to(torch.float16).cpu().numpy()
            bound = O.page_bound(qs, stats[b][0], stats[b][1])
        else:
            bound = O.page_bound_group(q[b], stats[b][0].astype(np.float32),
                                       stats[b][1].astype(np.float32), group)
        sel = O.topk_sinks(bound, min(top_k, P - sinks), sinks)
        if select == "union":
            ids = np.unique(sel.reshape(-1))
            sel = np.repeat(ids[:, None], H, axis=1)
        want = O.selected_attention(q[b].astype(np.float64), kb, vb, sel, lambda h: h // group,
                                    num_tokens=n)
        _check(got[b], want)


def test_union_pages_vs_numpy_on_a_reused_workspace(dev):
    """The union of the heads' pages (hkv_union_pages_ragged) against numpy,
    over calls of growing and shrinking page counts on one workspace: each
    call must leave the flags zero for the next, whatever its size."""
    from helix_kv.ops import union_pages

    for P, n, H in [(5000, 1250, 4), (300, 80, 2), (70000, 17500, 4), (100, 100, 4), (70000, 20, 1),
                    (40, 10, 4), (2048, 600, 3), (2049, 600, 3)]:
        sel = np.stack([RNG.choice(P, n, replace=False) for _ in range(H)], axis=1).astype(np.int64)
        got = union_pages(_t(sel, dev), P).cpu().numpy()
        u = np.unique(sel)
        want = np.full((P, H), -1, np.int64)
        want[: len(u)] = u[:, None]
        assert np.array_equal(got, want), (P, n, H)


@pytest.mark.parametrize("layout", ["back_to_back", "gapped", "many"])
def test_decode_step_batch_equals_single_steps(dev, layout):
    """The batched step (one ragged selection, one union, one decode launch;
    the gapped layout takes the per-sequence path; 70 sequences run as
    batches of 64 and 6) equals decode_step on each sequence's view with the
    same pages_per_split, bit for bit, in both select modes; and a HIP graph
    of the batched step replays it exactly."""
    from helix_kv.ops import (NuqLayerTables, compact_view, decode_step, decode_step_batch,
                              nuq_pack_compact)

    H, group, D, top_k, sinks, pps = 4, 7, 128, 20, 4, 8
    lens = [700, 1601, 40, 2100, 16]
    if layout == "many":
        lens = [int(n) for n in np.random.default_rng(70).integers(1, 300, 70)]
    gap = 32 if layout == "gapped" else 0
    starts = [0]
    for n in lens[:-1]:
        starts.append(starts[-1] + -(-n // PS) * PS + gap)
    T = starts[-1] + -(-lens[-1] // PS) * PS
    pos = np.zeros(T, np.int64)
    for s0, n in zip(starts, lens):
        pos[s0:s0 + -(-n // PS) * PS] = np.arange(-(-n // PS) * PS)
    k = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
    v = (RNG.standard_t(3, (T, H, D)) * 0.7).astype(np.float16)
    kp, ku, kl = _scales(H, D, 4, 1.2)
    vp, vu, vl = _scales(H, 1024, 16, 1.2)
    kt = NuqLayerTables(_t(kp, dev), _t(ku, dev), _t(kl, dev), per_token=False)
    vt = NuqLayerTables(_t(vp, dev), _t(vu, dev), _t(vl, dev), per_token=True)
    kc = nuq_pack_compact(_t(k, dev), kt, 2)
    vc = nuq_pack_compact(_t(v, dev), vt, 4, positions=torch.from_numpy(pos))
    kmin, kmax = _stats(k, T, H)
    kmin_d, kmax_d = _t(kmin, dev), _t(kmax, dev)
    qd = _t(RNG.standard_normal((len(lens), H * group, D)).astype(np.float16), dev)
    for select in ("union", "per_head"):
        got = decode_step_batch(qd, kc, kt, vc, vt, kmin_d, kmax_d, starts, lens, top_k, sinks,
                                select=select, pages_per_split=pps)
        for b, (t0, n) in enumerate(zip(starts, lens)):
            p0, p1 = t0 // PS, (t0 + n + PS - 1) // PS
            one = decode_step(qd[b], compact_view(kc, t0, t0 + n), kt, compact_view(vc, t0, t0 + n), vt,
                              kmin_d[p0:p1], kmax_d[p0:p1], top_k, sinks, select=select,
                              pages_per_split=pps)
            assert torch.equal(got[b].view(torch.int16), one.view(torch.int16)), (layout, select, b)
    if layout != "back_to_back":
        return
    out = torch.empty_like(got)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        decode_step_batch(qd, kc, kt, vc, vt, kmin_d, kmax_d, starts, lens, top_k, sinks,
                          pages_per_split=pps, out=out)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            decode_step_batch(qd, kc, kt, vc, vt, kmin_d, kmax_d, starts, lens, top_k, sinks,
                              pages_per_split=pps, out=out)
    torch.cuda.synchronize()
    want = decode_step_batch(qd, kc, kt, vc, vt, kmin_d, kmax_d, starts, lens, top_k, sinks,
                             pages_per_split=pps)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16))
