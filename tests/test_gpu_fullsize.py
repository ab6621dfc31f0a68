"""GPU parity at the benchmark's own sizes, against the oracle.

- The ragged Quest + gather workload exactly as the benchmark builds it
  (8 sequences, numpy default_rng(4), 102,832 pages): the selection bit-exact
  against the oracle's per-sequence bound + top-K, and every gathered
  (row, head) page of K and V bit-exact against the oracle's dequantisation
  of the same compact bytes.
- One decode layer at 1,048,576 tokens (65,536 pages per head), nuq2 and
  nuq4, as the decode benchmark builds it: the group-summed per-head
  selection bit-exact against the oracle; the fused decode attention over it
  (pages_per_split 88) and the reference-semantics step (mean query per KV
  head, union of the heads' pages) against the oracle's float64 attention
  over pages the oracle decodes from the compact bytes.  Tolerance: per head,
  relative L2 error and max-abs error over max |ref| both <= 1e-3.

The inputs are generated on the GPU by the benchmark's builders (seeded); the
expected results are computed on the CPU by the oracle only.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3
PS = 16


def _host_compact(cc):
    return (cc.packed.cpu().numpy(), cc.row_ptr.cpu().numpy().astype(np.int64),
            cc.col.cpu().numpy(), cc.val.cpu().numpy().view(np.uint16))


def _decode_rows(host, tokens, h, H, D, bits, poles, kind, positions=None):
    """Oracle dequantisation of rows (token, h) of a compact tensor:
    bit-unpacked codes, the rows' CSR entries, then the oracle's unpack with
    head h's scales.  Returns fp16 bits (n, D)."""
    packed, rp, col, val = host
    n = tokens.size
    codes = O.bitunpack(packed[tokens, h], bits, D)
    r = tokens * H + h
    cnt = rp[r + 1] - rp[r]
    tot = int(cnt.sum())
    m = np.zeros((n, D), np.uint8)
    v = np.zeros((n, D), np.uint16)
    if tot:
        row = np.repeat(np.arange(n), cnt)
        first = np.repeat(rp[r] - np.concatenate([[0], np.cumsum(cnt)[:-1]]), cnt)
        e = first + np.arange(tot)
        m[row, col[e].astype(np.int64)] = 1
        v[row, col[e].astype(np.int64)] = val[e]
    out = O.unpack(codes[:, None, :], v[:, None, :], m[:, None, :], poles[h:h + 1], kind,
                   positions=positions)
    return out[:, 0, :]


def _check(got, want):
    got = np.asarray(got, np.float64)
    for h in range(want.shape[0]):
        ref = want[h]
        err = got[h] - ref
        assert np.linalg.norm(err) <= TOL * np.linalg.norm(ref), h
        assert np.abs(err).max() <= TOL * np.abs(ref).max(), h


def test_ragged_workload_full_size(dev):
    import bench
    from helix_kv.ops import nuq_gather_pages, quest_select_ragged

    W = bench.build_ragged(dev)
    H, D = bench.H, bench.D
    offs, ks = W["offs"], W["ks"]
    assert W["Ptot"] == 102832
    sel, outs, scores = quest_select_ragged(W["q"], W["kmin"], W["kmax"], offs, ks, 4)
    gk = nuq_gather_pages(W["ck"], W["kt"], sel, offs, outs)
    gv = nuq_gather_pages(W["cv"], W["vt"], sel, offs, outs)
    torch.cuda.synchronize()
    wsel, wouts, wscores = O.select_ragged(W["q"].float().cpu().numpy(),
                                           W["kmin"].float().cpu().numpy(),
                                           W["kmax"].float().cpu().numpy(), offs, ks, 4)
    assert outs == wouts.tolist() and outs[-1] == 25737
    assert np.array_equal(scores.cpu().numpy(), wscores)
    sel_h = sel.cpu().numpy()
    assert np.array_equal(sel_h, wsel)
    rows = outs[-1]
    seq = np.searchsorted(np.asarray(outs), np.arange(rows), side="right") - 1
    kpoles = W["kt"].poles.float().cpu().numpy()
    vpoles = W["vt"].poles.float().cpu().numpy()
    hk, hv = _host_compact(W["ck"]), _host_compact(W["cv"])
    gk_h = gk.cpu().view(torch.int16).numpy().view(np.uint16)
    gv_h = gv.cpu().view(torch.int16).numpy().view(np.uint16)
    for h in range(H):
        lp = sel_h[:rows, h]
        tok = ((offs[seq] + lp)[:, None] * PS + np.arange(PS)[None, :]).reshape(-1)
        pos = (lp[:, None] * PS + np.arange(PS)[None, :]).reshape(-1)
        wk = _decode_rows(hk, tok, h, H, D, 4, kpoles, "k")
        wv = _decode_rows(hv, tok, h, H, D, 4, vpoles, "v", positions=pos)
        assert np.array_equal(gk_h[:rows, :, h].reshape(-1, D), wk), h
        assert np.array_equal(gv_h[:rows, :, h].reshape(-1, D), wv), h


@pytest.mark.parametrize("layer", [0, 27])   # nuq2, nuq4
def test_decode_layer_1m_tokens(dev, layer):
    import bench
    from helix_kv.ops import decode_attention, decode_step, quest_select

    (Ld,) = bench.build_decode_layers(dev, [layer])
    H, D, HQ = bench.H, bench.D, bench.HQ
    grp = HQ // H
    P = bench.DEC_TOK // PS
    assert Ld["bits"] == (2 if layer < bench.CUT else 4)
    k, s = P // 4, 4
    q = Ld["q"]
    sel, _ = quest_select(q, Ld["kmin"], Ld["kmax"], k, s)
    out = decode_attention(q, Ld["ck"], Ld["kt"], Ld["cv"], Ld["vt"], sel, pages_per_split=88,
                           out_dtype=torch.float32)
    out_u = decode_step(q, Ld["ck"], Ld["kt"], Ld["cv"], Ld["vt"], Ld["kmin"], Ld["kmax"], k, s,
                        gqa="mean", select="union", pages_per_split=88,
                        out_dtype=torch.float32)
    qm = q.reshape(H, grp, D).mean(dim=1).to(torch.float16).cpu().numpy()  # the reference's op
    torch.cuda.synchronize()
    kmin, kmax = Ld["kmin"].cpu().numpy(), Ld["kmax"].cpu().numpy()
    qh = q.cpu().numpy()
    wsel = O.topk_sinks(O.page_bound_group(qh, kmin, kmax, grp), k, s)
    assert np.array_equal(sel.cpu().numpy(), wsel)
    usel = O.topk_sinks(O.page_bound(qm, kmin, kmax), k, s)
    union = np.unique(usel.reshape(-1))
    assert k + s < union.size < P

    bits = Ld["bits"]
    kpoles = Ld["kt"].poles.float().cpu().numpy()
    vpoles = Ld["vt"].poles.float().cpu().numpy()
    hk, hv = _host_compact(Ld["ck"]), _host_compact(Ld["cv"])
    q64 = qh.astype(np.float64)
    want = np.zeros((HQ, D))
    want_u = np.zeros((HQ, D))
    for g in range(H):
        for pages, dst in ((wsel[:, g], want), (union, want_u)):
            tok = (pages[:, None] * PS + np.arange(PS)[None, :]).reshape(-1)
            kd = O.h2f(_decode_rows(hk, tok, g, H, D, bits, kpoles, "k"))
            vd = O.h2f(_decode_rows(hv, tok, g, H, D, bits, vpoles, "v", positions=tok))
            n = pages.size
            kp = kd.reshape(n, PS, 1, D)
            vp = vd.reshape(n, PS, 1, D)
            ids = np.arange(n, dtype=np.int64)[:, None]
            dst[g * grp:(g + 1) * grp] = O.selected_attention(q64[g * grp:(g + 1) * grp], kp, vp,
                                                              ids, lambda h: 0)
    _check(out.cpu().numpy(), want)
    _check(out_u.cpu().numpy(), want_u)
