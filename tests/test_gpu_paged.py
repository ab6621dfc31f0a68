"""GPU parity of the paged compact pool (hkv_paged_write / hkv_paged_gather)
against the oracle's restatement (oracle.paged_write / paged_gather), bit-exact:
codes, per-page outlier counts and entries, K page statistics, status; and the
append property: a prefill followed by single-token appends leaves the pool
exactly as one write of all the tokens does."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(1601)
H, D, PS = 4, 128, 16


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _scales(per_token, L, rows=None, thr=1.6, dtype=np.float16):
    n = rows if per_token else D
    poles = np.sort(RNG.standard_normal((H, n, L)), axis=-1).astype(dtype)
    up = RNG.uniform(thr * 0.8, thr * 1.2, (H, n)).astype(dtype)
    return poles, up, (-up).astype(dtype)


def _tables(dev, sc, per_token):
    from helix_kv.ops import NuqLayerTables

    return NuqLayerTables(_t(sc[0], dev), _t(sc[1], dev), _t(sc[2], dev), per_token=per_token)


def _diff(a, b) -> int:
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    return int((a != b).sum())


def logical_entries(side) -> np.ndarray:
    """Every page-head's stored entries in order, (NB, H, 2048) u32: the
    first cap inline, the rest from the page-head's overflow chunk."""
    NB, Hh, cap = side.num_blocks, side.heads, side.cap
    full = np.zeros((NB, Hh, PS * D), np.uint32)
    full[:, :, :cap] = side.oent.cpu().numpy().view(np.uint32)
    if side.ovf is not None:
        idx = side.ovf.cpu().numpy()
        m = idx >= 0
        full[m, cap:] = side.ovf_ent.cpu().numpy().view(np.uint32)[idx[m]]
    return full


def _check(side, want, cap):
    assert _diff(side.codes.cpu().numpy(), want["codes"]) == 0
    cnt = side.ocnt.cpu().numpy()
    assert _diff(cnt, want["ocnt"]) == 0
    room = want["room"]
    ent = logical_entries(side)[:, :, :room]
    live = np.arange(room)[None, None, :] < np.minimum(cnt, room)[..., None]
    assert _diff(np.where(live, ent, 0), np.where(live, want["oent"], 0)) == 0
    if "kmin" in want:
        assert _diff(side.kmin.cpu().view(torch.int16).numpy().view(np.uint16), want["kmin"]) == 0
        assert _diff(side.kmax.cpu().view(torch.int16).numpy().view(np.uint16), want["kmax"]) == 0
    assert int(side.status.item()) == want["status"]


def _slot_mapping(T, NB, kind):
    if kind == "aligned":      # whole pages, scattered over the pool
        pages = RNG.permutation(NB)[: -(-T // PS)]
        return (pages[:, None] * PS + np.arange(PS)[None, :]).reshape(-1)[:T]
    if kind == "offset":       # a sequence continuing mid-page over scattered pages, then
        pages = RNG.permutation(NB)[: -(-(T + 5) // PS)]     # padding tokens (slot -1)
        s = (pages[:, None] * PS + np.arange(PS)[None, :]).reshape(-1)[5:5 + T].copy()
        s[T - T // 20:] = -1
        return s
    if kind == "batch":        # one token per sequence: each its own page and row
        pages = RNG.permutation(NB)[:T]
        return pages * PS + RNG.integers(0, PS, T)
    raise ValueError(kind)


@pytest.mark.parametrize("per_token,L,kind,T,cap,arena", [
    (False, 16, "aligned", 1024, 256, True), (False, 4, "offset", 777, 256, True),
    (True, 16, "offset", 500, 256, True), (True, 4, "aligned", 1024, 256, True),
    (False, 16, "batch", 40, 256, True), (True, 16, "batch", 40, 64, True),
    (False, 4, "aligned", 256, 8, True),    # every page-head past cap: entries in overflow chunks
    (True, 16, "offset", 700, 40, True),    # overflow with mid-page starts
    (False, 4, "aligned", 256, 8, False),   # no arena: status set, the first 8 kept
])
def test_paged_write_vs_oracle(dev, per_token, L, kind, T, cap, arena):
    from helix_kv.paged import PagedSide, paged_write

    NB, bits = 128, 2 if L <= 4 else 4
    rows = 300
    sc = _scales(per_token, L, rows)
    t = _tables(dev, sc, per_token)
    x = (RNG.standard_t(3, (T, H, D)) * 0.8).astype(np.float16)
    slots = _slot_mapping(T, NB, kind)
    pos = RNG.integers(0, 2 * rows, T) if per_token else None
    side = PagedSide.empty(NB, H, bits, cap, dev, stats=not per_token,
                           n_chunks=NB * H if arena else 0)
    paged_write(side, _t(x, dev), t, _t(slots, dev), None if pos is None else _t(pos, dev))
    want = O.paged_empty(NB, H, D, bits, cap, stats=not per_token, arena=arena)
    O.paged_write(want, x, slots, [a.astype(np.float32) for a in sc], per_token, positions=pos)
    torch.cuda.synchronize()
    _check(side, want, cap)
    if cap == 8:
        assert int(want["ocnt"].max()) > cap
        assert want["status"] == (0 if arena else 1)


@pytest.mark.parametrize("per_token,L", [(False, 16), (False, 4), (True, 16), (True, 4)])
def test_prefill_then_appends_equals_one_write(dev, per_token, L):
    """A sequence written as a prefill of T0 tokens then one token per call
    (decode appends) leaves codes, outlier lists and statistics exactly as a
    single write of all its tokens; the block table scatters its pages."""
    from helix_kv.paged import PagedSide, paged_write

    NB, bits, cap = 64, 2 if L <= 4 else 4, 256
    T0, N = 203, 45
    T = T0 + N
    sc = _scales(per_token, L, rows=512)
    t = _tables(dev, sc, per_token)
    x = (RNG.standard_t(3, (T, H, D)) * 0.8).astype(np.float16)
    table = RNG.permutation(NB)[: -(-T // PS)]
    slots = table[np.arange(T) // PS] * PS + np.arange(T) % PS
    pos = np.arange(T)
    one = PagedSide.empty(NB, H, bits, cap, dev, stats=not per_token, n_chunks=NB * H)
    inc = PagedSide.empty(NB, H, bits, cap, dev, stats=not per_token, n_chunks=NB * H)
    xd, sd, pd = _t(x, dev), _t(slots, dev), _t(pos, dev)
    paged_write(one, xd, t, sd, pd if per_token else None)
    paged_write(inc, xd[:T0].contiguous(), t, sd[:T0], pd[:T0] if per_token else None)
    for i in range(T0, T):
        paged_write(inc, xd[i:i + 1].contiguous(), t, sd[i:i + 1], pd[i:i + 1] if per_token else None)
    torch.cuda.synchronize()
    assert torch.equal(one.codes, inc.codes)
    assert torch.equal(one.ocnt, inc.ocnt)
    m = torch.minimum(one.ocnt, torch.tensor(cap, device=dev))
    live = torch.arange(cap, device=dev)[None, None, :] < m[..., None]
    assert torch.equal(torch.where(live, one.oent, 0), torch.where(live, inc.oent, 0))
    if not per_token:
        assert torch.equal(one.kmin.view(torch.int16), inc.kmin.view(torch.int16))
        assert torch.equal(one.kmax.view(torch.int16), inc.kmax.view(torch.int16))
    want = O.paged_empty(NB, H, D, bits, cap, stats=not per_token)
    O.paged_write(want, x, slots, [a.astype(np.float32) for a in sc], per_token, positions=pos)
    _check(inc, want, cap)


def test_rewrite_truncates_the_page(dev):
    """Rewriting rows 5.. of a full page (a rollback) keeps the outliers of
    rows 0-4, replaces the rest, and folds the statistics."""
    from helix_kv.paged import PagedSide, paged_write

    NB, bits, cap = 8, 4, 256
    sc = _scales(False, 16)
    t = _tables(dev, sc, False)
    a = (RNG.standard_t(3, (16, H, D)) * 0.8).astype(np.float16)
    b = (RNG.standard_t(3, (7, H, D)) * 0.8).astype(np.float16)
    s_a = 3 * PS + np.arange(16)
    s_b = 3 * PS + 5 + np.arange(7)
    side = PagedSide.empty(NB, H, bits, cap, dev, stats=True)
    paged_write(side, _t(a, dev), t, _t(s_a, dev))
    paged_write(side, _t(b, dev), t, _t(s_b, dev))
    want = O.paged_empty(NB, H, D, bits, cap, stats=True)
    f32 = [x.astype(np.float32) for x in sc]
    O.paged_write(want, a, s_a, f32, False)
    O.paged_write(want, b, s_b, f32, False)
    torch.cuda.synchronize()
    _check(side, want, cap)
    ent = want["oent"][3, 0, : want["ocnt"][3, 0]]
    assert (ent >> 24).min() < 5 and (ent >> 24).max() >= 5


@pytest.mark.parametrize("per_token,L", [(False, 16), (True, 4)])
def test_paged_gather_vs_oracle(dev, per_token, L):
    from helix_kv.paged import PagedSide, paged_gather, paged_write

    NB, bits, cap, T = 96, 2 if L <= 4 else 4, 256, 1200
    sc = _scales(per_token, L, rows=700)
    t = _tables(dev, sc, per_token)
    x = (RNG.standard_t(3, (T, H, D)) * 0.8).astype(np.float16)
    slots = _slot_mapping(T, NB, "offset")
    pos = np.arange(T)
    side = PagedSide.empty(NB, H, bits, cap, dev, stats=False, n_chunks=NB * H)
    paged_write(side, _t(x, dev), t, _t(slots, dev), _t(pos, dev) if per_token else None)
    want = O.paged_empty(NB, H, D, bits, cap, stats=False)
    O.paged_write(want, x, slots, [a.astype(np.float32) for a in sc], per_token,
                  positions=pos if per_token else None)
    ids = np.concatenate([RNG.permutation(NB)[:50], [-1, NB, NB + 7]]).astype(np.int64)
    first = RNG.integers(0, 900, ids.size).astype(np.int64)
    got = paged_gather(side, t, _t(ids, dev), _t(first, dev))
    torch.cuda.synchronize()
    exp = O.paged_gather(want, ids, first, sc[0].astype(np.float32), per_token)
    assert _diff(got.cpu().view(torch.int16).numpy().view(np.uint16), exp) == 0


def test_paged_write_full_layer(dev):
    """A 131,072-token prefill of one K layer (nuq4, heavy tails: about 5%
    outliers) into scattered pages, every byte against the oracle."""
    from helix_kv.paged import PagedSide, paged_write

    T, NB, cap = 131072, 8192 + 64, 256
    sc = _scales(False, 16, thr=2.2)
    t = _tables(dev, sc, False)
    x = RNG.standard_t(3, (T, H, D)).astype(np.float16)
    slots = _slot_mapping(T, NB, "aligned")
    want = O.paged_empty(NB, H, D, 4, cap, stats=True)
    O.paged_write(want, x, slots, [a.astype(np.float32) for a in sc], False)
    over = int((want["ocnt"] > cap).sum())     # arena sized as a caller would: one chunk per
    side = PagedSide.empty(NB, H, 4, cap, dev, stats=True, n_chunks=over)   # overflowing page-head
    paged_write(side, _t(x, dev), t, _t(slots, dev))
    torch.cuda.synchronize()
    assert 0.02 < want["ocnt"].sum() / x.size < 0.2
    assert over > 0 and int(side.ovf_next.item()) == over
    _check(side, want, cap)


def test_paged_write_arena_used_up(dev):
    """With fewer overflow chunks than overflowing page-heads, the chunks go
    to some of them (first come, first served), every page-head keeps its
    counts and first cap entries, those with a chunk keep all of theirs, and
    status flags the loss."""
    from helix_kv.paged import PagedSide, paged_write

    NB, bits, cap, T, chunks = 64, 4, 64, 1024, 10
    sc = _scales(False, 16)
    t = _tables(dev, sc, False)
    x = (RNG.standard_t(3, (T, H, D)) * 0.8).astype(np.float16)
    slots = _slot_mapping(T, NB, "aligned")
    side = PagedSide.empty(NB, H, bits, cap, dev, stats=True, n_chunks=chunks)
    paged_write(side, _t(x, dev), t, _t(slots, dev))
    want = O.paged_empty(NB, H, D, bits, cap, stats=True)
    O.paged_write(want, x, slots, [a.astype(np.float32) for a in sc], False)
    torch.cuda.synchronize()
    assert int((want["ocnt"] > cap).sum()) > chunks
    assert _diff(side.codes.cpu().numpy(), want["codes"]) == 0
    cnt = side.ocnt.cpu().numpy()
    assert _diff(cnt, want["ocnt"]) == 0
    ovf = side.ovf.cpu().numpy()
    owned = ovf >= 0
    assert owned.sum() == chunks and np.array_equal(np.sort(ovf[owned]), np.arange(chunks))
    ent, ref = logical_entries(side), want["oent"]
    live = np.arange(PS * D)[None, None, :] < np.where(owned, cnt, np.minimum(cnt, cap))[..., None]
    assert _diff(np.where(live, ent, 0), np.where(live, ref, 0)) == 0
    assert _diff(side.kmin.cpu().view(torch.int16).numpy().view(np.uint16), want["kmin"]) == 0
    assert int(side.status.item()) == 1
