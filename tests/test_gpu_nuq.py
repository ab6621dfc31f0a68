"""GPU parity of the nuq kernels against the CPU oracle (bit-exact).

Covers: decision tables, the dense (reference byte-format) pack/unpack for K
and V in the per-head and batched APIs, the compact (bit-packed + CSR)
pack/unpack, the broadcasting spec functions, and the reference's own
known-answer and batched==per-head tests.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(99)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _kscales(H, D, L, dtype=np.float16, scale=1.0, thr=1.5):
    poles = (np.sort(RNG.standard_normal((H, D, L)), axis=-1) * scale).astype(dtype)
    up = np.full((H, D), thr * scale, dtype)
    return poles, up, (-up).astype(dtype)


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# ------------------------------------------------------------------ tables

def test_tables_bit_exact_vs_oracle(dev):
    from helix_kv.ops import build_tables

    tabs = []
    for i in range(300):
        L = [4, 16, 3, 8, 1][i % 5]
        p = np.sort(RNG.standard_normal(L) * 10.0 ** RNG.uniform(-3, 3))
        tabs.append(np.pad(p, (0, 16 - L), constant_values=np.nan)[:16])
    for L in (4, 16):
        poles = np.stack([t[:L] for t in tabs if not np.isnan(t[:L]).any()]).astype(np.float32)
        poles = np.concatenate([poles, np.array([[3, 2, 1, 0] * (L // 4)], np.float32),
                                np.zeros((1, L), np.float32)])
        n = poles.shape[0]
        up = RNG.uniform(-1, 3, n).astype(np.float32)
        lo = -RNG.uniform(-1, 3, n).astype(np.float32)
        up[:3] = [np.inf, 0.0, np.nan]
        lo[:3] = [-np.inf, 0.0, np.nan]
        for pd in (np.float32, np.float16):
            p16 = poles.astype(pd)
            want = O.prep_tables(p16.astype(np.float32), up.astype(pd).astype(np.float32),
                                 lo.astype(pd).astype(np.float32))
            got = build_tables(_t(p16, dev), _t(up.astype(pd), dev), _t(lo.astype(pd), dev))
            assert np.array_equal(got.cpu().numpy().view(O.TABLE_DTYPE).reshape(-1), want)


# ------------------------------------------------------------ dense format

@pytest.mark.parametrize("T,H,D,L", [(128, 4, 128, 16), (130, 4, 128, 4), (64, 2, 32, 16),
                                     (10, 1, 8, 4), (33, 3, 24, 16), (7, 2, 256, 8)])
def test_pack_dense_keys_vs_oracle(dev, T, H, D, L):
    from kvquant.triton_batched import pack_keys_per_channel_batched, unpack_keys_per_channel_batched

    x = RNG.standard_normal((T, H, D)).astype(np.float16)
    poles, up, lo = _kscales(H, D, L)
    c, v, m = pack_keys_per_channel_batched(_t(x, dev), _t(poles, dev), _t(up, dev), _t(lo, dev))
    wc, wv, wm = O.pack_k(x, poles.astype(np.float32), up.astype(np.float32), lo.astype(np.float32))
    assert np.array_equal(c.cpu().numpy(), wc)
    assert np.array_equal(_bits(v), wv)
    assert np.array_equal(m.cpu().numpy(), wm)
    out = unpack_keys_per_channel_batched(c, v, m, _t(poles, dev))
    assert np.array_equal(_bits(out), O.unpack(wc, wv, wm, poles.astype(np.float32), "k"))


@pytest.mark.parametrize("T,H,D,L", [(128, 4, 128, 16), (100, 4, 128, 4), (9, 2, 16, 3)])
def test_pack_dense_values_vs_oracle(dev, T, H, D, L):
    from kvquant.triton_batched import pack_values_per_token_batched, unpack_values_per_token_batched

    x = RNG.standard_normal((T, H, D)).astype(np.float16)
    poles = np.sort(RNG.standard_normal((H, T, L)), axis=-1).astype(np.float16)
    up = RNG.uniform(0.5, 2.0, (H, T)).astype(np.float16)
    lo = (-RNG.uniform(0.5, 2.0, (H, T))).astype(np.float16)
    c, v, m = pack_values_per_token_batched(_t(x, dev), _t(poles, dev), _t(up, dev), _t(lo, dev))
    wc, wv, wm = O.pack_v(x, poles.astype(np.float32), up.astype(np.float32), lo.astype(np.float32))
    assert np.array_equal(c.cpu().numpy(), wc)
    assert np.array_equal(_bits(v), wv)
    assert np.array_equal(m.cpu().numpy(), wm)
    out = unpack_values_per_token_batched(c, v, m, _t(poles, dev))
    assert np.array_equal(_bits(out), O.unpack(wc, wv, wm, poles.astype(np.float32), "v"))


def test_every_fp16_input_both_paths(dev):
    """All 65,536 fp16 bit patterns against 128 tables of very different scales,
    with fp32 and fp16 scales: codes, outliers, dequant bit-exact."""
    from helix_kv.ops import NuqLayerTables, nuq_pack_dense, nuq_unpack_dense

    allx = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(512, 1, 128)
    x = allx.view(np.float16)
    D = 128
    scales = 10.0 ** np.linspace(-4, 4, D)
    poles = (np.sort(RNG.standard_normal((1, D, 16)), axis=-1) * scales[None, :, None])
    poles[0, 5] = [0, 0, 0, 1, 1, 2, 2, 2, 3, 3, 3, 3, 4, 4, 5, 6]   # duplicates
    poles[0, 6] = np.arange(16)[::-1]                                  # unsorted -> scan
    poles[0, 7, :4] = [0, 2.0 ** -24, 2.0 ** -23, 2.0 ** -22]         # gaps below criterion
    up = (1.5 * scales)[None].copy()
    lo = -up
    up[0, 8], lo[0, 8] = np.inf, -np.inf
    up[0, 9], lo[0, 9] = 0.0, 0.0
    for pd in (np.float32, np.float16):
        p, u, l_ = poles.astype(pd), up.astype(pd), lo.astype(pd)
        t = NuqLayerTables(_t(p, dev), _t(u, dev), _t(l_, dev), per_token=False)
        c, v, m = nuq_pack_dense(_t(x, dev), t)
        wc, wv, wm = O.pack_k(allx, p.astype(np.float32), u.astype(np.float32), l_.astype(np.float32))
        assert np.array_equal(c.cpu().numpy(), wc)
        assert np.array_equal(m.cpu().numpy(), wm)
        assert np.array_equal(_bits(v), wv)
        out = nuq_unpack_dense(c, v, m, t)
        assert np.array_equal(_bits(out), O.unpack(wc, wv, wm, p.astype(np.float32), "k"))


def test_every_fp16_input_per_token(dev):
    from helix_kv.ops import NuqLayerTables, nuq_pack_dense

    allx = np.arange(65536, dtype=np.uint32).astype(np.uint16).reshape(512, 1, 128)
    T = 512
    sc = 10.0 ** np.linspace(-3, 3, T)
    poles = (np.sort(RNG.standard_normal((1, T, 16)), axis=-1) * sc[None, :, None]).astype(np.float16)
    up = (1.2 * sc)[None].astype(np.float16)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(-up, dev), per_token=True)
    c, v, m = nuq_pack_dense(_t(allx.view(np.float16), dev), t)
    wc, wv, wm = O.pack_v(allx, poles.astype(np.float32), up.astype(np.float32),
                          (-up).astype(np.float32))
    assert np.array_equal(c.cpu().numpy(), wc) and np.array_equal(m.cpu().numpy(), wm)
    assert np.array_equal(_bits(v), wv)


def test_batched_equals_per_head(dev):
    # src/kvquant/tests/test_triton_batched.py:84-133 (bit-exact)
    from kvquant.triton_batched import pack_keys_per_channel_batched, pack_values_per_token_batched
    from kvquant.triton_kernels import pack_keys_per_channel, pack_values_per_token

    T, H, D, L = 128, 4, 128, 16
    g = torch.Generator(device=dev).manual_seed(0)
    vals = torch.randn(T, H, D, generator=g, device=dev, dtype=torch.float16)
    kp = torch.randn(H, D, L, generator=g, device=dev, dtype=torch.float16).sort(-1).values
    vp = torch.randn(H, T, L, generator=g, device=dev, dtype=torch.float16).sort(-1).values
    sig = vals.abs().mean()
    ku = (sig * 1.5).expand(H, D).to(torch.float16).contiguous()
    vu = (sig * 1.5).expand(H, T).to(torch.float16).contiguous()
    bk = pack_keys_per_channel_batched(vals, kp, ku, -ku)
    bv = pack_values_per_token_batched(vals, vp, vu, -vu)
    for h in range(H):
        pk = pack_keys_per_channel(vals[:, h].contiguous(), kp[h].contiguous(), ku[h], -ku[h])
        pv = pack_values_per_token(vals[:, h].contiguous(), vp[h].contiguous(), vu[h], -vu[h])
        for a, b in zip(bk, pk):
            assert torch.equal(a[:, h], b)
        for a, b in zip(bv, pv):
            assert torch.equal(a[:, h], b)


def test_reference_known_answers_on_gpu(dev):
    # src/kvquant/tests/test_triton_kernels.py:120-129 and test_nuq_roundtrip.py:65-75
    from kvquant.triton_kernels import pack_keys_per_channel, unpack_keys_per_channel

    T, D = 16, 32
    x = torch.randn(T, D, dtype=torch.float16, device=dev)
    qs = torch.tensor([0.125, 0.375, 0.625, 0.875], device=dev)
    poles = torch.quantile(x.float(), qs, dim=0).T.contiguous().half()
    up = torch.quantile(x.float(), 0.99, dim=0).half()
    lo = torch.quantile(x.float(), 0.01, dim=0).half()
    x[0, 0] = 99.0
    c, v, m = pack_keys_per_channel(x, poles, up, lo)
    assert m[0, 0].item() == 1 and v[0, 0].item() == 99.0
    assert unpack_keys_per_channel(c, v, m, poles)[0, 0].item() == 99.0
    assert c.max().item() <= 3

    vals = torch.tensor([[-5.0, -0.3, 0.0, 0.4, 7.0]], device=dev).half()  # (T=1, D=5)
    pl = torch.tensor([-0.5, 0.0, 0.5], device=dev).half().expand(5, 3).contiguous()
    c, v, m = pack_keys_per_channel(vals, pl, torch.ones(5, device=dev).half(),
                                    -torch.ones(5, device=dev).half())
    out = unpack_keys_per_channel(c, v, m, pl)
    assert out[0].tolist() == [-5.0, -0.5, 0.0, 0.5, 7.0]
    assert m[0].tolist() == [1, 0, 0, 0, 1]


def test_dense_errors_match_reference(dev):
    from kvquant.triton_batched import pack_keys_per_channel_batched

    x = torch.randn(4, 2, 8, device=dev).float()
    p = torch.zeros(2, 8, 4, device=dev)
    with pytest.raises(AssertionError):
        pack_keys_per_channel_batched(x, p, p[..., 0], p[..., 0])  # fp32 values
    with pytest.raises(AssertionError):
        pack_keys_per_channel_batched(x.half().transpose(0, 1), p, p[..., 0], p[..., 0])


# ----------------------------------------------------------- compact format

@pytest.mark.parametrize("T,H,D,L,thr", [(1000, 4, 128, 16, 1.0), (777, 4, 128, 4, 0.7),
                                         (100, 2, 64, 16, 1.5), (50, 3, 128, 16, 1.0),
                                         (3, 4, 128, 4, 0.2), (64, 1, 32, 16, 0.05)])
def test_compact_keys_vs_oracle(dev, T, H, D, L, thr):
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact, nuq_unpack_compact

    bits = 2 if L <= 4 else 4
    x = (RNG.standard_t(3, (T, H, D))).astype(np.float16)
    poles, up, lo = _kscales(H, D, L, thr=thr)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(lo, dev), per_token=False)
    cc = nuq_pack_compact(_t(x, dev), t, bits, capacity=16)  # forces the re-issue path
    wc, wv, wm = O.pack_k(x, poles.astype(np.float32), up.astype(np.float32), lo.astype(np.float32))
    pk, rp, col, val = O.pack_compact(wc, wv, wm, bits)
    assert cc.nnz == len(col)
    assert np.array_equal(cc.packed.cpu().numpy(), pk)
    assert np.array_equal(cc.row_ptr.cpu().numpy(), rp)
    assert np.array_equal(cc.col.cpu().numpy(), col)
    assert np.array_equal(_bits(cc.val), val)
    out = nuq_unpack_compact(cc, t)
    assert np.array_equal(_bits(out), O.unpack(wc, wv, wm, poles.astype(np.float32), "k"))


@pytest.mark.parametrize("T,Tcal,L,offset", [(900, 256, 16, 0), (300, 512, 4, 100), (64, 16, 16, 5)])
def test_compact_values_vs_oracle(dev, T, Tcal, L, offset):
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact, nuq_unpack_compact

    H, D = 4, 128
    bits = 2 if L <= 4 else 4
    x = RNG.standard_t(3, (T, H, D)).astype(np.float16)
    poles = np.sort(RNG.standard_normal((H, Tcal, L)), axis=-1).astype(np.float16)
    up = RNG.uniform(0.8, 2.5, (H, Tcal)).astype(np.float16)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(-up, dev), per_token=True)
    cc = nuq_pack_compact(_t(x, dev), t, bits, pos_offset=offset)
    pos = np.arange(T) + offset
    wc, wv, wm = O.pack_v(x, poles.astype(np.float32), up.astype(np.float32),
                          (-up).astype(np.float32), positions=pos)
    pk, rp, col, val = O.pack_compact(wc, wv, wm, bits)
    assert np.array_equal(cc.packed.cpu().numpy(), pk)
    assert np.array_equal(cc.row_ptr.cpu().numpy(), rp)
    assert np.array_equal(cc.col.cpu().numpy(), col)
    assert np.array_equal(_bits(cc.val), val)
    out = nuq_unpack_compact(cc, t, pos_offset=offset)
    assert np.array_equal(_bits(out), O.unpack(wc, wv, wm, poles.astype(np.float32), "v", positions=pos))
    # explicit positions give the same result as the offset
    cc2 = nuq_pack_compact(_t(x, dev), t, bits, positions=torch.from_numpy(pos))
    assert torch.equal(cc2.packed, cc.packed) and torch.equal(cc2.row_ptr, cc.row_ptr)


@pytest.mark.parametrize("per_token,L", [(False, 16), (True, 4)])
def test_compact_many_tiles_vs_oracle(dev, per_token, L):
    """65,536 tokens x 4 heads: thousands of tiles, so the CSR offsets cross
    many copy blocks; every byte against the oracle."""
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact, nuq_unpack_compact

    T, H, D = 65536, 4, 128
    bits = 2 if L <= 4 else 4
    x = RNG.standard_t(3, (T, H, D)).astype(np.float16)
    rows = D if not per_token else 4096
    poles = np.sort(RNG.standard_normal((H, rows, L)), axis=-1).astype(np.float16)
    up = RNG.uniform(1.5, 3.0, (H, rows)).astype(np.float16)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(-up, dev), per_token=per_token)
    cc = nuq_pack_compact(_t(x, dev), t, bits)
    f32 = [a.astype(np.float32) for a in (poles, up, -up)]
    if per_token:
        wc, wv, wm = O.pack_v(x, *f32, positions=np.arange(T))
    else:
        wc, wv, wm = O.pack_k(x, *f32)
    pk, rp, col, val = O.pack_compact(wc, wv, wm, bits)
    assert cc.nnz == len(col) and 0.01 < cc.nnz / x.size < 0.5
    assert np.array_equal(cc.row_ptr.cpu().numpy(), rp)
    assert np.array_equal(cc.packed.cpu().numpy(), pk)
    assert np.array_equal(cc.col.cpu().numpy(), col)
    assert np.array_equal(_bits(cc.val), val)
    out = nuq_unpack_compact(cc, t)
    want = O.unpack(wc, wv, wm, f32[0], "v" if per_token else "k",
                    positions=np.arange(T) if per_token else None)
    assert np.array_equal(_bits(out), want)


@pytest.mark.parametrize("per_token,L,T", [(False, 16, 262144), (True, 4, 131072),
                                           (False, 4, 131072), (True, 16, 131072)])
def test_compact_full_size_vs_oracle(dev, per_token, L, T):
    """Prefill-sized calls, all four stage kernels (K / V at nuq2 / nuq4) at
    the full (131072, 4, 128) layer shape or larger: thousands of wave tiles,
    so the CSR copy runs with 32 to 128 tiles per block; every byte against
    the oracle."""
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact

    H, D = 4, 128
    bits = 2 if L <= 4 else 4
    rng = np.random.default_rng(11)
    x = rng.standard_t(3, (T, H, D)).astype(np.float16)
    rows = D if not per_token else 4096
    poles = np.sort(rng.standard_normal((H, rows, L)), axis=-1).astype(np.float16)
    up = rng.uniform(1.5, 3.0, (H, rows)).astype(np.float16)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(-up, dev), per_token=per_token)
    cc = nuq_pack_compact(_t(x, dev), t, bits)
    f32 = [a.astype(np.float32) for a in (poles, up, -up)]
    if per_token:
        wc, wv, wm = O.pack_v(x, *f32, positions=np.arange(T))
    else:
        wc, wv, wm = O.pack_k(x, *f32)
    pk, rp, col, val = O.pack_compact(wc, wv, wm, bits)
    assert cc.nnz == len(col) and 0.01 < cc.nnz / x.size < 0.5
    assert np.array_equal(cc.row_ptr.cpu().numpy(), rp)
    assert np.array_equal(cc.packed.cpu().numpy(), pk)
    assert np.array_equal(cc.col.cpu().numpy(), col)
    assert np.array_equal(_bits(cc.val), val)


@pytest.mark.parametrize("per_token,L,thr", [(False, 16, 0.3), (True, 16, 0.3), (False, 4, 0.1),
                                             (True, 4, 0.6)])
def test_compact_dense_outliers_vs_oracle(dev, per_token, L, thr):
    """Thresholds so tight that 30-90% of the elements are outliers: every
    64-row chunk holds more outliers than its wave keeps in LDS, so the
    entries past that are found again from the input after the chunk's
    offset is known.  Every byte against the oracle, and the workspace's
    error word stays zero."""
    from helix_kv import _native as N
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact, pack_workspace

    T, H, D = 3000, 4, 128
    bits = 2 if L <= 4 else 4
    x = RNG.standard_t(3, (T, H, D)).astype(np.float16)
    rows = D if not per_token else 512
    poles = np.sort(RNG.standard_normal((H, rows, L)), axis=-1).astype(np.float16)
    up = RNG.uniform(thr, 2 * thr, (H, rows)).astype(np.float16)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(-up, dev), per_token=per_token)
    cc = nuq_pack_compact(_t(x, dev), t, bits, capacity=T * H * D)
    f32 = [a.astype(np.float32) for a in (poles, up, -up)]
    if per_token:
        wc, wv, wm = O.pack_v(x, *f32, positions=np.arange(T))
    else:
        wc, wv, wm = O.pack_k(x, *f32)
    pk, rp, col, val = O.pack_compact(wc, wv, wm, bits)
    assert cc.nnz == len(col) and cc.nnz / x.size > 0.25
    assert np.array_equal(cc.row_ptr.cpu().numpy(), rp)
    assert np.array_equal(cc.packed.cpu().numpy(), pk)
    assert np.array_equal(cc.col.cpu().numpy(), col)
    assert np.array_equal(_bits(cc.val), val)
    ws = pack_workspace(T, H, D, dev)
    assert int(ws[12:16].view(torch.int32).item()) == 0  # no look-back gave up


def test_compact_batch_equals_single_calls(dev):
    """One hkv_nuq_pack_compact_batch over tensors of all four kernel
    variants, several heads counts and sizes (including an empty tensor and
    more tensors of one variant than a launch takes): each result is
    identical to its own hkv_nuq_pack_compact call; two against the oracle."""
    from helix_kv.ops import CompactCodes, NuqLayerTables, nuq_pack_compact, nuq_pack_compact_batch

    rng = np.random.default_rng(5)
    D = 128
    specs = [(False, 16, 4, 3000), (True, 4, 4, 2000), (False, 4, 4, 1), (True, 16, 4, 0),
             (False, 16, 2, 700), (True, 16, 4, 1500)] + [(False, 4, 4, 100 + 37 * i) for i in range(18)]
    jobs, singles, host = [], [], []
    for per_token, L, H, T in specs:
        bits = 2 if L <= 4 else 4
        x = rng.standard_t(3, (T, H, D)).astype(np.float16)
        rows = D if not per_token else 1024
        poles = np.sort(rng.standard_normal((H, rows, L)), axis=-1).astype(np.float16)
        up = rng.uniform(1.2, 2.5, (H, rows)).astype(np.float16)
        t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(-up, dev), per_token=per_token)
        xd = _t(x, dev)
        cap = max(64, T * H * D // 4)
        jobs.append((xd, t, bits, CompactCodes.empty(T, H, D, bits, cap, dev)))
        singles.append(nuq_pack_compact(xd, t, bits, capacity=cap))
        host.append((x, poles, up, per_token, bits))
    outs = nuq_pack_compact_batch(jobs)
    torch.cuda.synchronize()
    for cc, ref in zip(outs, singles):
        n = int(cc.row_ptr[-1].item())
        assert n == ref.nnz
        assert torch.equal(cc.packed, ref.packed) and torch.equal(cc.row_ptr, ref.row_ptr)
        assert torch.equal(cc.col[:n], ref.col[:n]) and torch.equal(cc.val[:n], ref.val[:n])
    # the batched unpack of the same tensors equals the single-tensor unpack
    from helix_kv.ops import CompactUnpackBatch, nuq_unpack_compact
    ujobs = [(cc, job[1], torch.empty_like(job[0])) for cc, job in zip(outs, jobs)]
    CompactUnpackBatch(ujobs)()
    for (cc, t, out), job in zip(ujobs, jobs):
        assert torch.equal(out.view(torch.int16), nuq_unpack_compact(cc, t).view(torch.int16))
    for i in (0, 1):
        x, poles, up, per_token, bits = host[i]
        f32 = [a.astype(np.float32) for a in (poles, up, -up)]
        if per_token:
            wc, wv, wm = O.pack_v(x, *f32, positions=np.arange(x.shape[0]))
        else:
            wc, wv, wm = O.pack_k(x, *f32)
        pk, rp, col, val = O.pack_compact(wc, wv, wm, bits)
        cc = outs[i]
        assert np.array_equal(cc.packed.cpu().numpy(), pk) and np.array_equal(cc.row_ptr.cpu().numpy(), rp)
        n = len(col)
        assert np.array_equal(cc.col[:n].cpu().numpy(), col) and np.array_equal(_bits(cc.val[:n]), val)


@pytest.mark.parametrize("H,per_token,L,T", [(1, False, 16, 257), (2, False, 4, 129), (8, False, 16, 333),
                                          (8, True, 16, 333), (16, True, 4, 77), (2, True, 16, 5)])
def test_compact_unpack_heads_and_positions(dev, H, per_token, L, T):
    """D = 128 unpack for every power-of-two head count, partial last tiles,
    and per-token rows from explicit positions, some outside the calibrated
    rows (clamped), and from a negative offset."""
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact, nuq_unpack_compact

    D = 128
    bits = 2 if L <= 4 else 4
    x = RNG.standard_t(3, (T, H, D)).astype(np.float16)
    rows = D if not per_token else 40
    poles = np.sort(RNG.standard_normal((H, rows, L)), axis=-1).astype(np.float16)
    up = RNG.uniform(1.0, 2.5, (H, rows)).astype(np.float16)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(-up, dev), per_token=per_token)
    f32 = [a.astype(np.float32) for a in (poles, up, -up)]
    cases = [("none", None)]
    if per_token:
        cases = [("array", RNG.integers(-20, rows + 20, T)), ("offset", np.arange(T) - 7)]
    for kind, pos in cases:
        if per_token:
            wc, wv, wm = O.pack_v(x, *f32, positions=pos)
        else:
            wc, wv, wm = O.pack_k(x, *f32)
        want = O.unpack(wc, wv, wm, f32[0], "v" if per_token else "k", positions=pos)
        if kind == "offset":  # the same rows from an offset
            cc = nuq_pack_compact(_t(x, dev), t, bits, pos_offset=-7)
            got = nuq_unpack_compact(cc, t, pos_offset=-7)
        else:
            kw = {} if pos is None else dict(positions=torch.from_numpy(pos))
            cc = nuq_pack_compact(_t(x, dev), t, bits, **kw)
            got = nuq_unpack_compact(cc, t, **kw)
        pk, rp, col, val = O.pack_compact(wc, wv, wm, bits)
        assert np.array_equal(cc.packed.cpu().numpy(), pk)
        assert np.array_equal(cc.row_ptr.cpu().numpy(), rp)
        assert np.array_equal(_bits(got), want)


def test_compact_unpack_respects_capacity(dev):
    """CSR entries beyond the col/val capacity are never read: those outliers
    decode as their poles, everything else is unchanged."""
    from helix_kv.ops import CompactCodes, NuqLayerTables, nuq_pack_compact, nuq_unpack_compact

    T, H, D, L = 256, 4, 128, 16
    x = RNG.standard_t(3, (T, H, D)).astype(np.float16)
    poles, up, lo = _kscales(H, D, L, thr=1.0)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(lo, dev), per_token=False)
    full = nuq_pack_compact(_t(x, dev), t, 4)
    keep = full.nnz // 2
    cut = CompactCodes(full.packed, full.row_ptr, full.col[:keep].clone(), full.val[:keep].clone(), 4)
    got = _bits(nuq_unpack_compact(cut, t))
    wc, wv, wm = O.pack_k(x, poles.astype(np.float32), up.astype(np.float32), lo.astype(np.float32))
    flat_m = wm.reshape(-1).copy()
    idx = np.flatnonzero(flat_m)
    flat_m[idx[keep:]] = 0
    want = O.unpack(wc, wv, flat_m.reshape(wm.shape), poles.astype(np.float32), "k")
    assert np.array_equal(got, want)


def test_compact_reused_out_keeps_capacity(dev):
    """A sync=True pack into a caller's CompactCodes returns trimmed views and
    leaves the caller's col / val at full capacity, so a later sync=False pack
    into the same object with more outliers is complete; a sync=True pack
    whose outliers exceed the given capacity raises."""
    from helix_kv.ops import CompactCodes, NuqLayerTables, nuq_pack_compact

    T, H, D, L = 1024, 4, 128, 16
    poles, up, lo = _kscales(H, D, L, thr=2.0)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(lo, dev), per_token=False)
    f32 = [a.astype(np.float32) for a in (poles, up, lo)]
    few = (RNG.standard_normal((T, H, D)) * 0.7).astype(np.float16)
    many = (RNG.standard_t(3, (T, H, D)) * 1.5).astype(np.float16)
    cap = T * H * D // 2
    out = CompactCodes.empty(T, H, D, 4, cap, dev)
    r1 = nuq_pack_compact(_t(few, dev), t, 4, out=out, sync=True)
    assert out.col.numel() == cap and out.val.numel() == cap
    assert r1.col.numel() == r1.nnz and out.nnz == r1.nnz
    r2 = nuq_pack_compact(_t(many, dev), t, 4, out=out, sync=False)
    assert r2 is out
    torch.cuda.synchronize()
    nnz2 = int(out.row_ptr[-1])
    assert r1.nnz < nnz2 <= cap
    pk, rp, col, val = O.pack_compact(*O.pack_k(many, *f32), 4)
    assert np.array_equal(out.row_ptr.cpu().numpy(), rp)
    assert np.array_equal(out.col[:nnz2].cpu().numpy(), col)
    assert np.array_equal(_bits(out.val[:nnz2]), val)
    small = CompactCodes.empty(T, H, D, 4, r1.nnz, dev)
    with pytest.raises(RuntimeError, match="exceed the capacity"):
        nuq_pack_compact(_t(many, dev), t, 4, out=small, sync=True)


def test_compact_empty_and_repeat_calls(dev):
    """Empty input; and the look-back workspace is reused across calls."""
    from helix_kv.ops import NuqLayerTables, nuq_pack_compact

    H, D = 4, 128
    poles, up, lo = _kscales(H, D, 16, thr=0.5)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(lo, dev), per_token=False)
    cc = nuq_pack_compact(torch.empty((0, H, D), dtype=torch.float16, device=dev), t, 4)
    assert cc.row_ptr.tolist() == [0] and cc.nnz == 0
    x = RNG.standard_normal((2048, H, D)).astype(np.float16)
    first = nuq_pack_compact(_t(x, dev), t, 4)
    for _ in range(5):
        again = nuq_pack_compact(_t(x, dev), t, 4)
        assert torch.equal(again.row_ptr, first.row_ptr) and torch.equal(again.col, first.col)


# --------------------------------------------------- spec functions (nuq.py)

@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_spec_functions_vs_oracle(dev, dt):
    from kvquant.nuq import dequantize_nuq, find_outliers, nearest_pole_index, quantize_nuq

    v = torch.randn(64, 32).to(dt)
    p = torch.sort(torch.randn(64, 32, 16), dim=-1).values.to(dt)
    up = torch.full((64, 32), 1.2).to(dt)
    codes, recon, mask = O.nuq_py_semantics(v.numpy(), p.numpy(), up.numpy(), (-up).numpy())
    r, m = quantize_nuq(v.to(dev), p.to(dev), up.to(dev), -up.to(dev))
    assert np.array_equal(m.cpu().numpy(), mask)
    assert np.array_equal(r.cpu().numpy(), recon)
    assert np.array_equal(nearest_pole_index(v.to(dev), p.to(dev)).cpu().numpy(), codes)
    assert torch.equal(find_outliers(v.to(dev), up.to(dev), -up.to(dev)), m)
    outl = torch.where(m, v.to(dev), torch.zeros_like(v.to(dev)))
    deq = dequantize_nuq(torch.from_numpy(codes).to(dev), outl, m, p.to(dev))
    assert torch.equal(deq, r)


def test_spec_known_answers_on_gpu(dev):
    # src/kvquant/tests/test_nuq_roundtrip.py:25-48
    from kvquant.nuq import find_outliers, quantize_nuq, round_to_nearest_pole

    values = torch.tensor([0.1, 0.4, -0.6, 1.2], device=dev)
    poles = torch.tensor([-1.0, -0.5, 0.0, 0.5, 1.0], device=dev).expand(4, 5)
    assert round_to_nearest_pole(values, poles).tolist() == [0.0, 0.5, -0.5, 1.0]
    m = find_outliers(torch.tensor([[-2.0, -0.4, 0.1, 0.7, 3.5]], device=dev),
                      torch.tensor([[1.0]], device=dev), torch.tensor([[-1.0]], device=dev))
    assert m.tolist() == [[True, False, False, False, True]]
    z = torch.zeros(5, 4, device=dev)
    m = find_outliers(z, torch.full((5, 4), 1.0, device=dev), torch.full((5, 4), -1.0, device=dev),
                      first_few_fp16=2, seq_dim=0)
    assert m[:2].all() and not m[2:].any()
    vals = torch.linspace(-1, 1, 256, device=dev)
    pl = torch.tensor([-1.0, -0.33, 0.33, 1.0], device=dev).expand(256, 4)
    out, mask = quantize_nuq(vals, pl, torch.full((256,), 100.0, device=dev),
                             torch.full((256,), -100.0, device=dev))
    assert mask.sum() == 0 and (out - vals).abs().max().item() < 0.34


@pytest.mark.parametrize("per_token", [False, True])
def test_compact_pack_capacity_guard(dev, per_token):
    """hkv_nuq_pack_compact with a CSR capacity below nnz, called through the C
    ABI: row_ptr is complete (row_ptr[T*H] = the true nnz), the entries below
    the capacity are the oracle's, and nothing at or past the capacity is
    written (sentinel-filled guard region)."""
    from helix_kv import _native as N
    from helix_kv.ops import NuqLayerTables, pack_workspace

    T, H, D, L = 8192, 4, 128, 16
    x = RNG.standard_t(3, (T, H, D)).astype(np.float16)
    rows = D if not per_token else 1024
    poles = np.sort(RNG.standard_normal((H, rows, L)), axis=-1).astype(np.float16)
    up = RNG.uniform(1.5, 3.0, (H, rows)).astype(np.float16)
    t = NuqLayerTables(_t(poles, dev), _t(up, dev), _t(-up, dev), per_token=per_token)
    f32 = [a.astype(np.float32) for a in (poles, up, -up)]
    if per_token:
        wc, wv, wm = O.pack_v(x, *f32, positions=np.arange(T))
    else:
        wc, wv, wm = O.pack_k(x, *f32)
    pk, rp, col, val = O.pack_compact(wc, wv, wm, 4)
    nnz = len(col)
    cap = nnz // 3 + 7
    guard = 4096
    xd = _t(x, dev)
    packed = torch.empty((T, H, D // 2), dtype=torch.uint8, device=dev)
    row_ptr = torch.empty(T * H + 1, dtype=torch.int32, device=dev)
    gcol = torch.full((cap + guard,), 0xAB, dtype=torch.uint8, device=dev)
    gval = torch.full((cap + guard,), 0x1234, dtype=torch.int16, device=dev)
    ws = pack_workspace(T, H, D, dev)
    st = N.lib().hkv_nuq_pack_compact(N.ptr(xd), T, H, D, 4, t.struct(), N.ptr(packed),
                                      N.ptr(row_ptr), N.ptr(gcol), N.ptr(gval), cap, N.ptr(ws),
                                      ws.numel(), N.stream_of(xd))
    assert st == 0
    torch.cuda.synchronize()
    assert np.array_equal(row_ptr.cpu().numpy(), rp) and int(row_ptr[-1]) == nnz > cap
    assert np.array_equal(packed.cpu().numpy(), pk)
    gc = gcol.cpu().numpy()
    gv = gval.cpu().numpy().view(np.uint16)
    assert np.array_equal(gc[:cap], col[:cap]) and np.array_equal(gv[:cap], val[:cap])
    assert (gc[cap:] == 0xAB).all() and (gv[cap:] == 0x1234).all()
