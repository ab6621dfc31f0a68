"""GPU parity of the compact pool (write_kv / unpack_to_staging) and the Quest
block selector against the oracle -- bit-exact codes, masks, outlier values,
staging and block statistics -- plus the reference's own pool and selector
tests (src/kvquant/tests/test_compact_pool.py, test_quest_selector.py) run
through the drop-in API."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(77)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _scales(L, H, D, Tcal, LK, LV, dtype=torch.float16, thr=1.5):
    from kvquant.scales import KVScales, PerChannelScale, PerTokenScale

    keys, vals = [], []
    for _ in range(L):
        kp = torch.from_numpy(np.sort(RNG.standard_normal((H, D, LK)), -1)).to(dtype)
        vp = torch.from_numpy(np.sort(RNG.standard_normal((H, Tcal, LV)), -1)).to(dtype)
        ku = torch.from_numpy(RNG.uniform(0.5 * thr, 1.5 * thr, (H, D))).to(dtype)
        vu = torch.from_numpy(RNG.uniform(0.5 * thr, 1.5 * thr, (H, Tcal))).to(dtype)
        keys.append(PerChannelScale(kp, ku, -ku, 4 if LK > 4 else 2))
        vals.append(PerTokenScale(vp, vu, -vu, 4 if LV > 4 else 2))
    return KVScales(per_layer_keys=keys, per_layer_values=vals, first_few_fp16=4, num_bits=2)


def _np_scale(s):
    return tuple(t.float().cpu().numpy() for t in (s.poles, s.upper_threshold, s.lower_threshold))


def _pool_np(pool, layer):
    return {n: (getattr(pool, n)[layer].cpu().numpy() if n in ("k_min", "k_max") else
                getattr(pool, n)[layer].cpu().contiguous().numpy().view(
                    np.uint16 if n.endswith("outv") else np.uint8))
            for n in ("k_codes", "k_outv", "k_outm", "v_codes", "v_outv", "v_outm", "k_min", "k_max")}


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("NB,BS,H,D,LK,LV", [(64, 16, 4, 128, 16, 4), (10, 8, 2, 64, 4, 16),
                                             (7, 5, 3, 16, 16, 16)])
def test_pool_write_gather_vs_oracle(dev, dtype, NB, BS, H, D, LK, LV):
    from kvquant.compact_pool import CompactKVPool

    L, Tcal = 2, 40
    scales = _scales(L, H, D, Tcal, LK, LV, dtype=dtype)
    pool = CompactKVPool(L, NB, BS, H, D, scales, device="cuda:0")
    ref = [{n: a.copy() for n, a in _pool_np(pool, l).items()} for l in range(L)]
    for layer in range(L):
        ks, vs = _np_scale(scales.per_layer_keys[layer]), _np_scale(scales.per_layer_values[layer])
        for T in (3 * BS + 1, 1, 2 * BS):  # prefill chunk then decode-style appends
            key = RNG.standard_t(3, (T, H, D)).astype(np.float16)
            val = RNG.standard_t(3, (T, H, D)).astype(np.float16)
            slots = RNG.choice(NB * BS, size=T, replace=False).astype(np.int64)
            slots[RNG.random(T) < 0.1] = -1
            pos = RNG.integers(0, 2 * Tcal, T).astype(np.int64)
            pool.write_kv(layer, torch.from_numpy(key).to(dev), torch.from_numpy(val).to(dev),
                          torch.from_numpy(slots).to(dev), torch.from_numpy(pos).to(dev))
            O.pool_write(ref[layer], key, val, slots, pos, ks, vs, BS)
        got = _pool_np(pool, layer)
        for n in got:
            if n in ("k_min", "k_max"):
                assert np.array_equal(got[n].view(np.uint32), ref[layer][n].view(np.uint32)), n
            else:
                assert np.array_equal(got[n], ref[layer][n]), n
        ids = RNG.choice(NB, size=min(NB, 5), replace=False).astype(np.int64)
        first = (ids * BS + RNG.integers(-3, 3 * Tcal, ids.size)).clip(0).astype(np.int64)
        sk = torch.empty((ids.size, BS, H, D), dtype=torch.float16, device=dev)
        sv = torch.empty_like(sk)
        pool.unpack_to_staging(layer, torch.from_numpy(ids).to(dev), torch.from_numpy(first).to(dev),
                               sk, sv)
        wk, wv = O.pool_gather(ref[layer], ids, first, ks, vs)
        assert np.array_equal(_bits(sk), wk)
        assert np.array_equal(_bits(sv), wv)


def test_pool_gather_bad_block_ids_give_zero_rows(dev):
    from kvquant.compact_pool import CompactKVPool

    NB, BS, H, D = 4, 4, 2, 16
    scales = _scales(1, H, D, 8, 16, 4)
    pool = CompactKVPool(1, NB, BS, H, D, scales)
    x = torch.randn((NB * BS, H, D), dtype=torch.float16, device=dev)
    pos = torch.arange(NB * BS, device=dev)
    pool.write_kv(0, x, x, pos, pos)
    ids = torch.tensor([1, -2, NB, 3], device=dev)
    sk = torch.full((4, BS, H, D), 7.0, dtype=torch.float16, device=dev)
    sv = sk.clone()
    pool.unpack_to_staging(0, ids, ids.clamp(min=0) * BS, sk, sv)
    assert torch.all(sk[1] == 0) and torch.all(sk[2] == 0) and torch.all(sv[2] == 0)
    assert not torch.all(sk[0] == 0)


# ------------------------------ the reference's own pool tests (drop-in API)

def _tiny_ref_scales(L=2, H=2, D=16, T_cal=32, NL_K=16, NL_V=4, seed=0):
    """src/kvquant/tests/test_compact_pool.py:32-46 (inputs drawn here)."""
    from kvquant.scales import KVScales, PerChannelScale, PerTokenScale

    g = torch.Generator(device="cpu").manual_seed(seed)
    keys, vals = [], []
    for _ in range(L):
        kp = torch.randn(H, D, NL_K, generator=g).half().sort(dim=-1).values.cuda()
        ku = torch.full((H, D), 1.5, dtype=torch.float16, device="cuda")
        keys.append(PerChannelScale(poles=kp, upper_threshold=ku, lower_threshold=-ku, num_bits=4))
        vp = torch.randn(H, T_cal, NL_V, generator=g).half().sort(dim=-1).values.cuda()
        vu = torch.full((H, T_cal), 1.5, dtype=torch.float16, device="cuda")
        vals.append(PerTokenScale(poles=vp, upper_threshold=vu, lower_threshold=-vu, num_bits=2))
    return KVScales(per_layer_keys=keys, per_layer_values=vals, first_few_fp16=4, num_bits=2)


def _ref_quant(values, poles, upper, lower):
    """src/kvquant/tests/test_compact_pool.py:49-69 (fp32 per-element restatement)."""
    v2 = values[:, None]
    if poles.dim() == 2:
        best = (v2 - poles).abs().argmin(dim=-1)
        recon = poles.gather(-1, best[:, None]).squeeze(-1)
    else:
        best = (v2 - poles[None, :]).abs().argmin(dim=-1)
        recon = poles[best]
    out = (values > upper) | (values < lower)
    return torch.where(out, values, recon), out


def test_reference_pool_pack_unpack_round_trip(dev):
    """src/kvquant/tests/test_compact_pool.py:136-195."""
    from kvquant.compact_pool import CompactKVPool

    torch.manual_seed(2)
    L, NB, BS, H, D, T_cal = 1, 3, 8, 2, 16, 64
    scales = _tiny_ref_scales(L=L, H=H, D=D, T_cal=T_cal)
    pool = CompactKVPool(num_layers=L, num_blocks=NB, block_size=BS, num_kv_heads=H,
                         head_size=D, scales=scales)
    T = 16
    key = torch.randn(T, H, D, dtype=torch.float16, device=dev)
    value = torch.randn_like(key)
    sm = torch.arange(T, dtype=torch.int64, device=dev)
    pool.write_kv(0, key, value, sm, sm)
    ids = torch.tensor([0, 1], dtype=torch.int64, device=dev)
    first = torch.tensor([0, BS], dtype=torch.int64, device=dev)
    sk = torch.empty((2, BS, H, D), dtype=torch.float16, device=dev)
    sv = torch.empty_like(sk)
    pool.unpack_to_staging(0, ids, first, sk, sv)
    ks, vs = scales.per_layer_keys[0], scales.per_layer_values[0]
    for k_idx in range(2):
        for ib in range(BS):
            abs_t = int(ids[k_idx]) * BS + ib
            pos = min(int(first[k_idx]) + ib, T_cal - 1)
            for h in range(H):
                k_ref, _ = _ref_quant(key[abs_t, h].float(), ks.poles[h].float(),
                                      ks.upper_threshold[h].float(), ks.lower_threshold[h].float())
                v_ref, _ = _ref_quant(value[abs_t, h].float(), vs.poles[h, pos].float(),
                                      vs.upper_threshold[h, pos].float(),
                                      vs.lower_threshold[h, pos].float())
                torch.testing.assert_close(sk[k_idx, ib, h].float(), k_ref, atol=1e-2, rtol=1e-2)
                torch.testing.assert_close(sv[k_idx, ib, h].float(), v_ref, atol=1e-2, rtol=1e-2)


def test_reference_pool_block_stats(dev):
    """src/kvquant/tests/test_compact_pool.py:198-240, tightened to exact."""
    from kvquant.compact_pool import CompactKVPool

    torch.manual_seed(1)
    L, NB, BS, H, D, T_cal = 1, 2, 4, 2, 8, 16
    scales = _tiny_ref_scales(L=L, H=H, D=D, T_cal=T_cal)
    pool = CompactKVPool(num_layers=L, num_blocks=NB, block_size=BS, num_kv_heads=H,
                         head_size=D, scales=scales)
    T = 8
    key = torch.randn(T, H, D, dtype=torch.float16, device=dev)
    sm = torch.arange(T, dtype=torch.int64, device=dev)
    pool.write_kv(0, key, torch.randn_like(key), sm, sm)
    ks = scales.per_layer_keys[0]
    for b in range(NB):
        rec = torch.stack([torch.stack([_ref_quant(key[t, h].float(), ks.poles[h].float(),
                                                   ks.upper_threshold[h].float(),
                                                   ks.lower_threshold[h].float())[0]
                                        for h in range(H)]) for t in range(b * BS, (b + 1) * BS)])
        assert torch.equal(pool.k_min[0, b], rec.amin(0))
        assert torch.equal(pool.k_max[0, b], rec.amax(0))


# ------------------------------------------------------------ block selector

def _sel_scales(L=1, H=2, D=8, T_cal=32, NL_K=16, NL_V=4):
    """src/kvquant/tests/test_quest_selector.py:20-37."""
    from kvquant.scales import KVScales, PerChannelScale, PerTokenScale

    keys = [PerChannelScale(
        poles=torch.linspace(-1.5, 1.5, NL_K, dtype=torch.float16, device="cuda")
        .reshape(1, 1, -1).expand(H, D, NL_K).contiguous(),
        upper_threshold=torch.full((H, D), 2.0, dtype=torch.float16, device="cuda"),
        lower_threshold=torch.full((H, D), -2.0, dtype=torch.float16, device="cuda"),
        num_bits=4) for _ in range(L)]
    vals = [PerTokenScale(
        poles=torch.linspace(-1.5, 1.5, NL_V, dtype=torch.float16, device="cuda")
        .reshape(1, 1, -1).expand(H, T_cal, NL_V).contiguous(),
        upper_threshold=torch.full((H, T_cal), 2.0, dtype=torch.float16, device="cuda"),
        lower_threshold=torch.full((H, T_cal), -2.0, dtype=torch.float16, device="cuda"),
        num_bits=2) for _ in range(L)]
    return KVScales(per_layer_keys=keys, per_layer_values=vals, first_few_fp16=4, num_bits=2)


def test_reference_selector_planted_block_and_sinks(dev):
    """src/kvquant/tests/test_quest_selector.py:41-95."""
    from kvquant.compact_pool import CompactKVPool
    from kvquant.quest_selector import select_top_blocks_for_layer

    H, D, BS, NB = 2, 8, 4, 6
    pool = CompactKVPool(num_layers=1, num_blocks=NB, block_size=BS, num_kv_heads=H,
                         head_size=D, scales=_sel_scales(H=H, D=D))
    T = 5 * BS
    key = torch.zeros(T, H, D, dtype=torch.float16, device=dev)
    key[3 * BS:4 * BS] = 1.0
    sm = torch.arange(T, dtype=torch.int64, device=dev)
    pool.write_kv(0, key, torch.zeros_like(key), sm, sm)
    q = torch.ones(H, D, dtype=torch.float16, device=dev)
    used = torch.arange(5, dtype=torch.int64, device=dev)
    sel, first = select_top_blocks_for_layer(pool, 0, q, used, block_size=BS, top_k=1,
                                             sink_blocks=0)
    assert sel.tolist() == [3] and first.tolist() == [3 * BS]
    pool2 = CompactKVPool(num_layers=1, num_blocks=NB, block_size=BS, num_kv_heads=H,
                          head_size=D, scales=_sel_scales(H=H, D=D))
    z = torch.zeros(T, H, D, dtype=torch.float16, device=dev)
    pool2.write_kv(0, z, z, sm, sm)
    sel, _ = select_top_blocks_for_layer(pool2, 0, q, used, block_size=BS, top_k=1, sink_blocks=2)
    assert 0 in sel.tolist() and 1 in sel.tolist()


@pytest.mark.parametrize("NB,NU,H,top_k,sinks", [(4096, 3000, 4, 700, 4), (64, 64, 2, 10, 1),
                                                 (100, 37, 3, 50, 4), (20, 0, 2, 3, 1)])
def test_selector_vs_oracle_random(dev, NB, NU, H, top_k, sinks):
    from kvquant.compact_pool import CompactKVPool
    from kvquant.quest_selector import select_top_blocks_for_layer

    D, BS = 64, 16
    pool = CompactKVPool(1, NB, BS, H, D, _scales(1, H, D, 8, 16, 4))
    mn = RNG.standard_normal((NB, H, D)).astype(np.float32)
    mx = (mn + RNG.random((NB, H, D))).astype(np.float32)
    pool.k_min[0].copy_(torch.from_numpy(mn))
    pool.k_max[0].copy_(torch.from_numpy(mx))
    used = RNG.permutation(NB)[:NU].astype(np.int64)  # not ascending: the union sorts by id
    q = RNG.standard_normal((H, D)).astype(np.float16)
    for _ in range(2):  # the flags are left clean for the next call
        sel, first = select_top_blocks_for_layer(pool, 0, torch.from_numpy(q).to(dev),
                                                 torch.from_numpy(used).to(dev), BS, top_k, sinks)
        if NU == 0:
            assert sel.numel() == 0
            continue
        bound = O.page_bound(q.astype(np.float32), mn[used], mx[used])
        want_ids, want_first = O.select_union(bound, used, top_k, sinks, BS)
        assert np.array_equal(sel.cpu().numpy(), want_ids)
        assert np.array_equal(first.cpu().numpy(), want_first)
