"""Pins of the torch restatement of the reference's CPU path
(oracle/torch_ref.py), the code the CPU baseline times: against the C/numpy
oracle, which the other oracle tests pin to the reference's known answers."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle as O
from oracle import torch_ref as R

RNG = np.random.default_rng(7)


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_quantize_matches_spec_semantics(dt):
    v = torch.from_numpy(RNG.standard_t(3, (300, 4, 32))).to(dt)
    p = torch.from_numpy(np.sort(RNG.standard_normal((4, 32, 16)), -1)).to(dt)
    up = torch.full((4, 32), 1.5, dtype=dt)
    recon, mask, idx = R.quantize_nuq(v, p.expand(300, 4, 32, 16), up, -up)
    codes, wrecon, wmask = O.nuq_py_semantics(v.numpy(), p.numpy(), up.numpy(), (-up).numpy())
    assert np.array_equal(idx.numpy(), codes)
    assert np.array_equal(mask.numpy(), wmask)
    assert np.array_equal(recon.numpy(), wrecon)
    deq = R.dequantize_nuq(idx, torch.where(mask, v, torch.zeros_like(v)), mask,
                           p.expand(300, 4, 32, 16))
    assert torch.equal(deq, recon)


def test_round_trip_per_token_clamp_and_chunks():
    T, H, D, L, rows = 700, 2, 16, 4, 100   # rows < T: the clamp; chunks of 256
    v = torch.from_numpy(RNG.standard_normal((T, H, D))).half()
    p = torch.from_numpy(np.sort(RNG.standard_normal((H, rows, L)), -1)).half()
    up = torch.from_numpy(RNG.uniform(0.5, 2.0, (H, rows))).half()
    codes, mask, deq = R.nuq_round_trip(v, p, up, -up, True, chunk=256)
    r = np.minimum(np.arange(T), rows - 1)
    pg = p.numpy()[:, r].transpose(1, 0, 2)[:, :, None, :]          # (T, H, 1, L)
    wc, wrecon, wmask = O.nuq_py_semantics(v.numpy(), np.broadcast_to(pg, (T, H, D, L)),
                                           up.numpy()[:, r].T[..., None],
                                           (-up).numpy()[:, r].T[..., None])
    assert np.array_equal(codes.numpy(), wc)
    assert np.array_equal(mask.numpy(), wmask)
    assert np.array_equal(deq.numpy(), wrecon)


@pytest.mark.parametrize("bits", [2, 4])
def test_pack_codes_csr_matches_oracle(bits):
    T, H, D = 50, 4, 32
    codes = RNG.integers(0, 1 << bits, (T, H, D)).astype(np.uint8)
    mask = RNG.random((T, H, D)) < 0.1
    vals = RNG.standard_normal((T, H, D)).astype(np.float16)
    got = R.pack_codes_csr(codes, mask, vals, bits)
    outv = np.where(mask, vals.view(np.uint16), 0).astype(np.uint16)
    want = O.pack_compact(codes, outv, mask.astype(np.uint8), bits)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_quest_leg_matches_oracle():
    P, S, H, D, group = 300, 16, 4, 64, 7
    K = torch.from_numpy(RNG.standard_normal((P, S, H, D)).astype(np.float32))
    mn, mx = R.compute_page_stats(K)
    wmn, wmx = O.page_stats(K.numpy())
    assert np.array_equal(mn.numpy(), wmn) and np.array_equal(mx.numpy(), wmx)
    q = torch.from_numpy(RNG.standard_normal((H * group, D)).astype(np.float32))
    b = R.page_upper_bound_group(q, mn, mx, group)
    wb = O.page_bound_group(q.numpy(), wmn, wmx, group)
    # fp32 sums in torch's order vs the oracle's canonical order
    assert np.allclose(b.numpy(), wb, rtol=1e-5, atol=1e-4)
    sel = R.topk_pages_with_sinks(torch.from_numpy(wb), 50, 4)   # distinct keys: ties impossible
    assert np.array_equal(sel.numpy(), O.topk_sinks(wb, 50, 4))
    one = R.page_upper_bound(q[:H], mn, mx)
    assert np.allclose(one.numpy(), O.page_bound(q[:H].numpy(), wmn, wmx), rtol=1e-5, atol=1e-4)
