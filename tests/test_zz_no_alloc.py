"""The allocation-free Quest selection (hkv_quest_select_noalloc), called
through the C ABI: bit-identical indices and scores to hkv_quest_select with
a caller workspace, on calls in a row (the second with a smaller input), and
a clean rejection of a problem larger than its fixed scratch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, P, H, group, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn((H * group, 128), generator=g).half().to(dev)
    mn = torch.randn((P, H, 128), generator=g).half()
    mx = (mn.float() + torch.rand((P, H, 128), generator=g)).half()
    return q, mn.to(dev), mx.to(dev)


def _select(N, q, mn, mx, k, sinks, noalloc):
    P, H, D = (int(x) for x in mn.shape)
    s = max(0, min(sinks, P))
    keff = max(0, min(k, P - s))
    out = torch.full((s + keff, H), -7, dtype=torch.int64, device=q.device)
    scores = torch.full((H, P), float("nan"), dtype=torch.float32, device=q.device)
    n_out = ctypes.c_int64(-1)
    st = N.stream_of(q)
    if noalloc:
        rc = N.lib().hkv_quest_select_noalloc(N.ptr(q), N.DT_F16, int(q.shape[0]), N.ptr(mn),
                                              N.ptr(mx), N.DT_F16, P, H, D, k, sinks, N.ptr(scores),
                                              N.ptr(out), n_out, st)
    else:
        nb = int(N.lib().hkv_quest_select_workspace_bytes(P, H))
        ws = torch.zeros(nb, dtype=torch.uint8, device=q.device)
        rc = N.lib().hkv_quest_select(N.ptr(q), N.DT_F16, int(q.shape[0]), N.ptr(mn), N.ptr(mx),
                                      N.DT_F16, P, H, D, k, sinks, N.ptr(scores), N.ptr(out), n_out,
                                      N.ptr(ws), nb, st)
    assert rc == 0, N.lib().hkv_status_string(rc)
    assert n_out.value == s + keff
    torch.cuda.synchronize()
    return out.cpu(), scores.cpu()


def test_noalloc_select_matches_workspace_select(dev):
    from helix_kv import _native as N

    # 65,536 pages (the 1M-token case), then fewer pages (fewer histogram
    # slices in the same scratch), then ties everywhere, then a larger problem
    cases = [(65536, 4, 7, 16384, 4, 1), (40000, 4, 7, 10000, 4, 2), (33000, 2, 1, 500, 0, 3),
             (600000, 4, 7, 150000, 4, 4)]
    for P, H, group, k, sinks, seed in cases:
        q, mn, mx = _inputs(dev, P, H, group, seed)
        if seed == 3:   # constant statistics: every bound ties
            mn.fill_(0.25)
            mx.fill_(0.5)
        want = _select(N, q, mn, mx, k, sinks, noalloc=False)
        got = _select(N, q, mn, mx, k, sinks, noalloc=True)
        assert torch.equal(got[0], want[0]), (P, H)
        assert torch.equal(got[1].view(torch.int32), want[1].view(torch.int32)), (P, H)
    # repeat the first case: the scratch was left reusable
    q, mn, mx = _inputs(dev, 65536, 4, 7, 1)
    again = _select(N, q, mn, mx, 16384, 4, noalloc=True)
    want = _select(N, q, mn, mx, 16384, 4, noalloc=False)
    assert torch.equal(again[0], want[0])


def test_noalloc_select_rejects_problems_beyond_its_scratch(dev):
    from helix_kv import _native as N

    L = N.lib()
    cap = int(L.hkv_quest_select_noalloc_max_workspace())
    assert cap == 8 << 20
    P, H = 2_000_000, 64
    assert int(L.hkv_quest_select_workspace_bytes(P, H)) > cap
    tiny = torch.zeros(16, dtype=torch.float16, device=dev)
    n_out = ctypes.c_int64(-1)
    rc = L.hkv_quest_select_noalloc(N.ptr(tiny), N.DT_F16, H, N.ptr(tiny), N.ptr(tiny), N.DT_F16,
                                    P, H, 128, 10, 4, N.ptr(tiny), N.ptr(tiny), n_out,
                                    N.stream_of(tiny))
    assert rc == N.HKV_ERR_SCRATCH
    assert b"scratch" in L.hkv_status_string(rc)
    torch.cuda.synchronize()
