"""The drop-in Quest functions with fp16 inputs against the reference's own
fp16 op sequence (restated in oracle/torch_ref.py, run with torch on the
CPU).

The drop-ins fix their arithmetic (quest/reference.py docstring): the bound
sums exact products in fp32 and rounds once, where the reference rounds every
fp16 product and each of the two partial sums (src/quest/reference.py:91-92);
selected_attention keeps scores and probabilities in fp32, where the
reference rounds the scores to fp16 and casts the fp32 softmax back to fp16
before the value product (:165-167).  These tests bound the difference:

* bound: |ours - reference| <= 2^-11 * sum_d |q_d| max(|min_d|, |max_d|)
  (one fp16 rounding of every product) + 2 fp16 ulps of the bound (the two
  partial-sum roundings and the final add), for every page and head; the
  top-K page sets agree except for pages whose bound lies within that
  tolerance of the K-th largest;
* attention: relative L2 error per head <= 1e-3 (the tolerance the path is
  held to for fp16 attention outputs), against the reference's fp16
  sequence, with both also checked against a float64 evaluation.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import torch_ref as R

pytestmark = pytest.mark.gpu


def _ulp16(x: torch.Tensor) -> torch.Tensor:
    """Spacing of fp16 at |x| (subnormal spacing near zero)."""
    a = x.abs().float().clamp(min=2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(a)) - 10)


@pytest.mark.parametrize("P,H,D,seed", [(4096, 4, 128, 0), (1000, 8, 64, 1), (65536, 4, 128, 2)])
def test_page_upper_bound_fp16_vs_reference_sequence(dev, P, H, D, seed):
    from quest import page_upper_bound, topk_pages_with_sinks

    g = torch.Generator().manual_seed(seed)
    q = torch.randn((H, D), generator=g).half()
    kmin = torch.randn((P, H, D), generator=g).half()
    kmax = (kmin.float() + torch.rand((P, H, D), generator=g) * 2).half()
    ref = R.page_upper_bound(q, kmin, kmax)  # fp16 products, fp32-accumulated sums, fp16 add
    assert ref.dtype == torch.float16
    ours = page_upper_bound(q.to(dev), kmin.to(dev), kmax.to(dev)).cpu()
    assert ours.dtype == torch.float16
    mag = (q.float().abs()[None] * torch.maximum(kmin.float().abs(), kmax.float().abs())).sum(-1)
    tol = mag * 2.0 ** -11 + 2 * _ulp16(ref)
    diff = (ours.float() - ref.float()).abs()
    assert (diff <= tol).all(), f"max excess {(diff - tol).max().item()}"
    assert (diff > 0).any() or P < 2000  # the two roundings do differ on real data
    # top-K: the sets agree away from the threshold
    k = P // 4
    s_ours = topk_pages_with_sinks(ours.to(dev), k, 4).cpu()
    s_ref = R.topk_pages_with_sinks(ref, k, 4)
    for h in range(H):
        a, b = set(s_ours[:, h].tolist()), set(s_ref[:, h].tolist())
        kth = torch.sort(ref[4:, h].float(), descending=True).values[k - 1]
        for p in a ^ b:
            assert abs(ref[p, h].float() - kth) <= 2 * tol[p, h], (h, p)


@pytest.mark.parametrize("H,Hv,D,sel,seed", [(4, 4, 128, 68, 0), (8, 2, 64, 40, 1)])
def test_selected_attention_fp16_vs_reference_sequence(dev, H, Hv, D, sel, seed):
    from quest import selected_attention

    g = torch.Generator().manual_seed(seed)
    P, S = 300, 16
    q = torch.randn((H, D), generator=g).half()
    K = torch.randn((P, S, H, D), generator=g).half()
    V = torch.randn((P, S, Hv, D), generator=g).half()
    idx = torch.stack([torch.randperm(P, generator=g)[:sel].sort().values for _ in range(H)], dim=1)
    ref = R.selected_attention(q, K, V, idx)
    ours = selected_attention(q.to(dev), K.to(dev), V.to(dev), idx.to(dev)).cpu()
    assert ours.dtype == torch.float16
    exact = R.selected_attention(q.double(), K.double(), V.double(), idx)
    for h in range(H):
        e = exact[h]
        r_ours = ((ours[h].double() - e).norm() / e.norm()).item()
        r_ref = ((ref[h].double() - e).norm() / e.norm()).item()
        r_pair = ((ours[h].double() - ref[h].double()).norm() / ref[h].double().norm()).item()
        assert r_pair <= 1e-3, (h, r_pair)
        assert r_ours <= 1e-3 and r_ref <= 1e-3, (h, r_ours, r_ref)
