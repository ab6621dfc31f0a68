"""The reference's PyTorch CPU path for the KV-cache hot path, restated with the
same torch op sequence, for the CPU baseline that the benchmark reports beside
the GPU figures.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): only ``tests/`` and the
``cpu_baseline`` leg of ``bench.py`` import this module, as the thing the CPU
is timed on -- never as part of the product.

Two legs:
  - nuq: find_outliers + round_to_nearest_pole + where (quantize_nuq), then
    dequantize_nuq, over fp16 K (per-channel scales) and V (per-token scales,
    the clamped pole rows pre-gathered as the vLLM backend does), chunked by
    tokens to bound the (..., L) temporaries; the bit-pack + CSR step, which
    the reference lacks, in numpy (``pack_codes_csr``), timed apart;
  - Quest: compute_page_stats + page_upper_bound + topk_pages_with_sinks.

Citations are relative to the reference checkout.
"""
from __future__ import annotations

import numpy as np
import torch


# --------------------------------------------------------------------- nuq

def find_outliers(values, upper, lower):
    """Strict compares: values < lower | values > upper.  src/kvquant/nuq.py:72."""
    return (values < lower) | (values > upper)


def round_to_nearest_pole(values, poles):
    """(reconstructed, codes): |v - pole| in the promoted dtype, first argmin,
    gather.  src/kvquant/nuq.py:36-38 (the codes are the argmin it computes;
    the reference's callers recompute them the same way,
    src/kvquant/tests/test_nuq_roundtrip.py:89-90)."""
    diff = (values.unsqueeze(-1) - poles).abs()
    idx = diff.argmin(dim=-1)
    return torch.gather(poles, -1, idx.unsqueeze(-1)).squeeze(-1), idx


def quantize_nuq(values, poles, upper, lower):
    """(reconstructed, outlier_mask, codes).  src/kvquant/nuq.py:97-132 without
    the cap / first-N options."""
    mask = find_outliers(values, upper, lower)
    q, idx = round_to_nearest_pole(values, poles)
    return torch.where(mask, values, q), mask, idx


def dequantize_nuq(codes, outliers, outlier_mask, poles):
    """where(mask, outliers, poles[code]).  src/kvquant/nuq.py:135-156."""
    rec = torch.gather(poles, -1, codes.unsqueeze(-1)).squeeze(-1)
    return torch.where(outlier_mask, outliers, rec.to(outliers.dtype))


def v_pole_rows(poles, upper, lower, t0: int, t1: int):
    """Per-token scales of tokens [t0, t1) pre-gathered at row min(t, rows-1)
    and laid out to broadcast against (T, H, D) values: poles (T, H, 1, L),
    thresholds (T, H, 1).  src/kvquant/vllm_backend.py:151-155."""
    rows = int(poles.shape[1])
    r = torch.arange(t0, t1).clamp(max=rows - 1)
    return (poles[:, r].permute(1, 0, 2).unsqueeze(2), upper[:, r].T.unsqueeze(-1),
            lower[:, r].T.unsqueeze(-1))


def nuq_round_trip(values, poles, upper, lower, per_token: bool, chunk: int = 8192):
    """Quantise then dequantise (T, H, D) fp16 in chunks of `chunk` tokens.
    Returns (codes u8 (T,H,D), outlier mask (T,H,D), dequantised (T,H,D))."""
    T = int(values.shape[0])
    codes = torch.empty(values.shape, dtype=torch.uint8)
    mask = torch.empty(values.shape, dtype=torch.bool)
    deq = torch.empty_like(values)
    for t0 in range(0, T, chunk):
        t1 = min(T, t0 + chunk)
        v = values[t0:t1]
        if per_token:
            p, up, lo = v_pole_rows(poles, upper, lower, t0, t1)
            p = p.expand(t1 - t0, v.shape[1], v.shape[2], p.shape[-1])
        else:
            p, up, lo = poles, upper, lower
            p = p.expand(t1 - t0, *p.shape)
        _, m, idx = quantize_nuq(v, p, up, lo)
        outl = torch.where(m, v, torch.zeros_like(v))
        deq[t0:t1] = dequantize_nuq(idx, outl, m, p)
        codes[t0:t1] = idx.to(torch.uint8)
        mask[t0:t1] = m
    return codes, mask, deq


def pack_codes_csr(codes: np.ndarray, mask: np.ndarray, values: np.ndarray, bits: int):
    """The bit-pack + CSR step in numpy (the reference has none): packed
    codes (T,H,D*bits/8), row_ptr (T*H+1) int32, col u8, val fp16 bits, in
    the build's compact format (little-endian codes within a byte, rows
    t*H+h, columns ascending)."""
    T, H, D = codes.shape
    per = 8 // bits
    c = codes.reshape(T, H, D // per, per).astype(np.uint8)
    packed = np.zeros((T, H, D // per), np.uint8)
    for j in range(per):
        packed |= (c[..., j] & ((1 << bits) - 1)) << (bits * j)
    m2 = mask.reshape(T * H, D)
    row_ptr = np.zeros(T * H + 1, np.int64)
    np.cumsum(m2.sum(axis=1), out=row_ptr[1:])
    r, col = np.nonzero(m2)
    val = values.reshape(T * H, D).view(np.uint16)[r, col]
    return packed, row_ptr.astype(np.int32), col.astype(np.uint8), val


# ------------------------------------------------------------------- Quest

def compute_page_stats(K_pages):
    """amin / amax over the page-slot dim.  src/quest/reference.py:38-56."""
    return K_pages.amin(dim=1), K_pages.amax(dim=1)


def page_upper_bound(query, K_min, K_max):
    """sum_d clamp(q,0)*max + clamp(q,max=0)*min in the inputs' dtype.
    src/quest/reference.py:59-93."""
    q_pos = query.clamp(min=0)
    q_neg = query.clamp(max=0)
    return (q_pos.unsqueeze(0) * K_max).sum(dim=-1) + (q_neg.unsqueeze(0) * K_min).sum(dim=-1)


def page_upper_bound_group(query, K_min, K_max, group: int):
    """The group-summed bound of the Quest benchmark configuration: query
    (H * group, D), query head j of KV head h at row h * group + j; the
    reference function evaluated once per position in the group, summed."""
    H = int(K_min.shape[1])
    qg = query.view(H, group, -1)
    out = page_upper_bound(qg[:, 0], K_min, K_max)
    for j in range(1, group):
        out = out + page_upper_bound(qg[:, j], K_min, K_max)
    return out


def topk_pages_with_sinks(bound, k: int, sink_pages: int = 1):
    """Sinks, then torch.topk over dim 0 of the masked bound, sorted per head.
    src/quest/reference.py:96-133."""
    P, H = bound.shape
    sink_pages = max(0, min(sink_pages, P))
    k_eff = max(0, min(k, P - sink_pages))
    sink_idx = torch.arange(sink_pages).unsqueeze(1).expand(-1, H)
    if k_eff == 0:
        return sink_idx
    masked = bound.clone()
    masked[:sink_pages, :] = float("-inf")
    top = torch.topk(masked, k=k_eff, dim=0)
    selected = torch.cat([sink_idx, top.indices], dim=0)
    return selected.sort(dim=0).values


def selected_attention(query, K_pages, V_pages, page_indices):
    """Per head h: scores = (K_h @ q_h) * D^-0.5 in the query's dtype, fp32
    softmax cast back to the query's dtype, then attn @ V_{h % H_v}.
    src/quest/reference.py:136-168 (same op sequence, same dtypes)."""
    import math

    P, page_size, H, D = K_pages.shape
    Hv, Dv = V_pages.shape[2], V_pages.shape[3]
    n = page_indices.shape[0]
    out = torch.zeros(H, Dv, dtype=query.dtype)
    scale = 1.0 / math.sqrt(D)
    for h in range(H):
        idx = page_indices[:, h]
        Kh = K_pages[idx, :, h, :].reshape(n * page_size, D)
        Vh = V_pages[idx, :, h % Hv, :].reshape(n * page_size, Dv)
        scores = (Kh @ query[h]) * scale
        attn = torch.softmax(scores.float(), dim=0).to(query.dtype)
        out[h] = attn @ Vh
    return out
