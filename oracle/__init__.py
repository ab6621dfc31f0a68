"""CPU oracle for helix-lite's KV-cache hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker -- never as the thing measured or shipped.  The product (the HIP
library under ``helix-lite_amd/csrc`` and the drop-in Python packages) never
imports it and has no CPU fallback.

The integer/byte semantics live in ``oracle.c`` (built to ``liboracle.so`` by
``oracle/Makefile``); this module wraps it with numpy and adds the byte-format
helpers (bit packing, CSR) and the attention reference in float64.

Reference files are cited as ``file:line`` relative to the reference checkout.
Every function here is pinned by at least one test in ``tests/test_oracle_*.py``
against the reference's own known answers, torch library routines, or
exhaustive enumeration; see each docstring.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_lib = None


def build(force: bool = False) -> Path:
    """Compile ``liboracle.so`` with the committed Makefile."""
    if force or not _LIB_PATH.exists() or (
        _LIB_PATH.stat().st_mtime < (_HERE / "oracle.c").stat().st_mtime
    ):
        subprocess.run(["make", "-s", "-B" if force else "liboracle.so"], cwd=_HERE, check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        build()
        _lib = ctypes.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int


def _declare(L: ctypes.CDLL) -> None:
    L.orc_nearest_code.argtypes = [ctypes.c_float, _p, _i32]
    L.orc_nearest_code.restype = _i32
    L.orc_pack_k.argtypes = [_p, _i64, _i32, _i32, _p, _p, _p, _i32, _p, _p, _p]
    L.orc_pack_v.argtypes = [_p, _i64, _i32, _i32, _p, _p, _p, _i32, _i64, _p, _p, _p, _p]
    L.orc_unpack.argtypes = [_p, _p, _p, _i64, _i32, _i32, _p, _i32, _i32, _i64, _p, _p]
    L.orc_prep_tables.argtypes = [_p, _p, _p, _i64, _i32, _p]
    L.orc_check_table_exhaustive.argtypes = [_p, _i32, ctypes.c_float, ctypes.c_float,
                                             ctypes.POINTER(_i64)]
    L.orc_check_table_exhaustive.restype = _i64
    L.orc_page_stats.argtypes = [_p, _i64, _i32, _i32, _i32, _p, _p]
    L.orc_page_bound.argtypes = [_p, _p, _p, _i64, _i32, _i32, _p]
    L.orc_page_bound_group.argtypes = [_p, _p, _p, _i64, _i32, _i32, _i32, _p]
    L.orc_topk_sinks.argtypes = [_p, _i64, _i32, _i64, _i64, _p]
    L.orc_topk_sinks.restype = _i64
    L.orc_kmeans_dp.argtypes = [_p, _i64, _i32, _p]
    L.orc_kmeans_dp.restype = _i32


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _h16(a) -> np.ndarray:
    """fp16 values as a contiguous uint16 bit array."""
    a = np.asarray(a)
    if a.dtype == np.uint16:
        return np.ascontiguousarray(a)
    return np.ascontiguousarray(a.astype(np.float16)).view(np.uint16)


# Table record layout shared with the GPU tables (80 bytes, see oracle.c).
TABLE_DTYPE = np.dtype([
    ("bp", np.uint16, 16), ("pf16", np.uint16, 16), ("lo", np.uint16), ("up", np.uint16),
    ("xsafe", np.uint16), ("flags", np.uint16), ("levels", np.uint16), ("pad", np.uint16, 3),
])
assert TABLE_DTYPE.itemsize == 80


# --------------------------------------------------------------- nuq (a1-a6)

def nearest_code(v: float, poles) -> int:
    """Strict-< ascending scan over fp32 |v - pole| (src/kvquant/triton_batched.py:65-72)."""
    p = _f32(poles)
    return int(lib().orc_nearest_code(ctypes.c_float(float(np.float32(v))), _ptr(p), p.size))


def pack_k(values, poles, upper, lower):
    """K per-channel pack, dense outliers (src/kvquant/triton_batched.py:28-82).

    values (T,H,D) fp16; poles (H,D,L); upper/lower (H,D).  Returns
    (codes u8, outlier_v fp16-bits u16, outlier_m u8), each (T,H,D).
    """
    x = _h16(values)
    T, H, D = x.shape
    p, up, lo = _f32(poles), _f32(upper), _f32(lower)
    L = p.shape[-1]
    assert p.shape == (H, D, L) and up.shape == (H, D) and lo.shape == (H, D)
    codes = np.empty((T, H, D), np.uint8)
    outv = np.empty((T, H, D), np.uint16)
    outm = np.empty((T, H, D), np.uint8)
    lib().orc_pack_k(_ptr(x), T, H, D, _ptr(p), _ptr(up), _ptr(lo), L, _ptr(codes),
                     _ptr(outv), _ptr(outm))
    return codes, outv, outm


def pack_v(values, poles, upper, lower, positions=None):
    """V per-token pack, dense outliers.

    poles (H,Tt,L), upper/lower (H,Tt); row t uses scale row
    min(positions[t], Tt-1) (positions default to arange(T)).
    src/kvquant/triton_batched.py:179-232; clamp src/kvquant/compact_pool.py:467.
    """
    x = _h16(values)
    T, H, D = x.shape
    p, up, lo = _f32(poles), _f32(upper), _f32(lower)
    L = p.shape[-1]
    Tt = p.shape[1]
    assert p.shape == (H, Tt, L) and up.shape == (H, Tt) and lo.shape == (H, Tt)
    pos = None if positions is None else np.ascontiguousarray(np.asarray(positions, np.int64))
    codes = np.empty((T, H, D), np.uint8)
    outv = np.empty((T, H, D), np.uint16)
    outm = np.empty((T, H, D), np.uint8)
    lib().orc_pack_v(_ptr(x), T, H, D, _ptr(p), _ptr(up), _ptr(lo), L, Tt, _ptr(pos),
                     _ptr(codes), _ptr(outv), _ptr(outm))
    return codes, outv, outm


def unpack(codes, outv, outm, poles, mode: str, positions=None):
    """where(outlier_m, outlier_v, fp16(pole[code])) -> fp16 bits (T,H,D).

    mode "k": poles (H,D,L); mode "v": poles (H,Tt,L) with the clamp above.
    src/kvquant/triton_batched.py:85-122, :235-272; src/kvquant/nuq.py:155-156.
    """
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    v = _h16(outv)
    m = np.ascontiguousarray(outm, dtype=np.uint8)
    T, H, D = c.shape
    p = _f32(poles)
    L = p.shape[-1]
    Tt = p.shape[1] if mode == "v" else 0
    pos = None if positions is None else np.ascontiguousarray(np.asarray(positions, np.int64))
    out = np.empty((T, H, D), np.uint16)
    lib().orc_unpack(_ptr(c), _ptr(v), _ptr(m), T, H, D, _ptr(p), L, 0 if mode == "k" else 1,
                     Tt, _ptr(pos), _ptr(out))
    return out


def nuq_py_semantics(values, poles, upper, lower):
    """``quantize_nuq`` exactly as src/kvquant/nuq.py:36-38,72,131 computes it.

    The difference ``values - poles`` is formed in torch's promoted dtype: for
    fp16 inputs and fp16 poles the fp32 difference is rounded to fp16 before
    ``abs`` and ``argmin`` (first index on ties).  Returns (codes, recon, mask)
    with recon in the promoted dtype.  Broadcasting follows numpy rules.
    """
    v = np.asarray(values)
    p = np.asarray(poles)
    dt = np.result_type(v.dtype, p.dtype)
    diff = (v.astype(np.float32)[..., None] - p.astype(np.float32)).astype(dt)
    codes = np.abs(diff).argmin(axis=-1)
    q = np.take_along_axis(np.broadcast_to(p, codes.shape + (p.shape[-1],)),
                           codes[..., None], axis=-1)[..., 0].astype(dt)
    mask = (v < np.asarray(lower)) | (v > np.asarray(upper))
    recon = np.where(mask, v.astype(dt), q)
    return codes, recon, mask


# ----------------------------------------------------- fast decision tables

def prep_tables(poles, upper, lower) -> np.ndarray:
    """Decision tables (TABLE_DTYPE records) for poles (N,L), thresholds (N,)."""
    p, up, lo = _f32(poles), _f32(upper), _f32(lower)
    n, L = p.shape
    out = np.zeros(n, TABLE_DTYPE)
    lib().orc_prep_tables(_ptr(p), _ptr(up), _ptr(lo), n, L, _ptr(out))
    return out


def check_table_exhaustive(poles, upper: float, lower: float) -> tuple[int, int]:
    """(mismatches, covered inputs) of the fast path over all 65,536 fp16 inputs."""
    p = _f32(poles)
    cov = _i64(0)
    bad = lib().orc_check_table_exhaustive(_ptr(p), p.size, ctypes.c_float(upper),
                                           ctypes.c_float(lower), ctypes.byref(cov))
    return int(bad), int(cov.value)


# ---------------------------------------------- a5: bit packing and CSR

def bitpack(codes, bits: int) -> np.ndarray:
    """Pack codes (..., D) into little-endian bytes (..., D*bits/8).

    nuq4: byte j = c[2j] | c[2j+1] << 4; nuq2: byte j = c[4j] | c[4j+1] << 2 |
    c[4j+2] << 4 | c[4j+3] << 6.  (Format of this build; the reference stores
    one byte per code, src/kvquant/compact_pool.py:427-432.)
    """
    c = np.asarray(codes, dtype=np.uint8)
    per = 8 // bits
    assert c.shape[-1] % per == 0
    c = c.reshape(c.shape[:-1] + (c.shape[-1] // per, per)).astype(np.uint16)
    out = np.zeros(c.shape[:-1], np.uint16)
    for j in range(per):
        out |= (c[..., j] & ((1 << bits) - 1)) << (bits * j)
    return out.astype(np.uint8)


def bitunpack(packed, bits: int, D: int) -> np.ndarray:
    b = np.asarray(packed, dtype=np.uint8)
    per = 8 // bits
    out = np.empty(b.shape + (per,), np.uint8)
    for j in range(per):
        out[..., j] = (b >> (bits * j)) & ((1 << bits) - 1)
    return out.reshape(b.shape[:-1] + (D,))


def csr_encode(outm, outv):
    """Dense (R,D) outlier mask/values -> CSR (row_ptr int32 (R+1,), col u8, val fp16 bits).

    Rows are the flattened (token, head) rows; within a row columns ascend.
    """
    m = np.asarray(outm).astype(bool)
    R = m.shape[0]
    m2 = m.reshape(R, -1)
    v2 = _h16(outv).reshape(R, -1)
    counts = m2.sum(axis=1)
    row_ptr = np.zeros(R + 1, np.int64)
    np.cumsum(counts, out=row_ptr[1:])
    r, c = np.nonzero(m2)
    return row_ptr.astype(np.int32), c.astype(np.uint8), v2[r, c]


def csr_decode(row_ptr, col, val, R: int, D: int):
    m = np.zeros((R, D), np.uint8)
    v = np.zeros((R, D), np.uint16)
    rp = np.asarray(row_ptr, np.int64)
    rows = np.repeat(np.arange(R), np.diff(rp))
    m[rows, np.asarray(col, np.int64)] = 1
    v[rows, np.asarray(col, np.int64)] = np.asarray(val, np.uint16)
    return m, v


def pack_compact(codes, outv, outm, bits: int):
    """Dense (T,H,D) pack outputs -> (packed codes (T,H,D*bits/8), row_ptr, col, val)."""
    T, H, D = np.asarray(codes).shape
    rp, col, val = csr_encode(np.asarray(outm).reshape(T * H, D), np.asarray(outv).reshape(T * H, D))
    return bitpack(codes, bits), rp, col, val


# ------------------------------------------------------------ Quest a8-a11

def page_stats(K_pages):
    """(P,S,H,D) -> (min, max) (P,H,D) in K's dtype; -0 < +0; NaN propagates.

    src/quest/reference.py:38-56.
    """
    K = np.asarray(K_pages)
    P, S, H, D = K.shape
    k32 = _f32(K)
    mn = np.empty((P, H, D), np.float32)
    mx = np.empty((P, H, D), np.float32)
    lib().orc_page_stats(_ptr(k32), P, S, H, D, _ptr(mn), _ptr(mx))
    return mn.astype(K.dtype), mx.astype(K.dtype)


def page_bound(query, kmin, kmax):
    """(H,D) query, (P,H,D) stats -> (P,H) fp32 bound in the canonical order.

    src/quest/reference.py:59-93, src/quest/triton_kernels.py:25-57.
    """
    q, mn, mx = _f32(query), _f32(kmin), _f32(kmax)
    P, H, D = mn.shape
    out = np.empty((P, H), np.float32)
    lib().orc_page_bound(_ptr(q), _ptr(mn), _ptr(mx), P, H, D, _ptr(out))
    return out


def page_bound_group(query, kmin, kmax, group: int):
    """(Hq,D) query with Hq = Hkv*group -> (P,Hkv) group-sum bound (factorised order)."""
    q, mn, mx = _f32(query), _f32(kmin), _f32(kmax)
    P, H, D = mn.shape
    assert q.shape == (H * group, D)
    out = np.empty((P, H), np.float32)
    lib().orc_page_bound_group(_ptr(q), _ptr(mn), _ptr(mx), P, H, group, D, _ptr(out))
    return out


def _u8_deq(q, lo, step):
    """lo + q * step in float32, two roundings (the device's order)."""
    return (np.float32(lo) + (np.asarray(q).astype(np.float32) * np.float32(step)).astype(np.float32)).astype(np.float32)


def page_stats_u8(kmin, kmax):
    """Compact page metadata: (P,H,D) min/max -> (qmin u8, qmax u8, lo f32 (H,D), step f32 (H,D)).

    No counterpart in the reference, whose pool keeps fp32 page statistics
    (src/kvquant/compact_pool.py:434-441; the bound they feed is
    src/quest/reference.py:59-93).  Per (head, channel), over the finite
    statistics of all pages: lo = the smallest, hi = the largest;
    step = fl((hi - lo) / 255), raised one ulp at a time (at most 16) until
    deq(255) >= hi, where deq(q) = fl(lo + fl(q * step)) (step = 1 when
    hi <= lo or no statistic is finite, lo = 0 then).  A minimum x codes as
    floor(fl(fl(x - lo) / step)) clamped to [0, 255] and lowered (at most 4
    times, then 0) while deq(q) > x; a maximum as the ceiling, raised (at
    most 4 times, then 255) while deq(q) < x.  So deq(qmin) <= min and
    deq(qmax) >= max for every finite statistic: the bound computed from
    the dequantised statistics is never below the one from the originals.
    A non-finite statistic codes as 0 (minimum) / 255 (maximum).
    """
    mn, mx = _f32(kmin), _f32(kmax)
    P, H, D = mn.shape
    allv = np.concatenate([mn, mx], 0)
    fin = np.isfinite(allv)
    lo = np.where(fin, allv, np.inf).min(0).astype(np.float32)
    hi = np.where(fin, allv, -np.inf).max(0).astype(np.float32)
    none = ~np.isfinite(lo)
    lo = (np.where(none, np.float32(0), lo) + np.float32(0)).astype(np.float32)  # -0 -> +0
    hi = (np.where(none, np.float32(0), hi) + np.float32(0)).astype(np.float32)
    wide = hi > lo
    step = np.where(wide, ((hi - lo).astype(np.float32) / np.float32(255)).astype(np.float32),
                    np.float32(1)).astype(np.float32)
    for _ in range(16):
        short = wide & (_u8_deq(255, lo, step) < hi)
        if not short.any():
            break
        step = np.where(short, (step.view(np.uint32) + np.uint32(1)).view(np.float32), step)

    def code(x, up):
        t = ((x - lo).astype(np.float32) / step).astype(np.float32)
        t = np.ceil(t) if up else np.floor(t)
        q = np.clip(np.nan_to_num(t, nan=0.0, posinf=255.0, neginf=0.0), 0, 255).astype(np.int32)
        for _ in range(4):
            d = _u8_deq(q, lo, step)
            if up:
                q = np.where((q < 255) & (d < x), q + 1, q)
            else:
                q = np.where((q > 0) & (d > x), q - 1, q)
        d = _u8_deq(q, lo, step)
        q = np.where(up & (d < x), 255, q) if up else np.where(d > x, 0, q)
        q = np.where(np.isfinite(x), q, 255 if up else 0)
        return q.astype(np.uint8)

    return code(mn, False), code(mx, True), lo, step


def page_stats_u8_deq(qmin, qmax, lo, step):
    """The float32 statistics the bound reads from the compact metadata."""
    return _u8_deq(qmin, lo, step), _u8_deq(qmax, lo, step)


def topk_sinks(bound, k: int, sink_pages: int):
    """src/quest/reference.py:96-133 with lowest-index tie-break -> (s+k_eff, H) int64."""
    b = _f32(bound)
    P, H = b.shape
    s = max(0, min(sink_pages, P))
    keff = max(0, min(k, P - s))
    out = np.empty((s + keff, H), np.int64)
    lib().orc_topk_sinks(_ptr(b), P, H, k, sink_pages, _ptr(out))
    return out


def select_union(bound, used_block_ids, top_k: int, sink_blocks: int, block_size: int):
    """src/kvquant/quest_selector.py:38-90: union over heads, mapped to block ids, sorted."""
    used = np.asarray(used_block_ids, np.int64)
    NU = used.shape[0]
    sinks = max(0, min(sink_blocks, NU))
    keep = max(0, min(top_k, NU - sinks))
    sel = topk_sinks(bound, keep, sinks)
    uniq = np.unique(sel.reshape(-1))
    ids = np.sort(used[uniq])
    return ids, ids * block_size


def selected_attention(query, K_pages, V_pages, page_indices, kv_of_head, num_tokens=None,
                       scale=None):
    """softmax(q.K^T * scale).V over each head's selected pages, in float64.

    query (Hq,D); K_pages/V_pages (P,S,Hkv,D); page_indices (n,Hsel) where
    column j selects pages for KV head j (Hsel == Hkv) or for query head j
    (Hsel == Hq); kv_of_head(h) maps a query head to its KV head.  Slots of
    token index >= num_tokens (page * S + slot) are masked out, and so are page
    ids outside [0, P); scale defaults to 1/sqrt(D).
    src/quest/reference.py:136-168 (fp32 softmax there; float64 here, compared
    with a tolerance).
    """
    q = np.asarray(query, np.float64)
    K = np.asarray(K_pages, np.float64)
    V = np.asarray(V_pages, np.float64)
    idx = np.asarray(page_indices, np.int64)
    Hq, D = q.shape
    P, S = K.shape[0], K.shape[1]
    sc = 1.0 / np.sqrt(D) if scale is None else float(scale)
    ntok = P * S if num_tokens is None else int(num_tokens)
    out = np.zeros((Hq, V.shape[-1]))
    for h in range(Hq):
        g = kv_of_head(h)
        col = idx[:, h] if idx.shape[1] == Hq else idx[:, g]
        col = col[(col >= 0) & (col < P)]
        tok = (col[:, None] * S + np.arange(S)[None, :]).reshape(-1)
        keep = tok < ntok
        Kh = K[col, :, g, :].reshape(-1, D)[keep]
        Vh = V[col, :, g, :].reshape(-1, V.shape[-1])[keep]
        if Kh.shape[0] == 0:
            continue
        s = Kh @ q[h] * sc
        s = np.exp(s - s.max())
        out[h] = (s / s.sum()) @ Vh
    return out


def select_ragged(query, kmin, kmax, page_offsets, top_k, sink_pages: int):
    """Per-sequence Quest selection over a ragged batch: sequence b owns pages
    [page_offsets[b], page_offsets[b+1]) of the statistics and query query[b]
    (Hq, D); group-summed bound + topk_sinks per sequence (the per-sequence
    restatement of src/quest/reference.py:59-133, src/kvquant/quest_selector.py:
    64-78).  Returns (sel (rows, H) local indices, out_offsets (B+1,),
    scores (H, P_total))."""
    q = _f32(query)
    mn, mx = _f32(kmin), _f32(kmax)
    B, Hq, D = q.shape
    Ptot, H, _ = mn.shape
    sels, outs, scores = [], [0], np.zeros((H, Ptot), np.float32)
    for b in range(B):
        o0, o1 = int(page_offsets[b]), int(page_offsets[b + 1])
        if o1 > o0:
            bound = page_bound_group(q[b], mn[o0:o1], mx[o0:o1], Hq // H)
            scores[:, o0:o1] = bound.T
            sel = topk_sinks(bound, int(top_k[b]), sink_pages)
        else:
            sel = np.zeros((0, H), np.int64)
        sels.append(sel)
        outs.append(outs[-1] + sel.shape[0])
    return np.concatenate(sels), np.array(outs, np.int64), scores


def gather_pages(deq, sel, page_offsets, out_offsets, page_size: int = 16):
    """staging[i, j, h] = deq[(page_offsets[b] + sel[i, h]) * page_size + j, h]
    for row i of sequence b, zero rows for pages outside the sequence: the
    per-head, compact-format counterpart of unpack_to_staging
    (src/kvquant/compact_pool.py:492-537).  deq (T, H, D) fp16 bits."""
    d = np.asarray(deq, np.uint16)
    T, H, D = d.shape
    sel = np.asarray(sel, np.int64)
    rows = int(out_offsets[-1])
    out = np.zeros((rows, page_size, H, D), np.uint16)
    for b in range(len(page_offsets) - 1):
        P = int(page_offsets[b + 1]) - int(page_offsets[b])
        for i in range(int(out_offsets[b]), int(out_offsets[b + 1])):
            for h in range(H):
                lp = sel[i, h]
                if 0 <= lp < P:
                    t0 = (int(page_offsets[b]) + lp) * page_size
                    out[i, :, h] = d[t0:t0 + page_size, h]
    return out


def ordered_min_max(vals, axis):
    """min / max of fp32 values along ``axis`` with -0 ordered below +0 (the
    pool statistics' order), via the monotone integer key of each value."""
    v = np.ascontiguousarray(vals, np.float32)
    b = v.view(np.int32).astype(np.int64)
    key = np.where(b >= 0, b, -(b & 0x7FFFFFFF) - 1)
    lo = np.take_along_axis(v, np.expand_dims(key.argmin(axis), axis), axis).squeeze(axis)
    hi = np.take_along_axis(v, np.expand_dims(key.argmax(axis), axis), axis).squeeze(axis)
    return lo, hi


def pool_write(pool: dict, key, value, slot_mapping, abs_positions, kscale, vscale,
               block_size: int) -> None:
    """CompactKVPool.write_kv for one layer (src/kvquant/compact_pool.py:447-489,
    kernels :160-287), in place on ``pool``: numpy arrays k_codes, k_outv
    (fp16 bits), k_outm, v_codes, v_outv, v_outm (NB,BS,H,D) and k_min, k_max
    (NB,H,D) fp32.  kscale / vscale = (poles, upper, lower) as fp32 arrays
    holding the scales' values.  Slots < 0 (or past the pool) are skipped; V
    uses scale row min(abs_position, T_cal-1); the K statistics fold in the
    reconstructed value (input for outliers, fp32 pole otherwise) of each
    written token, -0 below +0."""
    key = np.asarray(key, np.float16)
    value = np.asarray(value, np.float16)
    slots = np.asarray(slot_mapping, np.int64)
    pos = np.asarray(abs_positions, np.int64)
    NB, BS, H, D = pool["k_codes"].shape
    keep = (slots >= 0) & (slots < NB * BS)
    if not keep.any():
        return
    k, v, sl, ps = key[keep], value[keep], slots[keep], pos[keep]
    kc, kv, km = pack_k(k, *kscale)
    vc, vv, vm = pack_v(v, *vscale, positions=ps)
    blk, off = sl // BS, sl % BS
    for name, arr in (("k_codes", kc), ("k_outv", kv), ("k_outm", km),
                      ("v_codes", vc), ("v_outv", vv), ("v_outm", vm)):
        pool[name][blk, off] = arr
    kp = _f32(kscale[0])
    hh, dd = np.meshgrid(np.arange(H), np.arange(D), indexing="ij")
    recon = np.where(km.astype(bool), h2f(kv), kp[hh[None], dd[None], kc.astype(np.int64)])
    for b in np.unique(blk):
        rows = recon[blk == b]
        lo, _ = ordered_min_max(np.concatenate([rows, pool["k_min"][b][None]]), axis=0)
        _, hi = ordered_min_max(np.concatenate([rows, pool["k_max"][b][None]]), axis=0)
        pool["k_min"][b], pool["k_max"][b] = lo, hi


def pool_gather(pool: dict, block_ids, first_pos, kscale, vscale):
    """CompactKVPool.unpack_to_staging (src/kvquant/compact_pool.py:492-537,
    kernels :292-395) -> (staging_k, staging_v) fp16 bits (NK,BS,H,D); V row of
    position p in kept block k is min(first_pos[k] + p, T_cal - 1)."""
    ids = np.asarray(block_ids, np.int64)
    fp = np.asarray(first_pos, np.int64)
    NB, BS, H, D = pool["k_codes"].shape
    NK = ids.shape[0]
    c = pool["k_codes"][ids].reshape(NK * BS, H, D)
    sk = unpack(c, pool["k_outv"][ids].reshape(NK * BS, H, D),
                pool["k_outm"][ids].reshape(NK * BS, H, D), kscale[0], "k")
    positions = (fp[:, None] + np.arange(BS)[None, :]).reshape(-1)
    sv = unpack(pool["v_codes"][ids].reshape(NK * BS, H, D),
                pool["v_outv"][ids].reshape(NK * BS, H, D),
                pool["v_outm"][ids].reshape(NK * BS, H, D), vscale[0], "v", positions=positions)
    return sk.reshape(NK, BS, H, D), sv.reshape(NK, BS, H, D)


def h2f(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def f2h(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


__all__ = [n for n in dir() if not n.startswith("_")]


# ------------------------------------------------------- calibration (f4)

def kmeans_1d(values, k: int, iters: int):
    """One 1-D k-means problem -> k fp32 centres, sorted ascending.

    The build's GPU calibration fit, restated (src/kvquant/calibration.py:106-123
    fits sklearn KMeans there): centres start at order statistics,
    c_l = sorted[floor((2l+1) n / 2k)], for n <= 8192 values, else evenly over
    [min, max], c_l = fl32(min + fl32(fl32(max - min) * fl32((2l+1) / 2k))); each of `iters`
    Lloyd steps assigns every value to the first centre of least fp32 |v - c|
    and moves each centre with members to fl32(float64 sum / count).  No values
    -> k zeros; n < k values -> the values and k - n zeros, sorted (the
    reference's padding, calibration.py:116-119).
    """
    v = np.asarray(values, np.float32).reshape(-1)
    n = v.size
    if n < k:
        return np.sort(np.concatenate([v, np.zeros(k - n, np.float32)])).astype(np.float32)
    if n <= 8192:
        c = np.sort(v)[((2 * np.arange(k) + 1) * n) // (2 * k)].astype(np.float32)
    else:
        mn, mx = v.min(), v.max()
        frac = (np.arange(k, dtype=np.float32) * np.float32(2) + np.float32(1)) / np.float32(2 * k)
        c = (mn + (mx - mn) * frac).astype(np.float32)
    for _ in range(iters):
        d = np.abs(v[:, None] - c[None, :])
        idx = np.argmin(d, axis=1)
        s = np.bincount(idx, weights=v.astype(np.float64), minlength=k)
        m = np.bincount(idx, minlength=k)
        c = np.where(m > 0, (s / np.maximum(m, 1)).astype(np.float32), c).astype(np.float32)
    return np.sort(c)


def kmeans_optimal(values, k: int) -> np.ndarray:
    """One 1-D k-means problem solved exactly (orc_kmeans_dp: dynamic
    programming over every split of the sorted values) -> k fp32 centres,
    ascending.  The objective of sklearn's KMeans in
    src/kvquant/calibration.py:106-123, minimised globally."""
    v = np.ascontiguousarray(np.asarray(values, np.float32).reshape(-1))
    out = np.empty(k, np.float32)
    lib().orc_kmeans_dp(v.ctypes.data if v.size else None, v.size, k, out.ctypes.data)
    return out


def kmeans_inertia(values, centers) -> float:
    """Sum of squared distances to the nearest centre (float64)."""
    v = np.asarray(values, np.float64).reshape(-1, 1)
    c = np.asarray(centers, np.float64).reshape(1, -1)
    return float(np.min((v - c) ** 2, axis=1).sum())


# ----------------------------------------------------- paged compact pool (f1)

PAGE = 16


def paged_empty(NB: int, H: int, D: int, bits: int, cap: int, stats: bool, arena: bool = True) -> dict:
    """An empty paged pool side (numpy): codes (NB,H,16,D*bits/8) u8, ocnt
    (NB,H) int64, oent (NB,H,room) u32 -- each page-head's entries in order,
    room = 16*D when an overflow arena takes the entries past cap (the device
    keeps the first cap inline and the rest in the page-head's chunk), else
    cap; kmin / kmax (NB,H,D) fp16 bits (K only; +inf / -inf), status int."""
    room = PAGE * D if arena else cap
    p = dict(codes=np.zeros((NB, H, PAGE, D * bits // 8), np.uint8), ocnt=np.zeros((NB, H), np.int64),
             oent=np.zeros((NB, H, room), np.uint32), bits=bits, cap=cap, room=room, status=0)
    if stats:
        p["kmin"] = np.full((NB, H, D), 0x7C00, np.uint16)
        p["kmax"] = np.full((NB, H, D), 0xFC00, np.uint16)
    return p


def paged_runs(slots, nslots: int):
    """Runs of a slot mapping: maximal stretches of consecutive tokens whose
    slots are in the pool and consecutive within one page, as (first token,
    length, page, first row)."""
    s = np.asarray(slots, np.int64)
    valid = (s >= 0) & (s < nslots)
    runs = []
    t = 0
    T = s.size
    while t < T:
        if not valid[t]:
            t += 1
            continue
        n = 1
        while (t + n < T and valid[t + n] and s[t + n] == s[t + n - 1] + 1 and s[t + n] % PAGE != 0):
            n += 1
        runs.append((t, n, int(s[t]) // PAGE, int(s[t]) % PAGE))
        t += n
    return runs


def _zero_plus(bits16):
    b = np.asarray(bits16, np.uint16).copy()
    b[b == 0x8000] = 0
    return b


def paged_write(pool: dict, values, slot_mapping, scale, per_token: bool, positions=None) -> None:
    """hkv_paged_write restated, in place on ``pool`` (see paged_empty).

    The pool's write of src/kvquant/compact_pool.py:447-489 (kernels :160-287)
    in the bit-packed, per-page-outlier layout: each run (paged_runs) writes
    its rows' codes (the K / V pack of pack_k / pack_v) into rows w0.. of its
    page for every head; the page-head keeps the outliers of rows < w0 (all of
    them, counted, when every stored one is below w0) and appends the run's
    outliers in (row, channel) order, storing the first room; K statistics are
    the min / max of the dequantised values over the run's rows (a zero as
    +0), replacing the page's at w0 = 0 and folded in otherwise.  scale =
    (poles, upper, lower) float32 arrays; V rows min(positions[t], rows - 1)."""
    x = _h16(values)
    T, H, D = x.shape
    bits, cap = pool["bits"], pool["room"]
    NB = pool["codes"].shape[0]
    pos = np.arange(T, dtype=np.int64) if positions is None else np.asarray(positions, np.int64)
    if per_token:
        codes, outv, outm = pack_v(x, *scale, positions=pos)
    else:
        codes, outv, outm = pack_k(x, *scale)
    stats = "kmin" in pool
    if stats:
        deq = unpack(codes, outv, outm, scale[0], "k")
    for t0, n, pg, w0 in paged_runs(slot_mapping, NB * PAGE):
        pool["codes"][pg, :, w0:w0 + n] = bitpack(codes[t0:t0 + n], bits).transpose(1, 0, 2)
        for h in range(H):
            cnt = int(pool["ocnt"][pg, h])
            m = min(cnt, cap)
            stored = pool["oent"][pg, h, :m]
            below = int(((stored >> 24) < w0).sum()) if w0 > 0 else 0
            base = 0 if w0 == 0 else (cnt if below == m else below)
            rr, dd = np.nonzero(outm[t0:t0 + n, h])
            ent = (outv[t0 + rr, h, dd].astype(np.uint32) | (dd.astype(np.uint32) << 16)
                   | ((w0 + rr).astype(np.uint32) << 24))
            idx = base + np.arange(ent.size)
            keep = idx < cap
            pool["oent"][pg, h, idx[keep]] = ent[keep]
            pool["ocnt"][pg, h] = base + ent.size
            if base + ent.size > cap:
                pool["status"] |= 1
            if stats:
                v = h2f(deq[t0:t0 + n, h])
                lo = _zero_plus(f2h(v.min(axis=0)))
                hi = _zero_plus(f2h(v.max(axis=0)))
                if w0 > 0:
                    lo = f2h(np.minimum(h2f(lo), h2f(pool["kmin"][pg, h])))
                    hi = f2h(np.maximum(h2f(hi), h2f(pool["kmax"][pg, h])))
                pool["kmin"][pg, h], pool["kmax"][pg, h] = lo, hi


def paged_gather(pool: dict, block_ids, first_pos, poles, per_token: bool, D: int = 128):
    """hkv_paged_gather restated: staging (NK,16,H,D) fp16 bits, kept block
    k dequantised (ids outside the pool: zeros), V row p at scale row
    min(first_pos[k] + p, rows - 1).  The pool's unpack_to_staging
    (src/kvquant/compact_pool.py:492-537) over the paged layout."""
    ids = np.asarray(block_ids, np.int64)
    NB, H = pool["codes"].shape[:2]
    bits, cap = pool["bits"], pool["room"]
    NK = ids.size
    out = np.zeros((NK, PAGE, H, D), np.uint16)
    for k, b in enumerate(ids):
        if not 0 <= b < NB:
            continue
        codes = bitunpack(pool["codes"][b], bits, D).transpose(1, 0, 2)  # (16, H, D)
        outv = np.zeros((PAGE, H, D), np.uint16)
        outm = np.zeros((PAGE, H, D), np.uint8)
        for h in range(H):
            m = min(int(pool["ocnt"][b, h]), cap)
            e = pool["oent"][b, h, :m]
            sl, ch = (e >> 24).astype(np.int64), ((e >> 16) & 255).astype(np.int64)
            outm[sl, h, ch] = 1
            outv[sl, h, ch] = (e & 0xFFFF).astype(np.uint16)
        if per_token:
            p = int(np.asarray(first_pos, np.int64)[k]) + np.arange(PAGE)
            out[k] = unpack(codes, outv, outm, poles, "v", positions=p)
        else:
            out[k] = unpack(codes, outv, outm, poles, "k")
    return out


__all__ = [n for n in dir() if not n.startswith("_")]
