"""Tensor-level wrappers over the helix_kv C ABI.

Every function validates shapes/dtypes on the host (raising the exception types
the reference raises for the same misuse), allocates outputs with
``torch.empty`` like the reference wrappers do, and launches on torch's current
stream.  Nothing here computes on the CPU.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple

import torch

from . import _native as N


# ------------------------------------------------------------ decision tables

def build_tables(poles: torch.Tensor, upper: torch.Tensor, lower: torch.Tensor) -> torch.Tensor:
    """Decision tables for poles (..., L) and thresholds (...) -> uint8 (n, 80)."""
    N.require_gpu(poles, upper, lower)
    L = int(poles.shape[-1])
    n = poles.numel() // max(L, 1)
    if upper.numel() != n or lower.numel() != n:
        raise AssertionError("thresholds must have one entry per pole row")
    p = poles.contiguous()
    up = upper.contiguous()
    lo = lower.contiguous()
    out = torch.empty((n, N.TABLE_BYTES), dtype=torch.uint8, device=poles.device)
    st = N.lib().hkv_nuq_build_tables(N.ptr(p), N.dtype_code(p), N.ptr(up), N.ptr(lo),
                                      N.dtype_code(up), n, L, N.ptr(out), N.stream_of(p))
    N.check(st, "hkv_nuq_build_tables", AssertionError)
    return out


@dataclass
class NuqLayerTables:
    """One layer's K (per-channel) or V (per-token) scales on the device, with
    their decision tables.

    per-channel: poles (H,D,L), thresholds (H,D)  (src/kvquant/scales.py:13-39)
    per-token:   poles (H,rows,L), thresholds (H,rows)  (src/kvquant/scales.py:42-69)
    """

    poles: torch.Tensor
    upper: torch.Tensor
    lower: torch.Tensor
    per_token: bool
    tables: torch.Tensor | None = None

    def __post_init__(self) -> None:
        N.require_gpu(self.poles, self.upper, self.lower)
        if self.poles.dim() != 3:
            raise AssertionError(f"poles must be 3-D, got {tuple(self.poles.shape)}")
        if tuple(self.upper.shape) != tuple(self.poles.shape[:2]) or \
                tuple(self.lower.shape) != tuple(self.poles.shape[:2]):
            raise AssertionError("thresholds must match poles[..., 0]")
        self.poles = self.poles.contiguous()
        self.upper = self.upper.contiguous()
        self.lower = self.lower.contiguous()
        if self.upper.dtype != self.lower.dtype:
            self.lower = self.lower.to(self.upper.dtype)

    @property
    def levels(self) -> int:
        return int(self.poles.shape[-1])

    @property
    def rows(self) -> int:
        return int(self.poles.shape[1]) if self.per_token else 0

    def ensure_tables(self) -> torch.Tensor:
        if self.tables is None:
            self.tables = build_tables(self.poles, self.upper, self.lower)
        return self.tables

    def struct(self, positions: torch.Tensor | None = None, pos_offset: int = 0,
               with_tables: bool = True) -> N.NuqScales:
        s = N.NuqScales()
        s.tables = self.ensure_tables().data_ptr() if with_tables else None
        s.poles = self.poles.data_ptr()
        s.upper = self.upper.data_ptr()
        s.lower = self.lower.data_ptr()
        s.poles_dtype = N.dtype_code(self.poles)
        s.thr_dtype = N.dtype_code(self.upper)
        s.levels = self.levels
        s.per_token = 1 if self.per_token else 0
        s.rows = self.rows
        s.positions = positions.data_ptr() if positions is not None else None
        s.pos_offset = int(pos_offset)
        return s


def _positions(positions, T: int, device) -> torch.Tensor | None:
    if positions is None:
        return None
    p = positions.to(device=device, dtype=torch.int64).contiguous()
    if p.numel() != T:
        raise AssertionError(f"positions must have {T} entries, got {p.numel()}")
    return p


def _check_values(values: torch.Tensor, H: int, D: int) -> None:
    N.require_gpu(values)
    assert values.dtype == torch.float16, "values must be fp16"
    assert values.is_contiguous(), "values must be contiguous (T, H, D)"
    if values.dim() != 3 or values.shape[1] != H or values.shape[2] != D:
        raise AssertionError(f"values shape {tuple(values.shape)} does not match scales (H={H}, D={D})")


def _HD(t: NuqLayerTables, values: torch.Tensor) -> tuple[int, int]:
    H = int(t.poles.shape[0])
    D = int(values.shape[-1]) if t.per_token else int(t.poles.shape[1])
    return H, D


# ---------------------------------------------------------------- dense (a3/a6)

def nuq_pack_dense(values: torch.Tensor, t: NuqLayerTables, positions=None, pos_offset: int = 0):
    """(T,H,D) fp16 -> (codes u8, outlier_v fp16, outlier_m u8), the reference format."""
    H, D = _HD(t, values)
    _check_values(values, H, D)
    T = int(values.shape[0])
    pos = _positions(positions, T, values.device)
    codes = torch.empty((T, H, D), dtype=torch.uint8, device=values.device)
    outv = torch.empty((T, H, D), dtype=torch.float16, device=values.device)
    outm = torch.empty((T, H, D), dtype=torch.uint8, device=values.device)
    if T == 0:
        return codes, outv, outm
    s = t.struct(pos, pos_offset)
    st = N.lib().hkv_nuq_pack_dense(N.ptr(values), T, H, D, s, N.ptr(codes), N.ptr(outv),
                                    N.ptr(outm), N.stream_of(values))
    N.check(st, "hkv_nuq_pack_dense", AssertionError)
    return codes, outv, outm


def nuq_unpack_dense(codes: torch.Tensor, outlier_v: torch.Tensor, outlier_m: torch.Tensor,
                     t: NuqLayerTables, positions=None, pos_offset: int = 0) -> torch.Tensor:
    N.require_gpu(codes, outlier_v, outlier_m)
    assert codes.dtype == torch.uint8, "codes must be uint8"
    assert codes.is_contiguous(), "codes must be contiguous"
    T, H, D = (int(x) for x in codes.shape)
    ov = outlier_v.to(torch.float16).contiguous()
    om = outlier_m.to(torch.uint8).contiguous()
    if ov.shape != codes.shape or om.shape != codes.shape:
        raise AssertionError("codes / outlier_v / outlier_m shapes differ")
    pos = _positions(positions, T, codes.device)
    out = torch.empty((T, H, D), dtype=torch.float16, device=codes.device)
    if T == 0:
        return out
    s = t.struct(pos, pos_offset, with_tables=False)
    st = N.lib().hkv_nuq_unpack_dense(N.ptr(codes), N.ptr(ov), N.ptr(om), T, H, D, s, N.ptr(out),
                                      N.stream_of(codes))
    N.check(st, "hkv_nuq_unpack_dense", AssertionError)
    return out


# ----------------------------------------------------------- compact (a5/a6)

@dataclass
class CompactCodes:
    """Bit-packed codes + CSR outliers of one (T,H,D) tensor.

    packed (T,H,D*bits/8) u8; row_ptr (T*H+1) int32 over rows t*H+h;
    col (>= nnz) u8; val (>= nnz) fp16.  ``nnz`` is None until read.
    """

    packed: torch.Tensor
    row_ptr: torch.Tensor
    col: torch.Tensor
    val: torch.Tensor
    bits: int
    nnz: int | None = None

    @property
    def shape(self) -> tuple[int, int, int]:
        T, H, B = self.packed.shape
        return int(T), int(H), int(B) * 8 // self.bits

    @staticmethod
    def empty(T: int, H: int, D: int, bits: int, capacity: int, device) -> "CompactCodes":
        return CompactCodes(
            packed=torch.empty((T, H, D * bits // 8), dtype=torch.uint8, device=device),
            row_ptr=torch.empty((T * H + 1,), dtype=torch.int32, device=device),
            col=torch.empty((max(capacity, 1),), dtype=torch.uint8, device=device),
            val=torch.empty((max(capacity, 1),), dtype=torch.float16, device=device),
            bits=bits)

    def read_nnz(self) -> int:
        self.nnz = int(self.row_ptr[-1].item())
        return self.nnz


def pack_workspace(T: int, H: int, D: int, device) -> torch.Tensor:
    nb = int(N.lib().hkv_nuq_pack_compact_workspace_bytes(T, H, D))
    return N.workspace("nuq_pack", nb, device)


def nuq_pack_compact(values: torch.Tensor, t: NuqLayerTables, bits: int, *,
                     capacity: int | None = None, positions=None, pos_offset: int = 0,
                     out: CompactCodes | None = None, sync: bool = True) -> CompactCodes:
    """(T,H,D) fp16 -> CompactCodes.

    With sync=True the true nnz is read back.  The result is a new
    CompactCodes whose col / val are views trimmed to nnz; the tensors of a
    caller's ``out`` keep their full capacity (its ``nnz`` field is recorded).
    If nnz exceeds the capacity, the call is re-issued into larger buffers,
    unless ``out`` was given: then it raises, since the caller's buffers cannot
    hold the result.  With sync=False nothing is read back and ``out`` (or the
    new buffers) is returned as written; the caller compares row_ptr[-1] with
    the capacity when it next synchronises."""
    H, D = _HD(t, values)
    _check_values(values, H, D)
    if bits not in (2, 4):
        raise AssertionError("bits must be 2 or 4")
    if t.levels > (1 << bits):
        raise AssertionError(f"{t.levels} levels do not fit in {bits} bits")
    T = int(values.shape[0])
    if capacity is None:
        capacity = max(1024, (T * H * D) // 8)
    caller_out = out is not None
    if out is None:
        out = CompactCodes.empty(T, H, D, bits, capacity, values.device)
    elif out.shape != (T, H, D) or out.bits != bits or out.row_ptr.numel() != T * H + 1:
        raise AssertionError(f"out is {out.shape} at {out.bits} bits, the pack is {(T, H, D)} "
                             f"at {bits} bits")
    pos = _positions(positions, T, values.device)
    ws = pack_workspace(T, H, D, values.device)
    s = t.struct(pos, pos_offset)

    def launch(cc: CompactCodes) -> None:
        st = N.lib().hkv_nuq_pack_compact(
            N.ptr(values), T, H, D, bits, s, N.ptr(cc.packed), N.ptr(cc.row_ptr), N.ptr(cc.col),
            N.ptr(cc.val), int(cc.col.numel()), N.ptr(ws), ws.numel(), N.stream_of(values))
        N.check(st, "hkv_nuq_pack_compact", AssertionError)

    launch(out)
    if not sync:
        return out
    nnz = out.read_nnz()
    cap = min(int(out.col.numel()), int(out.val.numel()))
    if nnz > cap:
        if caller_out:
            raise RuntimeError(f"hkv_nuq_pack_compact: {nnz} outliers exceed the capacity {cap} "
                               "of the given out")
        out = CompactCodes.empty(T, H, D, bits, nnz, values.device)
        launch(out)
        out.read_nnz()
    return CompactCodes(packed=out.packed, row_ptr=out.row_ptr, col=out.col[:nnz],
                        val=out.val[:nnz], bits=bits, nnz=nnz)


class CompactPackBatch:
    """A prepared batch of compact packs (a prefill step: every layer's K and
    V), launched by calling it: as few launches as the tensors' kernel
    variants allow, each result identical to its own :func:`nuq_pack_compact`
    call.  ``jobs`` is a sequence of (values, tables, bits, out) or (values,
    tables, bits, out, positions, pos_offset) with caller-allocated ``out``
    CompactCodes.  Nothing is read back (the caller compares each
    out.row_ptr[-1] with its capacity when it next synchronises), so a call
    can be captured in a HIP graph.  The tensors must stay alive while the
    batch is in use."""

    def __init__(self, jobs) -> None:
        self.jobs = list(jobs)
        self.n = len(self.jobs)
        self.items = (N.PackItem * max(1, self.n))()
        self._keep = []
        dev = None
        for i, job in enumerate(self.jobs):
            values, t, bits, out = job[:4]
            positions = job[4] if len(job) > 4 else None
            pos_offset = job[5] if len(job) > 5 else 0
            H, D = _HD(t, values)
            _check_values(values, H, D)
            if bits not in (2, 4):
                raise AssertionError("bits must be 2 or 4")
            if t.levels > (1 << bits):
                raise AssertionError(f"{t.levels} levels do not fit in {bits} bits")
            T = int(values.shape[0])
            if out is None or out.shape != (T, H, D) or out.bits != bits or \
                    out.row_ptr.numel() != T * H + 1:
                raise AssertionError(f"job {i}: out must be CompactCodes of {(T, H, D)} at {bits} bits")
            if dev is None:
                dev = values.device
            elif values.device != dev:
                raise AssertionError("all tensors of a batch must be on one device")
            pos = _positions(positions, T, values.device)
            self._keep.append(pos)
            it = self.items[i]
            it.values = values.data_ptr()
            it.T, it.H, it.D, it.bits = T, H, D, bits
            it.scales = t.struct(pos, pos_offset)
            it.packed = out.packed.data_ptr()
            it.row_ptr = out.row_ptr.data_ptr()
            it.col = out.col.data_ptr()
            it.val = out.val.data_ptr()
            it.capacity = min(int(out.col.numel()), int(out.val.numel()))
        self.device = dev
        self.ws_bytes = int(N.lib().hkv_nuq_pack_compact_batch_workspace_bytes(self.items, self.n)) \
            if self.n else 0

    def __call__(self) -> list[CompactCodes]:
        if self.n:
            ws = N.workspace("nuq_pack", self.ws_bytes, self.device)
            st = N.lib().hkv_nuq_pack_compact_batch(self.items, self.n, N.ptr(ws), ws.numel(),
                                                    N.stream_of(self.jobs[0][0]))
            N.check(st, "hkv_nuq_pack_compact_batch", AssertionError)
        return [job[3] for job in self.jobs]


def nuq_pack_compact_batch(jobs) -> list[CompactCodes]:
    """Prepare and launch a :class:`CompactPackBatch` once."""
    return CompactPackBatch(jobs)()


def nuq_unpack_compact(cc: CompactCodes, t: NuqLayerTables, *, positions=None, pos_offset: int = 0,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    N.require_gpu(cc.packed, cc.row_ptr)
    T, H, D = cc.shape
    if out is None:
        out = torch.empty((T, H, D), dtype=torch.float16, device=cc.packed.device)
    if T == 0:
        return out
    pos = _positions(positions, T, cc.packed.device)
    s = t.struct(pos, pos_offset)
    st = N.lib().hkv_nuq_unpack_compact(
        N.ptr(cc.packed), N.ptr(cc.row_ptr), N.ptr(cc.col), N.ptr(cc.val),
        min(int(cc.col.numel()), int(cc.val.numel())), T, H, D, cc.bits, s,
        N.ptr(out), N.stream_of(out))
    N.check(st, "hkv_nuq_unpack_compact", AssertionError)
    return out


class CompactUnpackBatch:
    """A prepared batch of compact unpacks, launched by calling it: as few
    launches as the tensors' kernel variants allow, each result identical to
    its own :func:`nuq_unpack_compact` call.  ``jobs`` is a sequence of
    (cc, tables, out) or (cc, tables, out, positions, pos_offset) with
    caller-allocated fp16 ``out`` (T,H,D).  The tensors must stay alive while
    the batch is in use."""

    def __init__(self, jobs) -> None:
        self.jobs = list(jobs)
        self.n = len(self.jobs)
        self.items = (N.UnpackItem * max(1, self.n))()
        self._keep = []
        for i, job in enumerate(self.jobs):
            cc, t, out = job[:3]
            positions = job[3] if len(job) > 3 else None
            pos_offset = job[4] if len(job) > 4 else 0
            N.require_gpu(cc.packed, cc.row_ptr, out)
            T, H, D = cc.shape
            if tuple(out.shape) != (T, H, D) or out.dtype != torch.float16 or not out.is_contiguous():
                raise AssertionError(f"job {i}: out must be contiguous fp16 {(T, H, D)}")
            pos = _positions(positions, T, cc.packed.device)
            self._keep.append(pos)
            it = self.items[i]
            it.packed = cc.packed.data_ptr()
            it.row_ptr = cc.row_ptr.data_ptr()
            it.col = cc.col.data_ptr()
            it.val = cc.val.data_ptr()
            it.capacity = min(int(cc.col.numel()), int(cc.val.numel()))
            it.T, it.H, it.D, it.bits = T, H, D, cc.bits
            it.scales = t.struct(pos, pos_offset)
            it.out = out.data_ptr()

    def __call__(self) -> list[torch.Tensor]:
        if self.n:
            st = N.lib().hkv_nuq_unpack_compact_batch(self.items, self.n,
                                                      N.stream_of(self.jobs[0][2]))
            N.check(st, "hkv_nuq_unpack_compact_batch", AssertionError)
        return [job[2] for job in self.jobs]


# ------------------------------------------------------------------ Quest

def _fdt(t: torch.Tensor) -> int:
    if t.dtype not in (torch.float16, torch.float32):
        raise TypeError(f"unsupported dtype {t.dtype}")
    return N.dtype_code(t)


def quest_page_stats(K_pages: torch.Tensor):
    """(P,S,H,D) -> (K_min, K_max) (P,H,D), same dtype.  src/quest/reference.py:38-56."""
    if K_pages.dim() != 4:
        raise ValueError(f"expected (P, page, H, D), got {tuple(K_pages.shape)}")
    N.require_gpu(K_pages)
    K = K_pages.contiguous()
    P, S, H, D = (int(x) for x in K.shape)
    kmin = torch.empty((P, H, D), dtype=K.dtype, device=K.device)
    kmax = torch.empty((P, H, D), dtype=K.dtype, device=K.device)
    if P == 0:
        return kmin, kmax
    if S == 0:
        raise ValueError("pages must hold at least one slot")
    st = N.lib().hkv_quest_page_stats(N.ptr(K), _fdt(K), P, S, H, D, N.ptr(kmin), N.ptr(kmax),
                                      N.stream_of(K))
    N.check(st, "hkv_quest_page_stats", ValueError)
    return kmin, kmax


def quest_page_bound(query: torch.Tensor, K_min: torch.Tensor, K_max: torch.Tensor,
                     out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """(Hq,D) query, (P,H,D) stats -> (P,H) bound (canonical fp32 order).

    Hq == H: src/quest/reference.py:59-93; Hq = g*H: the group's bounds summed.
    """
    if query.dim() != 2:
        raise ValueError(f"query should be (H, D), got {tuple(query.shape)}")
    if K_min.shape != K_max.shape or K_min.dim() != 3:
        raise ValueError(
            f"K_min/K_max should be (P, H, D), got {tuple(K_min.shape)} and {tuple(K_max.shape)}")
    N.require_gpu(query, K_min, K_max)
    P, H, D = (int(x) for x in K_min.shape)
    Hq = int(query.shape[0])
    if int(query.shape[1]) != D or Hq % H != 0:
        raise ValueError(f"query {tuple(query.shape)} incompatible with stats {tuple(K_min.shape)}")
    kmin = K_min.contiguous()
    kmax = K_max.to(kmin.dtype).contiguous()
    q = query.contiguous()
    out = torch.empty((P, H), dtype=out_dtype, device=kmin.device)
    if P == 0:
        return out
    st = N.lib().hkv_quest_page_bound(N.ptr(q), N.dtype_code(q), Hq, N.ptr(kmin), N.ptr(kmax),
                                      _fdt(kmin), P, H, D, N.ptr(out), N.dtype_code(out),
                                      N.stream_of(q))
    N.check(st, "hkv_quest_page_bound", ValueError)
    return out


def quest_topk(bound: torch.Tensor, k: int, sink_pages: int = 1) -> torch.Tensor:
    """(P,H) bound -> (sinks + k_eff, H) int64 (src/quest/reference.py:96-133)."""
    if bound.dim() != 2:
        raise ValueError(f"bound should be (P, H), got {tuple(bound.shape)}")
    N.require_gpu(bound)
    b = bound if bound.dtype in (torch.float16, torch.float32) else bound.float()
    b = b.contiguous()
    P, H = (int(x) for x in b.shape)
    s = max(0, min(int(sink_pages), P))
    keff = max(0, min(int(k), P - s))
    out = torch.empty((s + keff, H), dtype=torch.int64, device=b.device)
    if s + keff == 0:
        return out
    ws = N.workspace("quest_topk", int(N.lib().hkv_quest_topk_workspace_bytes(P, H)), b.device)
    n_out = N._i64(0)
    st = N.lib().hkv_quest_topk(N.ptr(b), N.dtype_code(b), P, H, int(k), int(sink_pages), N.ptr(out),
                                n_out, N.ptr(ws), ws.numel(), N.stream_of(b))
    N.check(st, "hkv_quest_topk", ValueError)
    return out


def quest_select(query: torch.Tensor, K_min: torch.Tensor, K_max: torch.Tensor, k: int,
                 sink_pages: int, *, scores: torch.Tensor | None = None,
                 out: torch.Tensor | None = None):
    """Bound + top-K for one decode step.

    query (Hq,D) with Hq a multiple of H; stats (P,H,D) fp16/fp32.  Returns
    (indices (sinks + k_eff, H) int64, scores (H,P) fp32 head-major -- the
    group-summed bound of every page).
    """
    N.require_gpu(query, K_min, K_max)
    if K_min.dim() != 3 or K_min.shape != K_max.shape:
        raise ValueError("K_min/K_max should be (P, H, D)")
    P, H, D = (int(x) for x in K_min.shape)
    Hq = int(query.shape[0])
    if query.dim() != 2 or int(query.shape[1]) != D or Hq % H:
        raise ValueError(f"query {tuple(query.shape)} incompatible with stats {tuple(K_min.shape)}")
    kmin = K_min.contiguous()
    kmax = K_max.to(kmin.dtype).contiguous()
    q = query.contiguous()
    s = max(0, min(int(sink_pages), P))
    keff = max(0, min(int(k), P - s))
    if out is None:
        out = torch.empty((s + keff, H), dtype=torch.int64, device=kmin.device)
    if scores is None:
        scores = torch.empty((H, P), dtype=torch.float32, device=kmin.device)
    if tuple(out.shape) != (s + keff, H) or tuple(scores.shape) != (H, P):
        raise ValueError("out must be (sinks + k_eff, H) and scores (H, P)")
    n_out = N._i64(0)
    ws = N.workspace("quest_select", int(N.lib().hkv_quest_select_workspace_bytes(P, H)), q.device)
    st = N.lib().hkv_quest_select(N.ptr(q), N.dtype_code(q), Hq, N.ptr(kmin), N.ptr(kmax),
                                  _fdt(kmin), P, H, D, int(k), int(sink_pages), N.ptr(scores),
                                  N.ptr(out), n_out, N.ptr(ws), ws.numel(), N.stream_of(q))
    N.check(st, "hkv_quest_select", ValueError)
    return out, scores


class QuestStatsU8(NamedTuple):
    """Compact page metadata: u8 codes of the page min / max (P,H,D) and the
    per-(head, channel) lo / step (H,D) fp32 that read them back."""
    qmin: torch.Tensor
    qmax: torch.Tensor
    lo: torch.Tensor
    step: torch.Tensor


def quest_page_stats_u8(K_min: torch.Tensor, K_max: torch.Tensor) -> QuestStatsU8:
    """(P,H,D) fp16/fp32 page statistics -> their compact u8 form, rounded so
    that the bound read from it is never below the bound from the originals
    (hkv_quest_page_stats_u8)."""
    N.require_gpu(K_min, K_max)
    if K_min.dim() != 3 or K_min.shape != K_max.shape:
        raise ValueError("K_min/K_max should be (P, H, D)")
    P, H, D = (int(x) for x in K_min.shape)
    kmin = K_min.contiguous()
    kmax = K_max.to(kmin.dtype).contiguous()
    dev = kmin.device
    qmin = torch.empty((P, H, D), dtype=torch.uint8, device=dev)
    qmax = torch.empty((P, H, D), dtype=torch.uint8, device=dev)
    lo = torch.empty((H, D), dtype=torch.float32, device=dev)
    step = torch.empty((H, D), dtype=torch.float32, device=dev)
    ws = torch.empty(max(4, int(N.lib().hkv_quest_page_stats_u8_workspace_bytes(H, D))) // 4,
                     dtype=torch.int32, device=dev)
    st = N.lib().hkv_quest_page_stats_u8(N.ptr(kmin), N.ptr(kmax), _fdt(kmin), P, H, D, N.ptr(qmin),
                                         N.ptr(qmax), N.ptr(lo), N.ptr(step), N.ptr(ws),
                                         ws.numel() * 4, N.stream_of(kmin))
    N.check(st, "hkv_quest_page_stats_u8", ValueError)
    return QuestStatsU8(qmin, qmax, lo, step)


def quest_select_u8(query: torch.Tensor, stats: QuestStatsU8, k: int, sink_pages: int, *,
                    scores: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """quest_select over the compact u8 metadata (hkv_quest_select_u8): returns
    (indices (sinks + k_eff, H) int64, scores (H,P) fp32)."""
    N.require_gpu(query, stats.qmin, stats.qmax, stats.lo, stats.step)
    if stats.qmin.dim() != 3 or stats.qmin.shape != stats.qmax.shape:
        raise ValueError("qmin/qmax should be (P, H, D)")
    P, H, D = (int(x) for x in stats.qmin.shape)
    if tuple(stats.lo.shape) != (H, D) or tuple(stats.step.shape) != (H, D):
        raise ValueError("lo/step should be (H, D)")
    Hq = int(query.shape[0])
    if query.dim() != 2 or int(query.shape[1]) != D or Hq % H:
        raise ValueError(f"query {tuple(query.shape)} incompatible with stats {(P, H, D)}")
    q = query.contiguous()
    s = max(0, min(int(sink_pages), P))
    keff = max(0, min(int(k), P - s))
    if out is None:
        out = torch.empty((s + keff, H), dtype=torch.int64, device=q.device)
    if scores is None:
        scores = torch.empty((H, P), dtype=torch.float32, device=q.device)
    if tuple(out.shape) != (s + keff, H) or tuple(scores.shape) != (H, P):
        raise ValueError("out must be (sinks + k_eff, H) and scores (H, P)")
    n_out = N._i64(0)
    ws = N.workspace("quest_select", int(N.lib().hkv_quest_select_workspace_bytes(P, H)), q.device)
    st = N.lib().hkv_quest_select_u8(
        N.ptr(q), N.dtype_code(q), Hq, N.ptr(stats.qmin.contiguous()), N.ptr(stats.qmax.contiguous()),
        N.ptr(stats.lo.contiguous()), N.ptr(stats.step.contiguous()), P, H, D, int(k), int(sink_pages),
        N.ptr(scores), N.ptr(out), n_out, N.ptr(ws), ws.numel(), N.stream_of(q))
    N.check(st, "hkv_quest_select_u8", ValueError)
    return out, scores


# ------------------------------------------------------------ decode attention

def decode_pages_per_split(nsel: int, H: int) -> int:
    """Pages per split of the decode kernel: about 3 blocks of 4 waves per CU
    over the (split, KV head) grid, a multiple of the block's 4 waves."""
    cus = N.num_cus()
    want = max(1, -(-nsel * H // (3 * cus)))
    return min(256, max(4, -(-want // 4) * 4))


def decode_attention(query: torch.Tensor, k: CompactCodes, kt: NuqLayerTables, v: CompactCodes,
                     vt: NuqLayerTables, sel: torch.Tensor, *, scale: float | None = None,
                     pages_per_split: int | None = None, out: torch.Tensor | None = None,
                     out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """softmax(q.K^T * scale).V per query head over its KV head's selected
    pages, read straight from the compact format (hkv_decode_attn).

    query (Hq, 128) fp16; k / v the CompactCodes of (T, H, 128) with their
    scales' tables (K per-channel, V per-token, token t at V row
    min(t, rows - 1)); sel (n, H) int64 page ids of 16 tokens (quest_topk's
    output).  Query head hq uses KV head hq // (Hq // H).  Returns (Hq, 128).
    """
    N.require_gpu(query, k.packed, v.packed, sel)
    T, H, D = k.shape
    if v.shape != (T, H, D):
        raise AssertionError("K and V must have the same (T, H, D)")
    if query.dim() != 2 or int(query.shape[1]) != D or int(query.shape[0]) % H:
        raise ValueError(f"query {tuple(query.shape)} incompatible with (T, H, D) = {(T, H, D)}")
    if query.dtype != torch.float16:
        raise AssertionError("query must be fp16")
    if kt.per_token or not vt.per_token:
        raise AssertionError("K scales are per-channel, V scales per-token")
    Hq = int(query.shape[0])
    if sel.dim() != 2 or int(sel.shape[1]) != H:
        raise ValueError(f"sel should be (n, {H}), got {tuple(sel.shape)}")
    s = sel.to(torch.int64).contiguous()
    nsel = int(s.shape[0])
    pps = int(pages_per_split) if pages_per_split else decode_pages_per_split(nsel, H)
    q = query.contiguous()
    if out is None:
        out = torch.empty((Hq, D), dtype=out_dtype, device=q.device)
    if tuple(out.shape) != (Hq, D) or out.dtype not in (torch.float16, torch.float32):
        raise AssertionError("out must be (Hq, D) fp16 or fp32")
    nb = int(N.lib().hkv_decode_workspace_bytes(nsel, Hq, pps))
    ws = N.workspace("decode", nb, q.device)
    sc = float(scale) if scale is not None else D ** -0.5
    st = N.lib().hkv_decode_attn(
        N.ptr(q), Hq, H, D, T,
        N.ptr(k.packed), N.ptr(k.row_ptr), N.ptr(k.col), N.ptr(k.val),
        min(int(k.col.numel()), int(k.val.numel())), k.bits, N.ptr(kt.ensure_tables()),
        N.ptr(v.packed), N.ptr(v.row_ptr), N.ptr(v.col), N.ptr(v.val),
        min(int(v.col.numel()), int(v.val.numel())), v.bits, N.ptr(vt.ensure_tables()), vt.rows,
        N.ptr(s), nsel, pps, sc, N.ptr(out), N.dtype_code(out), N.ptr(ws), ws.numel(),
        N.stream_of(q))
    N.check(st, "hkv_decode_attn", AssertionError)
    return out


def decode_step(query: torch.Tensor, k: CompactCodes, kt: NuqLayerTables, v: CompactCodes,
                vt: NuqLayerTables, K_min: torch.Tensor | None, K_max: torch.Tensor | None,
                top_k: int, sink_pages: int = 4, *, gqa: str = "mean", select: str = "union",
                scale: float | None = None, out: torch.Tensor | None = None,
                out_dtype: torch.dtype = torch.float16,
                pages_per_split: int | None = None,
                stats_u8: "QuestStatsU8 | None" = None) -> torch.Tensor:
    """One decode step of one sequence held in the compact format: Quest page
    selection from the page statistics, then the fused dequant + attention over
    the selected pages.  Every size is known on the host, so the step reads
    nothing back from the device and can be captured in a HIP graph.

    The sync-free counterpart of the compact backend's decode forward
    (src/kvquant/compact_backend.py:194-299), which reads seq_len, the selected
    count and the last block's position back to the host:
      - gqa="mean": the query heads of a group are averaged into one query per
        KV head, in the query's dtype (compact_backend.py:225-231); "sum": the
        bound of every query head, summed over the group.
      - select="union": every query head attends to the union over KV heads of
        the selected pages (src/kvquant/quest_selector.py:80, then all heads
        of each kept block, compact_pool.py:492-537); "per_head": each KV head
        attends to its own pages.  Sinks are the first sink_pages pages.
      - The sequence is the k.shape[0] tokens of k / v; the last page may be
        partial and its missing slots are masked (compact_backend.py:253-262).
    query (Hq, 128) fp16; K_min / K_max (ceil(T / 16), H, 128) page statistics
    of the sequence's K, or stats_u8 (their compact u8 form, quest_page_stats_u8:
    half the bytes, every bound at least the fp16 one) with K_min / K_max None.
    Returns (Hq, 128).
    """
    T, H, D = k.shape
    P = -(-T // 16)
    if stats_u8 is not None:
        N.require_gpu(query, stats_u8.qmin)
        if tuple(stats_u8.qmin.shape) != (P, H, D):
            raise ValueError(f"stats_u8 should be ({P}, {H}, {D}), got {tuple(stats_u8.qmin.shape)}")
    else:
        if K_min is None or K_max is None:
            raise ValueError("decode_step needs K_min / K_max or stats_u8")
        N.require_gpu(query, K_min, K_max)
        if K_min.dim() != 3 or tuple(K_min.shape) != (P, H, D) or K_max.shape != K_min.shape:
            raise ValueError(f"K_min/K_max should be ({P}, {H}, {D}), got {tuple(K_min.shape)}")
    if query.dim() != 2 or int(query.shape[0]) % H or int(query.shape[1]) != D:
        raise ValueError(f"query {tuple(query.shape)} incompatible with (T, H, D) = {(T, H, D)}")
    Hq = int(query.shape[0])
    if gqa == "mean":
        qs = query.reshape(H, Hq // H, D).mean(dim=1).to(torch.float16)
    elif gqa == "sum":
        qs = query
    else:
        raise ValueError(f"gqa must be 'mean' or 'sum', got {gqa!r}")
    if stats_u8 is not None:
        sel, _ = quest_select_u8(qs, stats_u8, top_k, sink_pages)
    else:
        sel, _ = quest_select(qs, K_min, K_max, top_k, sink_pages)
    if select == "union":
        # the union's pages ascending at the front, -1 after them: the decode
        # kernel's splits past the union's end find no valid page and return
        sel = union_pages(sel, P)
    elif select != "per_head":
        raise ValueError(f"select must be 'union' or 'per_head', got {select!r}")
    return decode_attention(query, k, kt, v, vt, sel, scale=scale, out=out, out_dtype=out_dtype,
                            pages_per_split=pages_per_split)


def union_pages(sel: torch.Tensor, P: int) -> torch.Tensor:
    """The union over KV heads of one sequence's selection (n, H) of pages in
    [0, P), as a (P, H) list of the union's pages ascending, every column
    alike, followed by -1 (hkv_union_pages_ragged: three launches, no read-back).
    src/kvquant/quest_selector.py:80."""
    import ctypes

    N.require_gpu(sel)
    n, H = (int(x) for x in sel.shape)
    s = sel.to(torch.int64).contiguous()
    out = torch.empty((max(P, 1), H), dtype=torch.int64, device=sel.device)
    flags = N.workspace("union_flags", int(N.lib().hkv_union_pages_workspace_bytes(P)), sel.device)
    c_rows = (ctypes.c_int64 * 2)(0, n)
    c_pages = (ctypes.c_int64 * 2)(0, P)
    st = N.lib().hkv_union_pages_ragged(N.ptr(s), H, 1, c_rows, c_pages, N.ptr(out), N.ptr(flags),
                                        flags.numel(), N.stream_of(s))
    N.check(st, "hkv_union_pages_ragged", ValueError)
    return out[:P]


def compact_view(c: CompactCodes, t0: int, t1: int) -> CompactCodes:
    """Tokens [t0, t1) of a CompactCodes, without copies: the packed rows and
    row_ptr entries are sliced, col / val stay whole (row_ptr holds absolute
    offsets into them)."""
    T, H, _ = c.shape
    if not 0 <= t0 <= t1 <= T:
        raise ValueError(f"token range [{t0}, {t1}) outside [0, {T})")
    return CompactCodes(packed=c.packed[t0:t1], row_ptr=c.row_ptr[t0 * H:t1 * H + 1], col=c.col,
                        val=c.val, bits=c.bits, nnz=c.nnz)


def decode_step_batch(queries: torch.Tensor, k: CompactCodes, kt: NuqLayerTables, v: CompactCodes,
                      vt: NuqLayerTables, K_min: torch.Tensor, K_max: torch.Tensor,
                      seq_starts, seq_lens, top_k, sink_pages: int = 4, *, gqa: str = "mean",
                      select: str = "union", scale: float | None = None,
                      out: torch.Tensor | None = None,
                      out_dtype: torch.dtype = torch.float16,
                      pages_per_split: int | None = None) -> torch.Tensor:
    """decode_step for B sequences held in one compact-format tensor, still
    without host reads.  Sequence b is tokens [seq_starts[b], seq_starts[b] +
    seq_lens[b]) of k / v (starts are multiples of the 16-token page; V was
    packed with positions counted from each sequence's start), its page
    statistics are K_min / K_max rows [seq_starts[b] / 16, ...).  The reference
    forward handles batch 1 only (src/kvquant/compact_backend.py:184-203).

    When the sequences lie back to back (each starts on the page after the
    previous one's last), each batch of up to 64 is one ragged Quest selection
    (hkv_quest_select_ragged), the per-sequence union of the heads' pages for
    select="union" (hkv_union_pages_ragged) and one batched decode + merge
    (hkv_decode_attn_batch); each sequence's result equals decode_step's with
    the same pages_per_split.  Otherwise decode_step runs per sequence.
    top_k: one int, or one per sequence.  queries (B, Hq, 128) fp16; returns
    (B, Hq, 128)."""
    import ctypes

    N.require_gpu(queries, K_min, K_max)
    starts = [int(s) for s in seq_starts]
    lens = [int(n) for n in seq_lens]
    B = len(starts)
    if queries.dim() != 3 or int(queries.shape[0]) != B or len(lens) != B:
        raise ValueError(f"queries {tuple(queries.shape)} do not match {B} sequences")
    if any(s % 16 for s in starts) or any(n < 1 for n in lens):
        raise ValueError("sequence starts must be multiples of 16 and lengths positive")
    ks = [int(top_k)] * B if not hasattr(top_k, '__len__') else [int(x) for x in top_k]
    if len(ks) != B:
        raise ValueError("one top_k per sequence")
    if gqa not in ("mean", "sum"):
        raise ValueError(f"gqa must be 'mean' or 'sum', got {gqa!r}")
    if select not in ("union", "per_head"):
        raise ValueError(f"select must be 'union' or 'per_head', got {select!r}")
    if out is None:
        out = torch.empty(tuple(queries.shape), dtype=out_dtype, device=queries.device)
    T, H, D = k.shape
    pages = [-(-n // 16) for n in lens]
    back_to_back = all(starts[b + 1] == starts[b] + 16 * pages[b] for b in range(B - 1))
    if back_to_back and B > 64 and starts[-1] + lens[-1] <= T and v.shape == (T, H, D):
        for c in range(0, B, 64):  # batches of 64 (each one launch of the decode)
            decode_step_batch(queries[c:c + 64], k, kt, v, vt, K_min, K_max, starts[c:c + 64],
                              lens[c:c + 64], ks[c:c + 64], sink_pages, gqa=gqa, select=select,
                              scale=scale, out=out[c:c + 64], pages_per_split=pages_per_split)
        return out
    if not back_to_back or starts[-1] + lens[-1] > T or v.shape != (T, H, D):
        for b, (t0, n) in enumerate(zip(starts, lens)):
            p0, p1 = t0 // 16, (t0 + n + 15) // 16
            decode_step(queries[b], compact_view(k, t0, t0 + n), kt, compact_view(v, t0, t0 + n), vt,
                        K_min[p0:p1], K_max[p0:p1], ks[b], sink_pages, gqa=gqa, select=select,
                        scale=scale, out=out[b], pages_per_split=pages_per_split)
        return out
    Hq = int(queries.shape[1])
    if Hq % H or int(queries.shape[2]) != D or queries.dtype != torch.float16:
        raise ValueError(f"queries {tuple(queries.shape)} incompatible with (T, H, D) = {(T, H, D)}")
    if tuple(out.shape) != (B, Hq, D) or out.dtype not in (torch.float16, torch.float32) or \
            not out.is_contiguous():
        raise AssertionError(f"out must be contiguous ({B}, {Hq}, {D}) fp16 or fp32")
    if kt.per_token or not vt.per_token:
        raise AssertionError("K scales are per-channel, V scales per-token")
    p0 = starts[0] // 16
    ptot = sum(pages)
    offs = [0]
    for n in pages:
        offs.append(offs[-1] + n)
    qs = queries.reshape(B, H, Hq // H, D).mean(dim=2).to(torch.float16) if gqa == "mean" else queries
    sel, rows, _ = quest_select_ragged(qs, K_min[p0:p0 + ptot], K_max[p0:p0 + ptot], offs, ks,
                                       sink_pages)
    dev = queries.device
    if select == "union":
        c_rows = (ctypes.c_int64 * (B + 1))(*rows)
        c_pages = (ctypes.c_int64 * (B + 1))(*offs)
        flags = N.workspace("union_flags", int(N.lib().hkv_union_pages_workspace_bytes(ptot)), dev)
        union = torch.empty((max(ptot, 1), H), dtype=torch.int64, device=dev)
        st = N.lib().hkv_union_pages_ragged(N.ptr(sel), H, B, c_rows, c_pages, N.ptr(union), N.ptr(flags),
                                            flags.numel(), N.stream_of(qs))
        N.check(st, "hkv_union_pages_ragged", ValueError)
        sel, sel_offs = union, offs
    else:
        sel_offs = rows
    nsel_all = sel_offs[-1]
    pps = int(pages_per_split) if pages_per_split else decode_pages_per_split(nsel_all, H)
    c_sel = (ctypes.c_int64 * (B + 1))(*sel_offs)
    c_tok = (ctypes.c_int64 * B)(*starts)
    c_len = (ctypes.c_int64 * B)(*lens)
    q = queries.contiguous()
    nb = int(N.lib().hkv_decode_batch_workspace_bytes(B, c_sel, Hq, pps))
    ws = N.workspace("decode", nb, dev)
    sc = float(scale) if scale is not None else D ** -0.5
    st = N.lib().hkv_decode_attn_batch(
        N.ptr(q), B, Hq, H, D, T, c_tok, c_len,
        N.ptr(k.packed), N.ptr(k.row_ptr), N.ptr(k.col), N.ptr(k.val),
        min(int(k.col.numel()), int(k.val.numel())), k.bits, N.ptr(kt.ensure_tables()),
        N.ptr(v.packed), N.ptr(v.row_ptr), N.ptr(v.col), N.ptr(v.val),
        min(int(v.col.numel()), int(v.val.numel())), v.bits, N.ptr(vt.ensure_tables()), vt.rows,
        N.ptr(sel), c_sel, pps, sc, N.ptr(out), N.dtype_code(out), N.ptr(ws), ws.numel(),
        N.stream_of(q))
    N.check(st, "hkv_decode_attn_batch", AssertionError)
    return out


def selected_attention(query: torch.Tensor, K_pages: torch.Tensor, V_pages: torch.Tensor,
                       page_indices: torch.Tensor, *, gqa: bool = False,
                       scale: float | None = None) -> torch.Tensor:
    """Attention of each query head over its selected dense pages
    (hkv_selected_attention).

    query (Hq, D); K_pages (P, page, Hk, D); V_pages (P, page, Hv, Dv);
    page_indices (n, Hq) or (n, Hk) int64.  gqa=False is the reference's head
    map (src/quest/reference.py:136-168: K head h, V head h % Hv, Hk == Hq);
    gqa=True maps query head h to KV head h // (Hq // Hk).  Returns (Hq, Dv) in
    query's dtype (fp16 / fp32 / bf16)."""
    N.require_gpu(query, K_pages, V_pages, page_indices)
    if query.dim() != 2 or K_pages.dim() != 4 or V_pages.dim() != 4 or page_indices.dim() != 2:
        raise ValueError("expected query (H, D), pages (P, page, H, D), page_indices (n, H)")
    Hq, D = (int(x) for x in query.shape)
    P, S, Hk, Dk = (int(x) for x in K_pages.shape)
    Pv, Sv, Hv, Dv = (int(x) for x in V_pages.shape)
    if Dk != D or Pv != P or Sv != S:
        raise ValueError(f"K_pages {tuple(K_pages.shape)} / V_pages {tuple(V_pages.shape)} do not "
                         f"match query {tuple(query.shape)}")
    kv_dt = K_pages.dtype
    k = K_pages.contiguous()
    v = V_pages.to(kv_dt).contiguous()
    q = query.contiguous()
    idx = page_indices.to(torch.int64).contiguous()
    nsel, cols = (int(x) for x in idx.shape)
    out = torch.empty((Hq, Dv), dtype=query.dtype, device=query.device)
    nb = int(N.lib().hkv_selected_attention_workspace_bytes(nsel, S, Hq, Dv))
    ws = N.workspace("selected_attention", nb, q.device)
    sc = float(scale) if scale is not None else D ** -0.5
    st = N.lib().hkv_selected_attention(
        N.ptr(q), N.dtype_code(q), Hq, D, N.ptr(k), N.ptr(v), N.dtype_code(k), P, S, Hk, Hv, Dv,
        N.ptr(idx), nsel, cols, 1 if gqa else 0, sc, N.ptr(out), N.dtype_code(out), N.ptr(ws),
        ws.numel(), N.stream_of(q))
    N.check(st, "hkv_selected_attention", ValueError)
    return out


# ------------------------------------------------------------ ragged batches

def _ragged_rows(page_offsets, top_k, sink_pages: int) -> list[int]:
    out = [0]
    for b in range(len(page_offsets) - 1):
        P = int(page_offsets[b + 1]) - int(page_offsets[b])
        s = max(0, min(int(sink_pages), P))
        keff = max(0, min(int(top_k[b]), P - s))
        out.append(out[-1] + s + keff)
    return out


def quest_select_ragged(query: torch.Tensor, K_min: torch.Tensor, K_max: torch.Tensor,
                        page_offsets, top_k, sink_pages: int, *,
                        scores: torch.Tensor | None = None):
    """Quest selection for a ragged batch of B decode queries (hkv_quest_select_ragged).

    query (B, Hq, D); K_min / K_max (P_total, H, D) fp16, sequence b owning
    pages page_offsets[b] .. page_offsets[b+1]-1; top_k an int or one per
    sequence.  Returns (sel (rows, H) int64 local page indices, ascending per
    sequence and head; out_offsets (B+1 ints): rows of sequence b are
    out_offsets[b] .. out_offsets[b+1]-1; scores (H, P_total) fp32)."""
    import ctypes

    N.require_gpu(query, K_min, K_max)
    if query.dim() != 3 or K_min.dim() != 3 or K_min.shape != K_max.shape:
        raise ValueError("query should be (B, Hq, D) and K_min/K_max (P_total, H, D)")
    B, Hq, D = (int(x) for x in query.shape)
    Ptot, H, Dk = (int(x) for x in K_min.shape)
    offs = [int(x) for x in page_offsets]
    if len(offs) != B + 1 or offs[0] != 0 or offs[-1] != Ptot or Dk != D or Hq % H:
        raise ValueError("page_offsets must be (B+1,) from 0 to P_total; shapes must agree")
    ks = [int(top_k)] * B if isinstance(top_k, int) else [int(x) for x in top_k]
    if len(ks) != B:
        raise ValueError("one top_k per sequence")
    rows = _ragged_rows(offs, ks, sink_pages)
    kmin = K_min.contiguous()
    kmax = K_max.to(kmin.dtype).contiguous()
    q = query.contiguous()
    out = torch.empty((max(rows[-1], 1), H), dtype=torch.int64, device=q.device)
    if scores is None:
        scores = torch.empty((H, max(Ptot, 1)), dtype=torch.float32, device=q.device)
    c_off = (ctypes.c_int64 * (B + 1))(*offs)
    c_k = (ctypes.c_int64 * B)(*ks)
    c_out = (ctypes.c_int64 * (B + 1))()
    st = N.lib().hkv_quest_select_ragged(N.ptr(q), N.dtype_code(q), B, Hq, N.ptr(kmin), N.ptr(kmax),
                                         N.dtype_code(kmin), H, D, c_off, c_k, int(sink_pages),
                                         N.ptr(scores), N.ptr(out), c_out, N.stream_of(q))
    N.check(st, "hkv_quest_select_ragged", ValueError)
    assert list(c_out) == rows
    return out[: rows[-1]], rows, scores[:, :Ptot]


def nuq_gather_pages(cc: CompactCodes, t: NuqLayerTables, sel: torch.Tensor, page_offsets,
                     out_offsets, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Gather + dequantise the selected (page, head) pairs of a compact K or V
    of B concatenated sequences into (rows, 16, H, 128) fp16
    (hkv_nuq_gather_pages); sel (rows, H) holds pages local to each sequence,
    as quest_select_ragged returns them with out_offsets."""
    import ctypes

    N.require_gpu(cc.packed, sel)
    T, H, D = cc.shape
    B = len(page_offsets) - 1
    rows = int(out_offsets[-1])
    if sel.dim() != 2 or int(sel.shape[1]) != H or int(sel.shape[0]) < rows:
        raise ValueError(f"sel should be ({rows}, {H})")
    if out is None:
        out = torch.empty((rows, 16, H, D), dtype=torch.float16, device=cc.packed.device)
    if tuple(out.shape) != (rows, 16, H, D) or out.dtype != torch.float16 or not out.is_contiguous():
        raise AssertionError(f"out must be contiguous ({rows}, 16, {H}, {D}) fp16")
    s = sel.to(torch.int64).contiguous()
    c_off = (ctypes.c_int64 * (B + 1))(*[int(x) for x in page_offsets])
    c_out = (ctypes.c_int64 * (B + 1))(*[int(x) for x in out_offsets])
    st = N.lib().hkv_nuq_gather_pages(
        N.ptr(cc.packed), N.ptr(cc.row_ptr), N.ptr(cc.col), N.ptr(cc.val),
        min(int(cc.col.numel()), int(cc.val.numel())), T, H, D, cc.bits, t.struct(), 16, B, c_off,
        c_out, N.ptr(s), N.ptr(out), N.stream_of(out))
    N.check(st, "hkv_nuq_gather_pages", AssertionError)
    return out


# ------------------------------------------------------------ calibration

def kmeans_1d(values: torch.Tensor, offsets: torch.Tensor, k: int, iters: int = 20) -> torch.Tensor:
    """Batched 1-D k-means (hkv_kmeans_1d): problem p is
    values[offsets[p]:offsets[p+1]] (fp32, finite); returns (n, k) fp32
    centres sorted ascending.  Replaces the sklearn fit of
    src/kvquant/calibration.py:106-123 (_kmeans_1d), one problem per call there;
    here every problem of a layer in one launch, with a deterministic start
    (centres evenly over [min, max]) and a fixed number of Lloyd steps."""
    N.require_gpu(values, offsets)
    if values.dim() != 1 or offsets.dim() != 1 or offsets.numel() < 1:
        raise ValueError("values must be (N,) and offsets (n + 1,)")
    v = values.to(torch.float32).contiguous()
    if v.numel() == 0:
        v = torch.zeros(1, dtype=torch.float32, device=values.device)
    off = offsets.to(torch.int64).contiguous()
    n = int(off.numel()) - 1
    centers = torch.empty((n, int(k)), dtype=torch.float32, device=values.device)
    st = N.lib().hkv_kmeans_1d(N.ptr(v), N.ptr(off), n, int(k), int(iters), N.ptr(centers),
                               N.stream_of(v))
    N.check(st, "hkv_kmeans_1d", ValueError)
    return centers


def kmeans_1d_optimal(values: torch.Tensor, offsets: torch.Tensor, k: int) -> torch.Tensor:
    """Batched optimal 1-D k-means (hkv_kmeans_1d_optimal): the problems of
    :func:`kmeans_1d`, each solved exactly by dynamic programming over its
    sorted values (at most 6144 values a problem; larger ones give NaN).
    Returns (n, k) fp32 centres sorted ascending."""
    N.require_gpu(values, offsets)
    if values.dim() != 1 or offsets.dim() != 1 or offsets.numel() < 1:
        raise ValueError("values must be (N,) and offsets (n + 1,)")
    v = values.to(torch.float32).contiguous()
    if v.numel() == 0:
        v = torch.zeros(1, dtype=torch.float32, device=values.device)
    off = offsets.to(torch.int64).contiguous()
    n = int(off.numel()) - 1
    centers = torch.empty((n, int(k)), dtype=torch.float32, device=values.device)
    ws = N.workspace("kmeans_dp", int(N.lib().hkv_kmeans_1d_optimal_workspace_bytes()), v.device)
    st = N.lib().hkv_kmeans_1d_optimal(N.ptr(v), N.ptr(off), n, int(k), N.ptr(centers), N.ptr(ws),
                                       ws.numel(), N.stream_of(v))
    N.check(st, "hkv_kmeans_1d_optimal", ValueError)
    return centers
