"""Tensor-level wrappers of the paged compact pool (hkv_paged_*).

One layer's K or V side of the pool (D = 128, 16 slots per block):
  codes (NB, H, 16, D*bits/8) u8 -- page-head blocks of bit-packed codes;
  ocnt (NB, H) int32, oent (NB, H, cap) int32 (u32 bit patterns: fp16 value |
  channel << 16 | slot << 24) -- each page-head's outliers, the first cap
  inline;
  ovf (NB, H) int32 -- the page-head's overflow chunk (-1: none) in ovf_ent
  (n_chunks, 2048 - cap), handed out from ovf_next when a page-head's
  outliers first pass cap;
  kmin / kmax (NB, H, D) fp16 -- K page statistics of the dequantised values;
  status (1,) int32 -- bit 0 once outliers were dropped (no room left).
Calls launch on torch's current stream and read nothing back.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native as N
from .ops import NuqLayerTables, union_pages

PAGE = 16
HEAD_DIM = 128
PAGE_ELEMS = PAGE * HEAD_DIM
DEFAULT_CAP = PAGE_ELEMS // 8   # 256 inline entries: 12.5% of a page-head


def bits_for_levels(levels: int) -> int:
    if levels <= 4:
        return 2
    if levels <= 16:
        return 4
    raise ValueError(f"{levels} levels exceed nuq4")


@dataclass
class PagedSide:
    codes: torch.Tensor
    ocnt: torch.Tensor
    oent: torch.Tensor
    bits: int
    ovf: torch.Tensor | None = None
    ovf_ent: torch.Tensor | None = None
    ovf_next: torch.Tensor | None = None
    kmin: torch.Tensor | None = None
    kmax: torch.Tensor | None = None
    status: torch.Tensor | None = None

    @property
    def num_blocks(self) -> int:
        return int(self.codes.shape[0])

    @property
    def heads(self) -> int:
        return int(self.codes.shape[1])

    @property
    def cap(self) -> int:
        return int(self.oent.shape[2])

    @property
    def n_chunks(self) -> int:
        return 0 if self.ovf_ent is None else int(self.ovf_ent.shape[0])

    @staticmethod
    def empty(num_blocks: int, H: int, bits: int, cap: int = DEFAULT_CAP, device="cuda",
              stats: bool = False, n_chunks: int | None = None) -> "PagedSide":
        """A zeroed side.  n_chunks overflow chunks of 2048 - cap entries
        (default: one per 8 page-heads; 0: no arena, outliers past cap are
        dropped and flagged)."""
        dev = torch.device(device)
        if not 0 <= cap <= PAGE_ELEMS:
            raise ValueError(f"cap must be in [0, {PAGE_ELEMS}]")
        if n_chunks is None:
            n_chunks = max(1, num_blocks * H // 8) if cap < PAGE_ELEMS else 0
        side = PagedSide(
            codes=torch.zeros((num_blocks, H, PAGE, HEAD_DIM * bits // 8), dtype=torch.uint8, device=dev),
            ocnt=torch.zeros((num_blocks, H), dtype=torch.int32, device=dev),
            oent=torch.zeros((num_blocks, H, cap), dtype=torch.int32, device=dev),
            bits=bits,
            status=torch.zeros(1, dtype=torch.int32, device=dev))
        if n_chunks > 0:
            side.ovf = torch.full((num_blocks, H), -1, dtype=torch.int32, device=dev)
            side.ovf_ent = torch.zeros((n_chunks, PAGE_ELEMS - cap), dtype=torch.int32, device=dev)
            side.ovf_next = torch.zeros(1, dtype=torch.int32, device=dev)
        if stats:
            side.kmin = torch.full((num_blocks, H, HEAD_DIM), float("inf"), dtype=torch.float16, device=dev)
            side.kmax = torch.full((num_blocks, H, HEAD_DIM), float("-inf"), dtype=torch.float16, device=dev)
        return side

    def desc(self) -> N.PagedSideDesc:
        d = N.PagedSideDesc()
        for name in ("codes", "ocnt", "oent", "ovf", "ovf_ent", "ovf_next", "kmin", "kmax", "status"):
            t = getattr(self, name)
            setattr(d, name, None if t is None else t.data_ptr())
        d.num_blocks = self.num_blocks
        d.heads = self.heads
        d.bits = self.bits
        d.cap = self.cap
        d.n_chunks = self.n_chunks
        return d

    def all_entries(self) -> torch.Tensor:
        """Every page-head's entry slots in order, (NB, H, 2048) int32 on the
        device: the cap inline ones, then the overflow chunk's (zeros where a
        page-head has none).  The first min(ocnt, stored) are live."""
        full = torch.zeros((self.num_blocks, self.heads, PAGE_ELEMS), dtype=torch.int32,
                           device=self.codes.device)
        full[:, :, : self.cap] = self.oent
        if self.ovf is not None:
            m = self.ovf >= 0
            full[:, :, self.cap:][m] = self.ovf_ent[self.ovf[m].long()]
        return full

    def entries(self, block: int, head: int) -> torch.Tensor:
        """The page-head's stored outlier entries in order (host read)."""
        n = int(self.ocnt[block, head])
        inline = self.oent[block, head, : min(n, self.cap)]
        if n <= self.cap or self.ovf is None or int(self.ovf[block, head]) < 0:
            return inline
        rest = self.ovf_ent[int(self.ovf[block, head]), : n - self.cap]
        return torch.cat([inline, rest])


def paged_write(side: PagedSide, values: torch.Tensor, t: NuqLayerTables, slot_mapping: torch.Tensor,
                positions: torch.Tensor | None = None) -> None:
    """Write (T, H, 128) fp16 into the side's slots (hkv_paged_write); V
    (per-token scales) uses scale row min(positions[t], rows - 1)."""
    N.require_gpu(values, slot_mapping, side.codes)
    assert values.dtype == torch.float16, "values must be fp16"
    assert values.is_contiguous(), "values must be contiguous (T, H, D)"
    T = int(values.shape[0])
    H = side.heads
    if tuple(values.shape) != (T, H, HEAD_DIM):
        raise AssertionError(f"values must be ({T}, {H}, {HEAD_DIM}), got {tuple(values.shape)}")
    if t.levels > (1 << side.bits):
        raise AssertionError(f"{t.levels} levels do not fit in {side.bits} bits")
    if t.per_token and side.kmin is not None:
        raise AssertionError("page statistics are kept for K (per-channel scales) only")
    slots = slot_mapping.to(torch.int64).contiguous()
    if slots.numel() != T:
        raise AssertionError("slot_mapping must have one entry per token")
    pos = None
    if positions is not None:
        pos = positions.to(device=values.device, dtype=torch.int64).contiguous()
        if pos.numel() != T:
            raise AssertionError("positions must have one entry per token")
    if T == 0:
        return
    st = N.lib().hkv_paged_write(N.ptr(values), T, t.struct(pos), N.ptr(slots), side.desc(),
                                 N.stream_of(values))
    N.check(st, "hkv_paged_write", AssertionError)


def paged_gather(side: PagedSide, t: NuqLayerTables, block_ids: torch.Tensor,
                 first_pos: torch.Tensor | None = None, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """Dequantise blocks block_ids into (NK, 16, H, 128) fp16 (hkv_paged_gather);
    V rows min(first_pos[k] + slot, rows - 1)."""
    N.require_gpu(block_ids, side.codes)
    ids = block_ids.to(torch.int64).contiguous()
    NK = int(ids.numel())
    H = side.heads
    if out is None:
        out = torch.empty((NK, PAGE, H, HEAD_DIM), dtype=torch.float16, device=side.codes.device)
    if tuple(out.shape) != (NK, PAGE, H, HEAD_DIM) or out.dtype != torch.float16 or not out.is_contiguous():
        raise AssertionError(f"staging must be contiguous ({NK}, {PAGE}, {H}, {HEAD_DIM}) fp16")
    fp = None
    if t.per_token:
        if first_pos is None:
            raise AssertionError("per-token scales need block first positions")
        fp = first_pos.to(device=ids.device, dtype=torch.int64).contiguous()
        if fp.numel() != NK:
            raise AssertionError("one first position per kept block")
    if NK == 0:
        return out
    st = N.lib().hkv_paged_gather(side.desc(), t.struct(), N.ptr(ids), N.ptr(fp), NK, N.ptr(out),
                                  N.stream_of(out))
    N.check(st, "hkv_paged_gather", AssertionError)
    return out


def _block_table(block_table: torch.Tensor, P: int) -> torch.Tensor:
    bt = block_table.to(torch.int64).contiguous()
    if bt.dim() != 1 or int(bt.numel()) < P:
        raise ValueError(f"block_table must list at least {P} blocks, got {tuple(bt.shape)}")
    return bt


def paged_select(query: torch.Tensor, kside: PagedSide, block_table: torch.Tensor, seq_len: int,
                 k: int, sink_pages: int, *, scores: torch.Tensor | None = None,
                 out: torch.Tensor | None = None):
    """Quest selection over the K page statistics of a paged sequence
    (hkv_quest_select_paged): logical page p of the sequence's ceil(seq_len /
    16) pages reads block block_table[p].  query (Hq, 128), Hq a multiple of
    H (the group's bounds summed; pass one query per KV head for the plain
    bound).  Returns (logical pages (sinks + k_eff, H) int64 ascending per
    head, scores (H, P) fp32)."""
    N.require_gpu(query, block_table)
    if kside.kmin is None:
        raise ValueError("the side holds no page statistics (K written with stats)")
    P = -(-int(seq_len) // PAGE)
    H = kside.heads
    Hq = int(query.shape[0])
    if query.dim() != 2 or int(query.shape[1]) != HEAD_DIM or Hq % H:
        raise ValueError(f"query {tuple(query.shape)} incompatible with {H} KV heads x {HEAD_DIM}")
    bt = _block_table(block_table, P)
    q = query.contiguous()
    s = max(0, min(int(sink_pages), P))
    keff = max(0, min(int(k), P - s))
    if out is None:
        out = torch.empty((s + keff, H), dtype=torch.int64, device=q.device)
    if scores is None:
        scores = torch.empty((H, max(P, 1)), dtype=torch.float32, device=q.device)
    n_out = N._i64(0)
    ws = N.workspace("quest_select", int(N.lib().hkv_quest_select_workspace_bytes(P, H)), q.device)
    st = N.lib().hkv_quest_select_paged(
        N.ptr(q), N.dtype_code(q), Hq, kside.desc(), N.ptr(bt), P, int(k), int(sink_pages),
        N.ptr(scores), N.ptr(out), n_out, N.ptr(ws), ws.numel(), N.stream_of(q))
    N.check(st, "hkv_quest_select_paged", ValueError)
    return out, scores


def paged_select_ragged(queries: torch.Tensor, kside: PagedSide, block_tables: torch.Tensor,
                        seq_lens, top_k, sink_pages: int, *, scores: torch.Tensor | None = None):
    """paged_select for B <= 64 sequences of one pool in one bound launch and
    one top-K launch (hkv_quest_select_paged_ragged): sequence b has
    seq_lens[b] tokens, query queries[b] (Hq, 128) and its logical page p at
    block block_tables[b, p].  The pool's KV heads must divide 4.  Returns
    (sel (rows, H) int64 logical pages, ascending per sequence and head;
    out_offsets (B+1 ints), the rows of sequence b; scores (H, total pages)
    fp32, sequence b's at columns out of the running page count)."""
    import ctypes
    from .ops import _ragged_rows

    N.require_gpu(queries, block_tables)
    if kside.kmin is None:
        raise ValueError("the side holds no page statistics (K written with stats)")
    lens = [int(n) for n in seq_lens]
    B = len(lens)
    H = kside.heads
    if queries.dim() != 3 or int(queries.shape[0]) != B or int(queries.shape[2]) != HEAD_DIM or \
            int(queries.shape[1]) % H:
        raise ValueError(f"queries {tuple(queries.shape)} incompatible with {B} sequences, {H} KV heads")
    if 16 % H:
        raise ValueError(f"the ragged paged selection needs 1, 2, 4, 8 or 16 KV heads, not {H}")
    pages = [-(-n // PAGE) for n in lens]
    if block_tables.dim() != 2 or int(block_tables.shape[0]) != B or \
            int(block_tables.shape[1]) < max(pages, default=0):
        raise ValueError(f"block_tables must be ({B}, >= {max(pages, default=0)}), got "
                         f"{tuple(block_tables.shape)}")
    M = int(block_tables.shape[1])
    bt = block_tables.to(torch.int64).contiguous()
    offs = [0]
    for P in pages:
        offs.append(offs[-1] + P)
    ks = [int(top_k)] * B if not hasattr(top_k, '__len__') else [int(x) for x in top_k]
    if len(ks) != B:
        raise ValueError("one top_k per sequence")
    rows = _ragged_rows(offs, ks, sink_pages)
    q = queries.contiguous()
    out = torch.empty((max(rows[-1], 1), H), dtype=torch.int64, device=q.device)
    if scores is None:
        scores = torch.empty((H, max(offs[-1], 1)), dtype=torch.float32, device=q.device)
    c_off = (ctypes.c_int64 * (B + 1))(*offs)
    c_k = (ctypes.c_int64 * B)(*ks)
    c_bt = (ctypes.c_int64 * B)(*[b * M for b in range(B)])
    c_out = (ctypes.c_int64 * (B + 1))()
    st = N.lib().hkv_quest_select_paged_ragged(
        N.ptr(q), N.dtype_code(q), B, int(q.shape[1]), kside.desc(), N.ptr(bt), c_bt, c_off, c_k,
        int(sink_pages), N.ptr(scores), N.ptr(out), c_out, N.stream_of(q))
    N.check(st, "hkv_quest_select_paged_ragged", ValueError)
    assert list(c_out) == rows
    return out[: rows[-1]], rows, scores[:, : offs[-1]]


def paged_decode_attention(query: torch.Tensor, kside: PagedSide, kt: NuqLayerTables,
                           vside: PagedSide, vt: NuqLayerTables, block_table: torch.Tensor,
                           seq_len: int, sel: torch.Tensor, *, scale: float | None = None,
                           pages_per_split: int | None = None, out: torch.Tensor | None = None,
                           out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """softmax(q.K^T * scale).V per query head over its KV head's selected
    logical pages of a paged sequence (hkv_paged_decode_attn).  query
    (Hq, 128) fp16; sel (n, H) logical pages; query head hq uses KV head
    hq // (Hq // H).  Returns (Hq, 128)."""
    from .ops import decode_pages_per_split

    N.require_gpu(query, sel, block_table)
    H = kside.heads
    Hq = int(query.shape[0])
    if query.dim() != 2 or int(query.shape[1]) != HEAD_DIM or Hq % H:
        raise ValueError(f"query {tuple(query.shape)} incompatible with {H} KV heads x {HEAD_DIM}")
    if query.dtype != torch.float16:
        raise AssertionError("query must be fp16")
    if kt.per_token or not vt.per_token:
        raise AssertionError("K scales are per-channel, V scales per-token")
    if vside.heads != H or vside.num_blocks != kside.num_blocks:
        raise AssertionError("K and V sides must have the same blocks and heads")
    if sel.dim() != 2 or int(sel.shape[1]) != H:
        raise ValueError(f"sel should be (n, {H}), got {tuple(sel.shape)}")
    T = int(seq_len)
    if T < 1:
        raise ValueError("the sequence must hold at least one token")
    bt = _block_table(block_table, -(-T // PAGE))
    s = sel.to(torch.int64).contiguous()
    nsel = int(s.shape[0])
    pps = int(pages_per_split) if pages_per_split else decode_pages_per_split(nsel, H)
    q = query.contiguous()
    if out is None:
        out = torch.empty((Hq, HEAD_DIM), dtype=out_dtype, device=q.device)
    if tuple(out.shape) != (Hq, HEAD_DIM) or out.dtype not in (torch.float16, torch.float32):
        raise AssertionError("out must be (Hq, 128) fp16 or fp32")
    nb = int(N.lib().hkv_decode_workspace_bytes(nsel, Hq, pps))
    ws = N.workspace("decode", nb, q.device)
    sc = float(scale) if scale is not None else HEAD_DIM ** -0.5
    st = N.lib().hkv_paged_decode_attn(
        N.ptr(q), Hq, T, N.ptr(bt), kside.desc(), N.ptr(kt.ensure_tables()), vside.desc(),
        N.ptr(vt.ensure_tables()), vt.rows, N.ptr(s), nsel, pps, sc, N.ptr(out), N.dtype_code(out),
        N.ptr(ws), ws.numel(), N.stream_of(q))
    N.check(st, "hkv_paged_decode_attn", AssertionError)
    return out


def paged_decode_step(query: torch.Tensor, kside: PagedSide, kt: NuqLayerTables, vside: PagedSide,
                      vt: NuqLayerTables, block_table: torch.Tensor, seq_len: int, top_k: int,
                      sink_pages: int = 4, *, gqa: str = "mean", select: str = "union",
                      scale: float | None = None, out: torch.Tensor | None = None,
                      out_dtype: torch.dtype = torch.float16,
                      pages_per_split: int | None = None) -> torch.Tensor:
    """One decode step of one paged sequence, with no host reads (graph
    capturable): Quest selection from the pool's K page statistics through
    the block table, then the fused dequant + attention over the selected
    logical pages.  The compact backend's forward (src/kvquant/
    compact_backend.py:194-299) without its host synchronisations, with the
    sinks the first logical pages and positions from the block table (not
    block id * block size, src/kvquant/quest_selector.py:85-89):
      gqa="mean": the group's queries averaged per KV head, in fp16
      (compact_backend.py:225-231); "sum": the group's bounds summed.
      select="union": every head attends to the union of the heads' pages
      (quest_selector.py:80); "per_head": each KV head to its own."""
    H = kside.heads
    Hq = int(query.shape[0])
    if query.dim() != 2 or Hq % H or int(query.shape[1]) != HEAD_DIM:
        raise ValueError(f"query {tuple(query.shape)} incompatible with {H} KV heads x {HEAD_DIM}")
    if gqa == "mean":
        qs = query.reshape(H, Hq // H, HEAD_DIM).mean(dim=1).to(torch.float16)
    elif gqa == "sum":
        qs = query
    else:
        raise ValueError(f"gqa must be 'mean' or 'sum', got {gqa!r}")
    P = -(-int(seq_len) // PAGE)
    sel, _ = paged_select(qs, kside, block_table, seq_len, top_k, sink_pages)
    if select == "union":
        sel = union_pages(sel, P)
    elif select != "per_head":
        raise ValueError(f"select must be 'union' or 'per_head', got {select!r}")
    return paged_decode_attention(query, kside, kt, vside, vt, block_table, seq_len, sel, scale=scale,
                                  pages_per_split=pages_per_split, out=out, out_dtype=out_dtype)


def paged_decode_step_batch(queries: torch.Tensor, kside: PagedSide, kt: NuqLayerTables,
                            vside: PagedSide, vt: NuqLayerTables, block_tables: torch.Tensor,
                            seq_lens, top_k, sink_pages: int = 4, *, gqa: str = "mean",
                            select: str = "union", scale: float | None = None,
                            out: torch.Tensor | None = None,
                            out_dtype: torch.dtype = torch.float16,
                            pages_per_split: int | None = None) -> torch.Tensor:
    """paged_decode_step for B sequences of one pool, with no host reads:
    sequence b has seq_lens[b] tokens, query queries[b] and its logical page p
    in block block_tables[b, p] (block_tables (B, M) as the attention
    metadata's block table, M >= ceil(seq_lens[b] / 16)).  One ragged Quest
    selection (hkv_quest_select_paged_ragged; one paged selection per sequence
    where the pool's KV heads do not divide 16), the per-sequence union of the
    heads' pages for select="union" (hkv_union_pages_ragged), then one batched
    decode + merge (hkv_paged_decode_attn_batch), per batch of up to 64
    sequences; each sequence's result equals paged_decode_step's with the
    same pages_per_split.  The reference forward
    falls back to dense attention for batches above one
    (src/kvquant/compact_backend.py:195-203).  top_k: one int, or one per
    sequence.  queries (B, Hq, 128) fp16; returns (B, Hq, 128)."""
    import ctypes
    from .ops import decode_pages_per_split

    N.require_gpu(queries, block_tables)
    lens = [int(n) for n in seq_lens]
    B = len(lens)
    H = kside.heads
    if queries.dim() != 3 or int(queries.shape[0]) != B or int(queries.shape[2]) != HEAD_DIM:
        raise ValueError(f"queries {tuple(queries.shape)} do not match {B} sequences x {HEAD_DIM}")
    Hq = int(queries.shape[1])
    if Hq % H or queries.dtype != torch.float16:
        raise ValueError(f"queries {tuple(queries.shape)} {queries.dtype}: fp16 with a multiple of {H} heads")
    if B < 1:
        raise ValueError("no sequences")
    if B > 64:  # batches of 64 (each one launch of the decode)
        if out is None:
            out = torch.empty((B, Hq, HEAD_DIM), dtype=out_dtype, device=queries.device)
        ks_all = [int(top_k)] * B if not hasattr(top_k, '__len__') else [int(x) for x in top_k]
        if len(ks_all) != B:
            raise ValueError("one top_k per sequence")
        for c in range(0, B, 64):
            paged_decode_step_batch(queries[c:c + 64], kside, kt, vside, vt, block_tables[c:c + 64],
                                    lens[c:c + 64], ks_all[c:c + 64], sink_pages, gqa=gqa,
                                    select=select, scale=scale, out=out[c:c + 64], out_dtype=out_dtype,
                                    pages_per_split=pages_per_split)
        return out
    if any(n < 1 for n in lens):
        raise ValueError("sequence lengths must be positive")
    ks = [int(top_k)] * B if not hasattr(top_k, '__len__') else [int(x) for x in top_k]
    if len(ks) != B:
        raise ValueError("one top_k per sequence")
    if gqa not in ("mean", "sum"):
        raise ValueError(f"gqa must be 'mean' or 'sum', got {gqa!r}")
    if select not in ("union", "per_head"):
        raise ValueError(f"select must be 'union' or 'per_head', got {select!r}")
    if kt.per_token or not vt.per_token:
        raise AssertionError("K scales are per-channel, V scales per-token")
    if vside.heads != H or vside.num_blocks != kside.num_blocks:
        raise AssertionError("K and V sides must have the same blocks and heads")
    pages = [-(-n // PAGE) for n in lens]
    if block_tables.dim() != 2 or int(block_tables.shape[0]) != B or \
            int(block_tables.shape[1]) < max(pages):
        raise ValueError(f"block_tables must be ({B}, >= {max(pages)}), got {tuple(block_tables.shape)}")
    M = int(block_tables.shape[1])
    bt = block_tables.to(torch.int64).contiguous()
    dev = queries.device
    if out is None:
        out = torch.empty((B, Hq, HEAD_DIM), dtype=out_dtype, device=dev)
    if tuple(out.shape) != (B, Hq, HEAD_DIM) or out.dtype not in (torch.float16, torch.float32) or \
            not out.is_contiguous():
        raise AssertionError(f"out must be contiguous ({B}, {Hq}, {HEAD_DIM}) fp16 or fp32")
    q = queries.contiguous()
    qs = q.reshape(B, H, Hq // H, HEAD_DIM).mean(dim=2).to(torch.float16) if gqa == "mean" else q
    sp = int(sink_pages)
    offs = [0]
    for P in pages:
        offs.append(offs[-1] + P)
    if 16 % H == 0:
        sel, rows, _ = paged_select_ragged(qs, kside, bt, lens, ks, sp)
    else:  # a bound lane cannot hold a fixed head: one selection per sequence
        from .ops import _ragged_rows

        rows = _ragged_rows(offs, ks, sp)
        sel = torch.empty((max(rows[-1], 1), H), dtype=torch.int64, device=dev)
        scores = torch.empty((H * max(pages),), dtype=torch.float32, device=dev)
        for b in range(B):
            paged_select(qs[b], kside, bt[b], lens[b], ks[b], sp, out=sel[rows[b]:rows[b + 1]],
                         scores=scores[:H * pages[b]].view(H, pages[b]))
    if select == "union":
        c_rows = (ctypes.c_int64 * (B + 1))(*rows)
        c_pages = (ctypes.c_int64 * (B + 1))(*offs)
        flags = N.workspace("union_flags", int(N.lib().hkv_union_pages_workspace_bytes(offs[-1])), dev)
        union = torch.empty((offs[-1], H), dtype=torch.int64, device=dev)
        st = N.lib().hkv_union_pages_ragged(N.ptr(sel), H, B, c_rows, c_pages, N.ptr(union),
                                            N.ptr(flags), flags.numel(), N.stream_of(qs))
        N.check(st, "hkv_union_pages_ragged", ValueError)
        sel, sel_offs = union, offs
    else:
        sel_offs = rows
    pps = int(pages_per_split) if pages_per_split else decode_pages_per_split(sel_offs[-1], H)
    c_sel = (ctypes.c_int64 * (B + 1))(*sel_offs)
    c_len = (ctypes.c_int64 * B)(*lens)
    c_bt = (ctypes.c_int64 * B)(*[b * M for b in range(B)])
    nb = int(N.lib().hkv_decode_batch_workspace_bytes(B, c_sel, Hq, pps))
    ws = N.workspace("decode", nb, dev)
    sc = float(scale) if scale is not None else HEAD_DIM ** -0.5
    st = N.lib().hkv_paged_decode_attn_batch(
        N.ptr(q), B, Hq, c_len, N.ptr(bt), c_bt, kside.desc(), N.ptr(kt.ensure_tables()),
        vside.desc(), N.ptr(vt.ensure_tables()), vt.rows, N.ptr(sel), c_sel, pps, sc, N.ptr(out),
        N.dtype_code(out), N.ptr(ws), ws.numel(), N.stream_of(q))
    N.check(st, "hkv_paged_decode_attn_batch", AssertionError)
    return out
