// nuq_compact.hip -- nuq pack into the compact format (its inverse is in nuq_unpack.hip).
//
// Format (this build's; the reference planned but never implemented it:
// src/kvquant/triton_kernels.py:7-18, src/kvquant/compact_pool.py:11-12):
//   packed codes (T,H,D*bits/8) u8, little-endian within a byte
//     nuq4: byte j = c[2j] | c[2j+1] << 4
//     nuq2: byte j = c[4j] | c[4j+1] << 2 | c[4j+2] << 4 | c[4j+3] << 6
//   CSR outliers over rows r = t*H + h: row_ptr (T*H+1) int32, col u8 = d,
//   val fp16 = the original value; (row, col) ascending.
//
// Pack is one kernel (pack_fused_kernel): waves take chunks of rows from a
// work counter, write the packed codes as they go, hold the chunk's outliers
// in LDS, and place them (and row_ptr) once a decoupled look-back over the
// chunks' published counts has given the chunk's offset.  One launch packs up
// to kPackItems tensors of the same kernel variant (a layer's K, or the K of
// many layers), so a whole prefill step takes a few launches.
#include "nuq_launch.h"

#include <vector>

namespace {

// Passes of 64/G rows per wave tile: 4 (smaller tiles, fewer registers, more
// waves a SIMD), or 8 for per-channel tables of up to 8 levels, whose search
// state is small enough that the longer tile's loads pay off (131072-token
// layers, us per stage kernel, 8 -> 4 passes: K nuq2 49.2 -> 50.5, V nuq2
// 48.1 -> 42.8, V nuq4 64.8 -> 59.3).
__host__ __device__ constexpr int pack_passes(bool per_token, int nb) { return (!per_token && nb < 4) ? 8 : 4; }

constexpr int kPackItems = kBatchItems;        // tensors per fused pack launch
constexpr int kPackWaveRows = 128;             // least rows a wave packs per chunk (per-token: half)
constexpr uint32_t kPackSpinLimit = 1u << 20;  // look-back rounds without progress before giving up
constexpr int kPackLookWindows = 8;            // look-back windows of 64 chunks read at once
constexpr size_t kPackHeader = 256;            // workspace header bytes

// One tensor of a fused pack launch (kernel argument, by value).
struct PackItem {
  const uint16_t* x;
  uint8_t* packed;
  int32_t* row_ptr;
  uint8_t* col;
  uint16_t* val;
  hkv_nuq_scales sc;
  int64_t nrows;
  uint32_t chunk0;  // number of the item's first chunk
  uint32_t cap;     // col / val capacity
};
struct PackBatch {
  PackItem it[kPackItems];
  int32_t n;
  int32_t H;  // heads (the same for every item of a launch)
  uint32_t nchunks;
  int32_t wr;  // rows of a wave's part of a chunk: whole wave tiles, at most the variant's WR
};

// Rows a wave packs per chunk: whole wave tiles, at least kPackWaveRows
// (per-token scales: half as many, so the two chunks' outliers a wave holds
// leave room for five blocks per CU).  A chunk is NW such parts, one per wave
// of a block.
__host__ __device__ constexpr int pack_tile_rows(int G, int passes) { return (64 / G) * passes; }
__host__ __device__ constexpr int pack_wave_rows(int G, int passes, bool per_token) {
  return pack_tile_rows(G, passes) >= (per_token ? kPackWaveRows / 2 : kPackWaveRows)
             ? pack_tile_rows(G, passes)
             : (per_token ? kPackWaveRows / 2 : kPackWaveRows);
}
__host__ __device__ constexpr int pack_chunk_rows(int G, int passes, bool per_token) {
  return (kThreads / 64) * pack_wave_rows(G, passes, per_token);
}
// Outliers of its part of a chunk a wave holds in LDS (one in ten elements);
// a part with more writes the rest when its chunk is flushed (pack_redo_rows).
__host__ __device__ constexpr int pack_ent_cap(int G, int passes, bool per_token) {
  return (pack_wave_rows(G, passes, per_token) * 8 * G / 10 + 63) & ~63;
}


HKV_DEV uint32_t wave_sum(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, 64);
  return v;
}

// v, hidden from the optimiser: item fields loaded through it are loaded
// again where they are used instead of being kept in scalar registers
// across the packing loop.
HKV_DEV int opaque_s(int v) {
  v = __builtin_amdgcn_readfirstlane(v);
  asm volatile("" : "+s"(v));
  return v;
}

// Chunk status words: epoch (24 bits) | flags (8 bits) | count (32 bits).
// kStAgg: the chunk's own outlier count; kStInc: the count of the tensor's
// chunks up to and including this one.  A word whose epoch is not the
// launch's (left by an earlier launch, or zero) counts as not yet written.
constexpr uint64_t kStAgg = 1, kStInc = 2;
HKV_DEV uint64_t st_word(uint32_t epoch, uint64_t flag, uint32_t v) {
  return ((uint64_t)(epoch & 0xffffffu) << 40) | (flag << 32) | v;
}
HKV_DEV void st_publish(uint64_t* p, uint64_t w) {
  __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The outliers of a chunk at chunk positions >= ecap (more than its wave's
// LDS holds; rare), found again from the input with the defining fp32
// threshold compare (v > upper || v < lower, as slow_one) and written at
// their final places.  Row r's outliers start at chunk position roff[r]; a
// row's lanes take two channels each, in channel order, so a ballot gives
// each outlier's rank within the row.
template <int D>
HKV_DEV void pack_redo_rows(const PackItem& it, int H, int64_t rbeg, int nrc, const uint16_t* roff,
                            uint32_t run, uint32_t base, uint32_t ecap, int lane) {
  const hkv_nuq_scales& sc = it.sc;
  const SlowInfo si = slow_info(sc);
#pragma unroll 1
  for (int rr = 0; rr < nrc; ++rr) {
    const uint32_t end = rr + 1 < nrc ? roff[rr + 1] : run;
    if (end <= ecap) continue;  // all of the row's entries were kept
    const int64_t r = rbeg + rr;
    const int64_t t = r / H;
    const int h = (int)(r - t * H);
    const int64_t trow = sc.per_token ? (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows) : 0;
    uint32_t o = roff[rr];
#pragma unroll 1
    for (int d0 = 0; d0 < D; d0 += 128) {
      const int d = d0 + 2 * lane;
      uint32_t xw = 0;
      int f0 = 0, f1 = 0;
      if (d < D) {
        xw = *reinterpret_cast<const uint32_t*>(it.x + r * D + d);
        const int64_t ta = sc.per_token ? trow : (int64_t)h * D + d;
        const int64_t tb = sc.per_token ? trow : ta + 1;
        const float v0 = h2f((uint16_t)(xw & 0xffffu)), v1 = h2f((uint16_t)(xw >> 16));
        f0 = (v0 > load_scale(si.upper, si.tdt, ta)) || (v0 < load_scale(si.lower, si.tdt, ta));
        f1 = (v1 > load_scale(si.upper, si.tdt, tb)) || (v1 < load_scale(si.lower, si.tdt, tb));
      }
      const uint64_t b0 = __ballot(f0), b1 = __ballot(f1);
      const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
      // elements before lane's first: both elements of every lower lane
      uint32_t q = o + (uint32_t)__popcll(b0 & below) + (uint32_t)__popcll(b1 & below);
      if (f0) {
        if (q >= ecap && base + q < it.cap) {
          it.col[base + q] = (uint8_t)d;
          it.val[base + q] = (uint16_t)(xw & 0xffffu);
        }
        ++q;
      }
      if (f1 && q >= ecap && base + q < it.cap) {
        it.col[base + q] = (uint8_t)(d + 1);
        it.val[base + q] = (uint16_t)(xw >> 16);
      }
      o += (uint32_t)__popcll(b0) + (uint32_t)__popcll(b1);
    }
  }
}

// The exact-scan inputs of a batch item, loaded where the rare exact scan
// needs them.
struct ItemSlow {
  const PackBatch* b;
  int j;
  HKV_DEV SlowInfo get() const { return slow_info(b->it[opaque_s(j)].sc); }
};

// Fused pack.  A launch packs up to kPackItems tensors of one kernel variant.
// Their rows are cut into chunks of NW * wr rows, numbered consecutively over
// the tensors.  A block takes the next chunk number from the work counter (one
// device-scope atomic per chunk: those on one address serialise at about
// 11 ns each on MI355X, so a chunk is large, wr = WR rows a wave, except in a
// launch too small to give every CU two such chunks); each wave packs its wr
// rows (codes straight to HBM, outliers and each row's offset within
// the wave's part into its LDS).  After a block barrier wave 0 publishes the
// chunk's count and takes the next number; the chunk's offset (the outliers
// of the tensor's earlier chunks) is found one chunk later, by a decoupled
// look-back over the status words once the block has packed its next chunk,
// so the earlier chunks, which were packed concurrently, have published their
// counts by then and the look-back rarely waits; every wave then writes the
// held chunk's row_ptr and outliers at their final places (its LDS holds two
// chunks).  Chunk numbers are handed out in increasing order, a chunk's count
// is published as soon as it is packed, and a look-back waits only for counts
// of lower chunks, held by running blocks: the scheme cannot deadlock.  The
// status words and the counters are accessed with device-scope relaxed
// atomics only (they carry the counts themselves; no other data crosses
// blocks), so no cache write-back is needed across the eight XCDs' L2s.
//
// The header holds the work counter, a count of finished blocks and the
// epoch; the last block to finish resets the counters and advances the epoch,
// so a zero-filled workspace serves any number of later launches in stream
// order.
//
// KFIX: the rows of one pass of a wave (RW = 64/G) are a multiple of H, so a
// lane's head is fixed (rw % H) and its token advances by RW / H per pass.
template <int NB, bool PT, int G, int BITS, bool KFIX, int PASSES>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(PT ? 5 : 3)))
pack_fused_kernel(const PackBatch B, uint32_t* __restrict__ hdr, uint64_t* __restrict__ status) {
  constexpr int RW = 64 / G;        // rows per wave per pass
  constexpr int WT = RW * PASSES;  // rows per wave tile
  constexpr int D = 8 * G;
  constexpr int RB = D * BITS / 8;  // packed bytes per row
  constexpr int NW = kThreads / 64;
  constexpr int WR = pack_wave_rows(G, PASSES, PT);  // most rows of a wave's part of a chunk
  constexpr int ECAP = pack_ent_cap(G, PASSES, PT);
  static_assert(WR % WT == 0 && NW * WR == pack_chunk_rows(G, PASSES, PT), "a part is whole wave tiles");
  // Per-token tables of a wave tile's rows are staged in the wave's LDS slice
  // when they fit in 4 KiB (D >= 128), already in search form (each
  // breakpoint and threshold duplicated into both 16-bit halves: words 0..14
  // breakpoints, 15 lower, 16 upper, 17 fast-path bound), so a row's lanes
  // read them without unpacking; otherwise each row reads its table through L1.
  constexpr bool STAGE = PT && WT * 80 <= 4096;
  constexpr int TW = 20;  // staged words per row (80 bytes, 16-byte aligned)
  __shared__ __align__(16) uint32_t s_tab[STAGE ? NW * WT * TW : 1];
  // each lane's current 8 values, read back by element index in the
  // outlier loop (one 16-byte slot per lane)
  __shared__ __align__(16) uint4 s_x[NW * 64];
  // two chunks per wave: the one being packed and the one held for its offset
  __shared__ uint16_t s_val[2][NW][ECAP];  // a wave's outliers, in (row, col) order
  __shared__ uint8_t s_col[2][NW][ECAP];
  __shared__ uint16_t s_roff[2][NW][WR];   // each row's first outlier within the wave's part
  __shared__ uint32_t s_wtot[3][NW];       // each wave's outliers (by chunk number mod 3)
  __shared__ uint32_t s_next, s_base;

  // the wave index through readfirstlane: tile bases are then uniform and
  // stay in scalar registers, addressed with 32-bit lane offsets
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = lane % G, rw = lane / G;
  uint32_t* wtab = s_tab + (STAGE ? wv * WT * TW : 0);
  const int hfix = KFIX ? rw % B.H : 0;
  const uint32_t epoch = __hip_atomic_load(hdr + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t nchunks = B.nchunks;
  // this launch's part and chunk rows (WR, or fewer tiles for a small batch)
  const int wr = B.wr;
  const int64_t cr = (int64_t)NW * wr;

  // Outliers of the tensor's chunks [first, c), by wave 0: lane i of window q
  // examines chunk hi - 1 - i - 64 q, kPackLookWindows windows requested
  // together (predecessors publish their inclusive counts one chunk late,
  // so the nearest is typically a few hundred chunks back).  The nearest
  // inclusive word ends the walk; every word before it must be at least an
  // aggregate, else the walk reads again from there.  A walk that makes no
  // progress for kPackSpinLimit rounds gives up and sets the error word (a
  // bug guard: it never waits forever).
  auto lookback = [&](uint32_t c, uint32_t first) -> uint32_t {
    uint32_t acc = 0, hi = c, spins = 0;
#pragma unroll 1
    for (;;) {
      uint64_t w[kPackLookWindows];
#pragma unroll
      for (int q = 0; q < kPackLookWindows; ++q) {
        const int64_t i = (int64_t)hi - 1 - lane - 64 * q;
        w[q] = st_word(epoch, kStInc, 0u);  // before the tensor's first chunk: nothing
        if (i >= (int64_t)first) w[q] = __hip_atomic_load(status + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      bool stop = false, found = false;
#pragma unroll
      for (int q = 0; q < kPackLookWindows; ++q) {
        if (!stop) {
          const uint32_t fl = (uint32_t)(w[q] >> 32) & 0xffu;
          const bool ok = (uint32_t)(w[q] >> 40) == (epoch & 0xffffffu) && fl != 0u;
          const uint64_t incm = __ballot(ok && (fl & kStInc));
          const uint64_t badm = __ballot(!ok);
          const int fp = incm ? __builtin_ctzll(incm) : 64;
          const uint64_t need = fp >= 63 ? ~0ull : ((2ull << fp) - 1ull);
          if (badm & need) {
            stop = true;  // a predecessor has not published yet: read again from hi
          } else {
            acc += wave_sum(lane <= fp ? (uint32_t)w[q] : 0u);
            if (fp < 64) {
              stop = found = true;
            } else {
              hi -= 64;
              spins = 0;
            }
          }
        }
      }
      if (found) return acc;
      if (stop) {
        if (++spins > kPackSpinLimit) {
          if (lane == 0) __hip_atomic_store(hdr + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          return acc;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
  };

  Search2<NB> S[PT ? 1 : 4];
  uint32_t xmin = 0;  // KFIX: the lane's smallest fast-path bound
  int cur = -1;       // item whose per-channel tables S holds

  if (tid == 0) s_next = __hip_atomic_fetch_add(hdr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  uint32_t c = s_next;
  // the held chunk (packed, offset not yet known): its number; it sits in
  // LDS buffer buf ^ 1 and its wave counts in s_wtot[(par + 2) % 3]
  bool held = false;
  uint32_t hc = 0;
  int buf = 0, par = 0;

  // Resolve the held chunk's offset (wave 0), then every wave writes its part.
  auto flush_held = [&]() {
    const int hbuf = buf ^ 1, hpar = par == 0 ? 2 : par - 1;
    int hj = 0;
    while (hj + 1 < B.n && hc >= B.it[hj + 1].chunk0) ++hj;
    hj = opaque_s(hj);
    const PackItem& ih = B.it[hj];
    const uint32_t hk = hc - ih.chunk0;
    if (wv == 0) {
      uint32_t tot = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) tot += s_wtot[hpar][w];
      uint32_t base = 0;  // outliers of the tensor's earlier chunks
      if (hk != 0) {
        base = lookback(hc, ih.chunk0);
        if (lane == 0) st_publish(status + hc, st_word(epoch, kStInc, base + tot));
      }
      if (lane == 0) s_base = base;
    }
    __syncthreads();
    const int64_t hwbeg = (int64_t)hk * cr + (int64_t)wv * wr;
    const int64_t hrest = ih.nrows - hwbeg;
    const int hnrw = hrest <= 0 ? 0 : (hrest < wr ? (int)hrest : wr);
    const uint32_t hrun = s_wtot[hpar][wv];
    uint32_t base = s_base;
#pragma unroll
    for (int w = 0; w < NW; ++w) base += w < wv ? s_wtot[hpar][w] : 0u;
    const uint16_t* wval = s_val[hbuf][wv];
    const uint8_t* wcol = s_col[hbuf][wv];
    const uint16_t* wroff = s_roff[hbuf][wv];
    const uint32_t kept = hrun < (uint32_t)ECAP ? hrun : (uint32_t)ECAP;
#pragma unroll 1
    for (uint32_t i = lane; i < kept; i += 64) {
      const uint32_t o = base + i;
      if (o < ih.cap) {
        ih.col[o] = wcol[i];
        ih.val[o] = wval[i];
      }
    }
#pragma unroll 1
    for (int i = lane; i < hnrw; i += 64) ih.row_ptr[hwbeg + i] = (int32_t)(base + wroff[i]);
    if (hnrw > 0 && hwbeg + hnrw == ih.nrows && lane == 0) ih.row_ptr[ih.nrows] = (int32_t)(base + hrun);
    if (wv == 0 && hk == 0 && ih.nrows == 0 && lane == 0) ih.row_ptr[0] = 0;  // an empty tensor
    if (hrun > (uint32_t)ECAP) pack_redo_rows<D>(ih, B.H, hwbeg, hnrw, wroff, hrun, base, (uint32_t)ECAP, lane);
    wave_sync();
  };

  while (c < nchunks) {
    int j = 0;
    while (j + 1 < B.n && c >= B.it[j + 1].chunk0) ++j;
    const PackItem& it = B.it[j];
    const hkv_nuq_scales sc = it.sc;
    const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;
    const ItemSlow si{&B, j};
    const int H = B.H;
    const int64_t nrows = it.nrows;
    const uint32_t k = c - it.chunk0;
    const int64_t wbeg = (int64_t)k * cr + (int64_t)wv * wr;  // first row of the wave's part
    const int64_t wrest = nrows - wbeg;
    const int nrw = wrest <= 0 ? 0 : (wrest < wr ? (int)wrest : wr);  // rows of the wave's part
    if constexpr (!PT && KFIX) {
      if (j != cur) {
        const int64_t tab0 = (int64_t)hfix * D + 8 * cg;
#pragma unroll
        for (int q = 0; q < 4; ++q)
          load_search_pair<NB>(tabs + tab0 + 2 * q, tabs + tab0 + 2 * q + 1, S[q]);
        xmin = xsafe_min<NB>(S);
        cur = j;
      }
    }
    uint32_t run = 0;  // the wave's outliers so far
    uint16_t* wval = s_val[buf][wv];
    uint8_t* wcol = s_col[buf][wv];
    uint16_t* wroff = s_roff[buf][wv];
#pragma unroll 1
    for (int tt = 0; tt * WT < wr; ++tt) {
      const int64_t r0 = wbeg + tt * WT;
      const int nv = nrw - tt * WT < WT ? nrw - tt * WT : WT;  // rows of this tile
      if (nv <= 0) break;
      const int64_t t0 = KFIX ? r0 / H : 0;  // token of row r0 (H divides r0)
      const uint16_t* xt = it.x + r0 * D;
      uint8_t* pt = it.packed + r0 * RB;
      uint32_t xs[PASSES][4];
#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        const int rr = p * RW + rw;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (rr < nv) v = load_stream(reinterpret_cast<const uint4*>(xt + (uint32_t)(rr * D + 8 * cg)));
        xs[p][0] = v.x; xs[p][1] = v.y; xs[p][2] = v.z; xs[p][3] = v.w;
      }
      if constexpr (STAGE) {
        // three 16-byte parts of each row's record: breakpoints 0-7, 8-14, and
        // the thresholds (the poles are not needed here)
        for (int i = lane; i < WT * 3; i += 64) {
          const int rr = i / 3, q = i - rr * 3;
          if (rr < nv) {
            int64_t t;
            int h;
            if constexpr (KFIX) {  // H divides r0: the row's token and head from rr
              const int kk = rr / H;
              t = t0 + kk;
              h = rr - kk * H;
            } else {
              const int64_t r = r0 + rr;
              t = r / H;
              h = (int)(r - t * H);
            }
            const int64_t tab = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
            const uint4 v = reinterpret_cast<const uint4*>(tabs + tab)[q == 2 ? 4 : q];
            uint32_t* dw = wtab + rr * TW;
            if (q < 2) {
              const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                const uint32_t hh = (w[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                if (8 * q + e < 15) dw[8 * q + e] = hh | (hh << 16);
              }
            } else {
              const uint32_t lo = v.x & 0xffffu, up = v.x >> 16;
              const uint32_t xsf = ((v.y >> 16) & 1u) ? (v.y & 0xffffu) : 0xffffu;
              dw[15] = lo | (lo << 16);
              dw[16] = up | (up << 16);
              dw[17] = xsf | (xsf << 16);
            }
          }
        }
        wave_sync();
      }

#pragma unroll
      for (int p = 0; p < PASSES; ++p) {
        const int rr = p * RW + rw;
        const int64_t r = r0 + rr;
        uint32_t m = 0;
        if (rr < nv) {
          int64_t t;
          int h;
          if constexpr (KFIX) {
            t = t0 + p * (RW / H) + rw / H;
            h = hfix;
          } else {
            t = r / H;
            h = (int)(r - t * H);
          }
          const uint4 xv = make_uint4(xs[p][0], xs[p][1], xs[p][2], xs[p][3]);
          s_x[wv * 64 + lane] = xv;
          uint32_t pk;
          if constexpr (PT) {
            const RowTabAt tab{sc.rows, sc.positions, sc.pos_offset, h, t};  // for the exact scan only
            if constexpr (STAGE) {
              const uint32_t* tw = wtab + rr * TW;
#pragma unroll
              for (int i = 0; i < (1 << NB) - 1; ++i) S[0].bp[i] = tw[i];
              S[0].lo = tw[15];
              S[0].up = tw[16];
              S[0].xsafe = tw[17];
            } else {
              load_search_bcast<NB>(tabs + tab(0), S[0]);
            }
            quant8_packed<NB, PT, BITS, RowTabAt, false, ItemSlow>(xv, S, si, tab, &pk, &m);
          } else {
            const int64_t tab0 = (int64_t)h * D + 8 * cg;
            if constexpr (!KFIX) {
#pragma unroll
              for (int q = 0; q < 4; ++q)
                load_search_pair<NB>(tabs + tab0 + 2 * q, tabs + tab0 + 2 * q + 1, S[q]);
            }
            if constexpr (KFIX) quant8_packed<NB, PT, BITS, ChanTab, true, ItemSlow>(xv, S, si, ChanTab{tab0}, &pk, &m, xmin);
            else quant8_packed<NB, PT, BITS, ChanTab, false, ItemSlow>(xv, S, si, ChanTab{tab0}, &pk, &m);
          }
          if constexpr (BITS == 4) {
            store_stream(reinterpret_cast<uint32_t*>(pt + (uint32_t)(rr * RB + 4 * cg)), pk);
          } else {
            store_stream(reinterpret_cast<uint16_t*>(pt + (uint32_t)(rr * RB + 2 * cg)), (uint16_t)pk);
          }
        }
        // lanes are in (row, channel) order, so the wave's exclusive count is
        // the position in (row, col) order
        uint32_t tot;
        const uint32_t pos = run + wave_excl_count_fused(__builtin_popcount(m), &tot);
        if (rr < nv && cg == 0) wroff[tt * WT + rr] = (uint16_t)pos;
        run += tot;
        // entries at positions >= ECAP are not kept: the chunk's epilogue
        // finds them again from the input
        const uint16_t* xl = reinterpret_cast<const uint16_t*>(s_x + wv * 64 + lane);
        const uint32_t c8 = 8u * cg;
        uint32_t o = pos;
        while (m) {
          const int e = __builtin_ctz(m);
          m &= m - 1u;
          if (o < (uint32_t)ECAP) {
            wval[o] = xl[e];
            wcol[o] = (uint8_t)(c8 + e);
          }
          ++o;
        }
      }
      if constexpr (STAGE) wave_sync();  // the slice is refilled for the next tile
    }

    // publish the chunk's count and take the next chunk (wave 0), then
    // resolve and write the chunk held from the previous round
    if (lane == 0) s_wtot[par][wv] = run;
    __syncthreads();
    if (wv == 0) {
      uint32_t tot = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) tot += s_wtot[par][w];
      if (lane == 0) {
        st_publish(status + c, st_word(epoch, k == 0 ? kStInc : kStAgg, tot));
        s_next = __hip_atomic_fetch_add(hdr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    if (held) flush_held();  // its barrier also orders s_next
    else __syncthreads();
    held = true;
    hc = c;
    c = s_next;
    buf ^= 1;
    par = par == 2 ? 0 : par + 1;
  }
  if (held) flush_held();

  if (tid == 0) {
    const uint32_t done = __hip_atomic_fetch_add(hdr + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1u) {  // every block has taken its last chunk number
      __hip_atomic_store(hdr + 0, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(hdr + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(hdr + 2, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

struct PackLaunch {
  hipStream_t s;
  uint32_t* hdr;
  uint64_t* status;
};

template <int NB, bool PT, int G, int BITS, bool KFIX>
void launch_fused(const PackBatch& b, const PackLaunch& l) {
  auto k = pack_fused_kernel<NB, PT, G, BITS, KFIX, pack_passes(PT, NB)>;
  hipLaunchKernelGGL(k, dim3(resident_grid(k, (int64_t)b.nchunks)), dim3(kThreads), 0, l.s, b, l.hdr,
                     l.status);
}

template <int NB, bool PT, int BITS, bool KFIX>
void launch_fused_g(int G, const PackBatch& b, const PackLaunch& l) {
  switch (G) {
    case 1: launch_fused<NB, PT, 1, BITS, KFIX>(b, l); break;
    case 2: launch_fused<NB, PT, 2, BITS, KFIX>(b, l); break;
    case 4: launch_fused<NB, PT, 4, BITS, KFIX>(b, l); break;
    case 8: launch_fused<NB, PT, 8, BITS, KFIX>(b, l); break;
    case 16: launch_fused<NB, PT, 16, BITS, KFIX>(b, l); break;
    default: launch_fused<NB, PT, 32, BITS, KFIX>(b, l); break;
  }
}

template <int NB, bool PT, int BITS>
void launch_fused_k(bool kfix, int G, const PackBatch& b, const PackLaunch& l) {
  if (kfix) launch_fused_g<NB, PT, BITS, true>(G, b, l);
  else launch_fused_g<NB, PT, BITS, false>(G, b, l);
}

template <bool PT, int BITS>
void launch_fused_nb(int nb, bool kfix, int G, const PackBatch& b, const PackLaunch& l) {
  switch (nb) {
    case 0: launch_fused_k<0, PT, BITS>(kfix, G, b, l); break;
    case 1: launch_fused_k<1, PT, BITS>(kfix, G, b, l); break;
    case 2: launch_fused_k<2, PT, BITS>(kfix, G, b, l); break;
    case 3: if constexpr (BITS == 4) launch_fused_k<3, PT, BITS>(kfix, G, b, l); break;
    default: if constexpr (BITS == 4) launch_fused_k<4, PT, BITS>(kfix, G, b, l); break;
  }
}

// The kernel variant of one item; items of equal keys share launches.
struct PackKey {
  int nb, pt, bits, G, kfix, H;
  bool operator==(const PackKey& o) const {
    return nb == o.nb && pt == o.pt && bits == o.bits && G == o.G && kfix == o.kfix && H == o.H;
  }
};

int check_pack_item(const hkv_pack_item& a) {
  const hkv_nuq_scales* sc = &a.scales;
  if (!sc->tables || !sc->poles || !sc->upper || !sc->lower) return HKV_ERR_ARG;
  if (a.bits != 2 && a.bits != 4) return HKV_ERR_ARG;
  if (sc->levels < 1 || sc->levels > (1 << a.bits)) return HKV_ERR_ARG;
  if (sc->per_token && sc->rows < 1) return HKV_ERR_SHAPE;
  if (a.T < 0 || a.H < 1 || !pow2_G(a.D)) return HKV_ERR_SHAPE;
  if (a.T * a.H * a.D >= ((int64_t)1 << 31)) return HKV_ERR_SHAPE;  // int32 row_ptr
  if (a.capacity < 0) return HKV_ERR_ARG;
  if (!a.row_ptr) return HKV_ERR_ARG;
  if (a.T > 0) {
    if (!a.values || !a.packed || (a.capacity > 0 && (!a.col || !a.val))) return HKV_ERR_ARG;
    if (((uintptr_t)a.values & 15u) || ((uintptr_t)a.packed & 3u)) return HKV_ERR_ARG;
  }
  return HKV_OK;
}

PackKey pack_key(const hkv_pack_item& a) {
  const int G = a.D / 8;
  return PackKey{nb_for_levels_host(a.scales.levels), a.scales.per_token != 0, a.bits, G,
                 (64 / G) % a.H == 0, a.H};
}

// Chunks of one item at cr rows a chunk (at least one, so an empty tensor
// still gets row_ptr[0]); cr = 0: the variant's full chunk.
int64_t pack_item_chunks(const hkv_pack_item& a, int64_t cr = 0) {
  const PackKey k = pack_key(a);
  if (cr <= 0) cr = pack_chunk_rows(k.G, pack_passes(k.pt, k.nb), k.pt);
  const int64_t n = (a.T * a.H + cr - 1) / cr;
  return n > 0 ? n : 1;
}

// A launch over few full chunks leaves most CUs idle (a 4096-token tensor is
// 32 chunks of 512 rows): its parts are halved, down to one wave tile, while
// the launch has fewer than two chunks per CU and stays within
// kPackSmallChunks chunks.  The workspace holds status words for
// max(full-chunk count, kPackSmallChunks) chunks.
constexpr int64_t kPackSmallChunks = 2048;

// Workspace bound: every chunk of every item (launches reuse the status words).
size_t pack_ws_bytes(int64_t chunks) {
  return kPackHeader + 8 * (size_t)(chunks > kPackSmallChunks ? chunks : kPackSmallChunks);
}

}  // namespace

extern "C" size_t hkv_nuq_pack_compact_workspace_bytes(int64_t T, int H, int D) {
  if (T < 0 || H < 1 || !pow2_G(D)) return 0;
  // every variant's full chunks are at least NW * kPackWaveRows / 2 rows
  const int64_t cr = (int64_t)(kThreads / 64) * (kPackWaveRows / 2);
  const int64_t n = (T * H + cr - 1) / cr;
  return pack_ws_bytes(n > 0 ? n : 1);
}

extern "C" size_t hkv_nuq_pack_compact_batch_workspace_bytes(const hkv_pack_item* items, int n) {
  if (!items || n < 0) return 0;
  int64_t chunks = 0;
  for (int i = 0; i < n; ++i) {
    if (items[i].T < 0 || items[i].H < 1 || !pow2_G(items[i].D)) return 0;
    chunks += pack_item_chunks(items[i]);
  }
  return pack_ws_bytes(chunks > 0 ? chunks : 1);
}

extern "C" int hkv_nuq_pack_compact_batch(const hkv_pack_item* items, int n, void* workspace,
                                          size_t workspace_bytes, void* stream) {
  if (n < 0 || (n > 0 && !items)) return HKV_ERR_ARG;
  if (n == 0) return HKV_OK;
  for (int i = 0; i < n; ++i) {
    const int st = check_pack_item(items[i]);
    if (st != HKV_OK) return st;
  }
  if (!workspace || ((uintptr_t)workspace & 255u) ||
      workspace_bytes < hkv_nuq_pack_compact_batch_workspace_bytes(items, n))
    return HKV_ERR_WORKSPACE;
  PackLaunch l;
  l.s = (hipStream_t)stream;
  l.hdr = (uint32_t*)workspace;
  l.status = (uint64_t*)((char*)workspace + kPackHeader);
  std::vector<char> done((size_t)n, 0);
  for (int i0 = 0; i0 < n; ++i0) {
    if (done[i0]) continue;
    const PackKey key = pack_key(items[i0]);
    const int passes = pack_passes(key.pt, key.nb);
    const int wt = pack_tile_rows(key.G, passes), wfull = pack_wave_rows(key.G, passes, key.pt);
    // the items of this variant, in order, kPackItems per launch; the part
    // rows of a launch follow from its items' full-chunk count
    std::vector<int> mine;
    for (int i = i0; i < n; ++i)
      if (!done[i] && pack_key(items[i]) == key) mine.push_back(i);
    for (size_t m0 = 0; m0 < mine.size(); m0 += kPackItems) {
      const size_t m1 = std::min(mine.size(), m0 + (size_t)kPackItems);
      int wr = wfull;
      auto chunks_at = [&](int w) {
        int64_t c = 0;
        for (size_t m = m0; m < m1; ++m) c += pack_item_chunks(items[mine[m]], (int64_t)(kThreads / 64) * w);
        return c;
      };
      while (wr > wt && chunks_at(wr) < 2 * (int64_t)num_cus() && chunks_at(wr / 2) <= kPackSmallChunks)
        wr /= 2;
      PackBatch b;
      b.n = 0;
      b.H = key.H;
      b.nchunks = 0;
      b.wr = wr;
      for (size_t m = m0; m < m1; ++m) {
        const hkv_pack_item& a = items[mine[m]];
        PackItem& p = b.it[b.n++];
        p.x = (const uint16_t*)a.values;
        p.packed = (uint8_t*)a.packed;
        p.row_ptr = a.row_ptr;
        p.col = a.col;
        p.val = a.val;
        p.sc = a.scales;
        p.nrows = a.T * a.H;
        p.chunk0 = b.nchunks;
        p.cap = (uint32_t)std::min<int64_t>(a.capacity, 0x7fffffff);
        b.nchunks += (uint32_t)pack_item_chunks(a, (int64_t)(kThreads / 64) * wr);
        done[mine[m]] = 1;
      }
      if (key.bits == 4) {
        if (key.pt) launch_fused_nb<true, 4>(key.nb, key.kfix, key.G, b, l);
        else launch_fused_nb<false, 4>(key.nb, key.kfix, key.G, b, l);
      } else {
        if (key.pt) launch_fused_nb<true, 2>(key.nb, key.kfix, key.G, b, l);
        else launch_fused_nb<false, 2>(key.nb, key.kfix, key.G, b, l);
      }
      HKV_CHECK_LAUNCH();
    }
  }
  return HKV_OK;
}

extern "C" int hkv_nuq_pack_compact(const void* values, int64_t T, int H, int D, int bits,
                                    const hkv_nuq_scales* scales, void* packed, int32_t* row_ptr,
                                    uint8_t* col, uint16_t* val, int64_t capacity, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (!scales) return HKV_ERR_ARG;
  hkv_pack_item a;
  a.values = values;
  a.T = T;
  a.H = H;
  a.D = D;
  a.bits = bits;
  a.reserved = 0;
  a.scales = *scales;
  a.packed = packed;
  a.row_ptr = row_ptr;
  a.col = col;
  a.val = val;
  a.capacity = capacity;
  return hkv_nuq_pack_compact_batch(&a, 1, workspace, workspace_bytes, stream);
}
