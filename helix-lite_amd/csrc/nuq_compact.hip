// nuq_compact.hip -- nuq pack into the compact format and its inverse.
//
// Format (this build's; the reference planned but never implemented it:
// src/kvquant/triton_kernels.py:7-18, src/kvquant/compact_pool.py:11-12):
//   packed codes (T,H,D*bits/8) u8, little-endian within a byte
//     nuq4: byte j = c[2j] | c[2j+1] << 4
//     nuq2: byte j = c[4j] | c[4j+1] << 2 | c[4j+2] << 4 | c[4j+3] << 6
//   CSR outliers over rows r = t*H + h: row_ptr (T*H+1) int32, col u8 = d,
//   val fp16 = the original value; (row, col) ascending.
//
// Pack runs as two kernels.  pack_stage_kernel streams the fp16 input once;
// its unit of work is a wave tile (PASSES passes of 64/G rows, G = D/8 lanes
// per row), handled by one wave on its own: no block-level barrier.  A wave
// writes the packed codes, each row's outlier offset within its wave tile
// (into row_ptr), the tile's outliers into the tile's own staging region, and
// the tile's outlier count.  copy_kernel turns the counts into offsets, adds
// them to row_ptr and copies the staged outliers into the dense col/val
// arrays.  No block ever waits on another: on gfx950 the eight XCDs' L2
// caches are not coherent, so a single-pass scan whose tiles wait on their
// predecessors pays a memory round trip per step.
#include "nuq_core.h"

namespace {

constexpr int kThreads = 256;
// Passes of 64/G rows per wave tile: 4 (smaller tiles, fewer registers, more
// waves a SIMD), or 8 for per-channel tables of up to 8 levels, whose search
// state is small enough that the longer tile's loads pay off (131072-token
// layers, us per stage kernel, 8 -> 4 passes: K nuq2 49.2 -> 50.5, V nuq2
// 48.1 -> 42.8, V nuq4 64.8 -> 59.3).
__host__ __device__ constexpr int pack_passes(bool per_token, int nb) { return (!per_token && nb < 4) ? 8 : 4; }

// Workspace: header, per-wave-tile counts, a region of (ntiles + 1) words
// kept so the workspace size stays what earlier versions asked for, then the
// staged entries (u32: value | column << 16), each region 256-byte aligned.  Staging holds a
// whole wave tile per wave tile, so no input can overflow it.
struct PackLayout {
  int64_t ntiles, tile_rows, tile_elems;
  size_t cnt_off, base_off, ent_off, bytes;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

HKV_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// KFIX: the rows of one pass of a wave (RW = 64/G) are a multiple of H, so a
// lane's head is fixed (rw % H) and its token advances by RW / H per pass.
template <int NB, bool PT, int G, int BITS, bool KFIX, int PASSES>
__global__ void __launch_bounds__(kThreads)
pack_stage_kernel(const uint16_t* __restrict__ x, int64_t nrows, int H, hkv_nuq_scales sc,
                  uint8_t* __restrict__ packed, int32_t* __restrict__ row_ptr,
                  uint32_t* __restrict__ sent, uint32_t* __restrict__ wt_cnt, int64_t nwt) {
  constexpr int RW = 64 / G;        // rows per wave per pass
  constexpr int WT = RW * PASSES;  // rows per wave tile
  constexpr int D = 8 * G;
  constexpr int RB = D * BITS / 8;  // packed bytes per row
  constexpr int NW = kThreads / 64;
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

  // the wave index through readfirstlane: tile bases are then uniform and
  // stay in scalar registers, addressed with 32-bit lane offsets
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = lane % G, rw = lane / G;
  uint32_t* wtab = s_tab + (STAGE ? wv * WT * TW : 0);
  const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;
  const SlowInfo si = slow_info(sc);
  const int hfix = KFIX ? rw % H : 0;

  Search2<NB> S[PT ? 1 : 4];
  if constexpr (!PT && KFIX) {
    const int64_t tab0 = (int64_t)hfix * D + 8 * cg;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      load_search_pair<NB>(tabs + tab0 + 2 * j, tabs + tab0 + 2 * j + 1, S[j]);
  }
  uint32_t xmin = 0;  // KFIX: the lane's smallest fast-path bound
  if constexpr (!PT && KFIX) xmin = xsafe_min<NB>(S);

  for (int64_t wt = (int64_t)blockIdx.x * NW + wv; wt < nwt; wt += (int64_t)gridDim.x * NW) {
    const int64_t r0 = wt * WT;
    const int64_t t0 = KFIX ? r0 / H : 0;  // token of row r0 (H divides r0)
    const int nv = nrows - r0 < WT ? (int)(nrows - r0) : WT;  // rows of this tile
    const uint16_t* xt = x + r0 * D;
    uint8_t* pt = packed + r0 * RB;
    int32_t* rpt = row_ptr + r0;
    uint32_t xs[PASSES][4];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int rr = p * RW + rw;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (rr < nv) v = *reinterpret_cast<const uint4*>(xt + (uint32_t)(rr * D + 8 * cg));
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
            const int k = rr / H;
            t = t0 + k;
            h = rr - k * H;
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
            for (int k = 0; k < 8; ++k) {
              const uint32_t hh = (w[k >> 1] >> (16 * (k & 1))) & 0xffffu;
              if (8 * q + k < 15) dw[8 * q + k] = hh | (hh << 16);
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

    uint32_t* st = sent + r0 * D;  // the wave tile's staging region
    uint32_t run = 0;              // outliers of the tile's earlier passes
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
          quant8_packed<NB, PT, BITS>(xv, S, si, tab, &pk, &m);
        } else {
          const int64_t tab0 = (int64_t)h * D + 8 * cg;
          if constexpr (!KFIX) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              load_search_pair<NB>(tabs + tab0 + 2 * j, tabs + tab0 + 2 * j + 1, S[j]);
          }
          if constexpr (KFIX) quant8_packed<NB, PT, BITS, ChanTab, true>(xv, S, si, ChanTab{tab0}, &pk, &m, xmin);
          else quant8_packed<NB, PT, BITS>(xv, S, si, ChanTab{tab0}, &pk, &m);
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
      uint32_t pos = run + wave_excl_count_fused(__builtin_popcount(m), &tot);
      run += tot;
      if (rr < nv && cg == 0)
        *reinterpret_cast<int32_t*>(reinterpret_cast<char*>(rpt) + 4u * (uint32_t)rr) = (int32_t)pos;
      // pos counts the tile's outliers before this one, so pos < WT * D: every
      // entry stays inside the tile's staging region
      const uint16_t* xl = reinterpret_cast<const uint16_t*>(s_x + wv * 64 + lane);
      const uint32_t colb = (uint32_t)(8 * cg) << 16;
      uint32_t off = 4u * pos;
      while (m) {
        const int e = __builtin_ctz(m);
        m &= m - 1u;
        *reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(st) + off) =
            (uint32_t)xl[e] | (colb + ((uint32_t)e << 16));
        off += 4u;
      }
    }
    if (lane == 0) wt_cnt[wt] = run;
    if constexpr (STAGE) wave_sync();  // the slice is refilled for the next tile
  }
}

// The dense CSR, in one kernel after the stage kernel.  Block b owns the
// wave tiles [b * tpb, (b + 1) * tpb) (tpb: a power of two from 32 to 256,
// the smallest that keeps the grid within kCopyBlocks blocks, or 256).  Its
// base is the sum of the counts of all earlier tiles, which it reads itself
// (at most nwt counts, from L2: no separate scan kernel and no inter-block
// waiting); its tiles' offsets are a block scan of their counts, one tile per
// thread.  Each wave then copies a run of the block's tiles, requesting the
// staged entries of several tiles (and the block's row_ptr entries) before
// storing any, so a block waits on few memory round trips.  The last block
// writes row_ptr[nrows] = nnz.
constexpr int kCopyBlocks = 256;
constexpr int kCopyThreads = 1024;
constexpr int kCopyMaxTPB = 256;
constexpr int kCopyU = 4;   // loads in flight per thread: prefix counts, row_ptr
constexpr int kCopyTW = 4;  // tiles per wave and batch of staged-entry loads
constexpr int kCopyUT = 4;  // staged-entry loads per lane and tile in a batch

HKV_DEV uint32_t wave_sum(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += (uint32_t)__shfl_xor((int)v, o, 64);
  return v;
}

__global__ void __launch_bounds__(kCopyThreads)
copy_kernel(const uint32_t* __restrict__ cnt, int64_t nwt, int tpb, int64_t WT, int64_t D,
            int64_t nrows, const uint32_t* __restrict__ sent, int32_t* __restrict__ row_ptr,
            uint8_t* __restrict__ col, uint16_t* __restrict__ val, uint32_t cap) {
  constexpr int NW = kCopyThreads / 64;
  __shared__ uint32_t s_off[kCopyMaxTPB + 1];
  __shared__ uint32_t s_pre[NW], s_run[NW];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t t0 = (int64_t)blockIdx.x * tpb;
  const int nt = (int)min<int64_t>(tpb, nwt - t0);
  const uint32_t region = (uint32_t)(WT * D);  // staging capacity of a tile
  // this block's tiles, one per thread, and the counts of all earlier tiles
  // (t0 is a multiple of 4: whole 16-byte groups), all requested together
  const uint32_t own = tid < nt ? min(cnt[t0 + tid], region) : 0u;
  uint32_t pre = 0;
  const uint4* c4 = reinterpret_cast<const uint4*>(cnt);
  for (int64_t i0 = tid; i0 < t0 / 4; i0 += (int64_t)kCopyThreads * kCopyU) {
    uint4 v[kCopyU];
#pragma unroll
    for (int u = 0; u < kCopyU; ++u) {
      const int64_t i = i0 + (int64_t)u * kCopyThreads;
      v[u] = i < t0 / 4 ? c4[i] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < kCopyU; ++u) pre += v[u].x + v[u].y + v[u].z + v[u].w;
  }
  pre = wave_sum(pre);
  const uint32_t inc = wave_incl_sum_fused(own);
  if (lane == 63) s_run[wv] = inc;
  if (lane == 0) s_pre[wv] = pre;
  __syncthreads();
  uint32_t base = 0, before = inc - own;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    base += s_pre[w];
    before += w < wv ? s_run[w] : 0u;
  }
  if (tid < tpb) s_off[tid] = before;
  if (tid == kCopyThreads - 1) s_off[tpb] = before + own;  // the block's total (tiles < tpb <= 256)
  __syncthreads();
  const uint32_t total = s_off[tpb];
  const int64_t r0 = t0 * WT;
  const uint32_t nr = (uint32_t)min<int64_t>(nrows - r0, (int64_t)nt * WT);
  const uint32_t wt32 = (uint32_t)WT;
  const uint32_t* src = sent + r0 * D;
  auto put = [&](uint32_t o, uint32_t e) {
    if (o < cap) {
      col[o] = (uint8_t)(e >> 16);
      val[o] = (uint16_t)e;
    }
  };
  // row_ptr: the first kCopyU rows per thread are requested together with
  // the first batch of entries; larger blocks loop over the rest
  int32_t rv[kCopyU];
#pragma unroll
  for (int u = 0; u < kCopyU; ++u) {
    const uint32_t i = tid + u * kCopyThreads;
    rv[u] = i < nr ? row_ptr[r0 + i] : 0;
  }
  // entries: wave wv copies tiles [wv * tpw, (wv + 1) * tpw), kCopyTW tiles
  // per batch, kCopyUT entries per lane and tile requested before any store
  // (a tile with more entries finishes in a loop after the batch)
  const int tpw = tpb / NW;  // 2 to 16
  for (int m0 = 0; m0 < tpw; m0 += kCopyTW) {
    uint32_t e[kCopyTW][kCopyUT];
#pragma unroll
    for (int m = 0; m < kCopyTW; ++m) {
      const int j = wv * tpw + m0 + m;
      const uint32_t n = (m0 + m < tpw && j < nt) ? s_off[j + 1] - s_off[j] : 0u;
#pragma unroll
      for (int u = 0; u < kCopyUT; ++u) {
        const uint32_t i = lane + 64u * u;
        e[m][u] = i < n ? src[(int64_t)j * region + i] : 0u;
      }
    }
    if (m0 == 0) {
#pragma unroll
      for (int u = 0; u < kCopyU; ++u) {
        const uint32_t i = tid + u * kCopyThreads;
        if (i < nr) row_ptr[r0 + i] = rv[u] + (int32_t)(base + s_off[i / wt32]);
      }
    }
#pragma unroll
    for (int m = 0; m < kCopyTW; ++m) {
      const int j = wv * tpw + m0 + m;
      const bool own_tile = m0 + m < tpw && j < nt;
      const uint32_t n = own_tile ? s_off[j + 1] - s_off[j] : 0u;
      const uint32_t o0 = base + (own_tile ? s_off[j] : 0u);
#pragma unroll
      for (int u = 0; u < kCopyUT; ++u) {
        const uint32_t i = lane + 64u * u;
        if (i < n) put(o0 + i, e[m][u]);
      }
      for (uint32_t i = lane + 64u * kCopyUT; i < n; i += 64u) put(o0 + i, src[(int64_t)j * region + i]);
    }
  }
  for (uint32_t i0 = tid + kCopyU * kCopyThreads; i0 < nr; i0 += kCopyThreads * kCopyU) {
#pragma unroll
    for (int u = 0; u < kCopyU; ++u) {
      const uint32_t i = i0 + u * kCopyThreads;
      rv[u] = i < nr ? row_ptr[r0 + i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kCopyU; ++u) {
      const uint32_t i = i0 + u * kCopyThreads;
      if (i < nr) row_ptr[r0 + i] = rv[u] + (int32_t)(base + s_off[i / wt32]);
    }
  }
  if (t0 + nt == nwt && tid == 0) row_ptr[nrows] = (int32_t)(base + total);
}

// Compact unpack.  Each wave owns a private LDS segment of kUPasses * RW
// rows (RW = 64 / G rows per pass): it dequantises its rows into the
// segment, scatters the rows' CSR entries into it, and writes the rows out
// with 128-bit stores.  Only wave-level ordering is needed between those
// steps (LDS operations of one wave complete in order), so waves proceed
// independently.  Blocks are persistent and loop over wave tiles.  Per-channel
// poles of all heads are staged once per block in LDS as [h][level][d] fp16
// when they fit (KLDS); per-token poles are staged per row.  CSR entries at or
// beyond `cap` (the col/val capacity) are never read.
constexpr int kUPasses = 4;

template <bool PT, int G, int BITS, bool KLDS>
__global__ void __launch_bounds__(kThreads)
unpack_compact_kernel(const uint8_t* __restrict__ packed, const int32_t* __restrict__ row_ptr,
                      const uint8_t* __restrict__ col, const uint16_t* __restrict__ val,
                      int64_t cap, int64_t nrows, int H, hkv_nuq_scales sc,
                      uint16_t* __restrict__ out, int64_t nwtiles) {
  constexpr int D = 8 * G;
  constexpr int RW = 64 / G;           // rows per wave per pass
  constexpr int WR = RW * kUPasses;    // rows per wave tile
  constexpr int RB = D * BITS / 8;     // packed bytes per row
  constexpr int NW = kThreads / 64;
  extern __shared__ uint16_t dyn[];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int cg = lane % G, rw = lane / G;
  uint16_t* seg = dyn + wv * (WR * D);
  uint16_t* prow = dyn + NW * WR * D + wv * (WR * 16);  // PT: poles of each row
  uint16_t* kp = dyn + NW * WR * D;                     // KLDS: [h][16][D]
  const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;

  if constexpr (!PT && KLDS) {
    for (int i = tid; i < H * D; i += kThreads) {
      const uint4* src = reinterpret_cast<const uint4*>(tabs[i].pf16);
      const uint4 a = src[0], b = src[1];
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      const int h = i / D, d = i - h * D;
#pragma unroll
      for (int l = 0; l < 16; ++l) kp[(h * 16 + l) * D + d] = (uint16_t)(w[l >> 1] >> (16 * (l & 1)));
    }
    __syncthreads();
  }

  // Three-stage pipeline over the wave's tiles: codes, row_ptr and (PT) pole
  // rows are loaded two tiles ahead, each row's first CSR entries one tile
  // ahead, so no global load is waited on right after it is issued.  Loads
  // are unconditional from clamped in-bounds rows (row nrows - 1 for rows past
  // the end, whose results are not stored).
  struct TileLoad {
    uint32_t cw[kUPasses];
    int2 rp[kUPasses];
    uint32_t pv[kUPasses];  // PT: pole cg of the row's 16 (G >= 16), or poles cg, cg+G, ...
  };
  struct TileCsr {
    uint32_t c[kUPasses], v[kUPasses];  // entry ra + cg of each pass's row
  };
  const int64_t nwaves = (int64_t)gridDim.x * NW;
  auto load_tile = [&](int64_t wt, TileLoad& L) {
#pragma unroll
    for (int p = 0; p < kUPasses; ++p) {
      int64_t r = wt * WR + p * RW + rw;
      r = r < nrows ? r : nrows - 1;
      if constexpr (BITS == 4) L.cw[p] = *reinterpret_cast<const uint32_t*>(packed + r * RB + 4 * cg);
      else L.cw[p] = *reinterpret_cast<const uint16_t*>(packed + r * RB + 2 * cg);
      L.rp[p] = *reinterpret_cast<const int2*>(row_ptr + r);
      if constexpr (PT) {
        const int ri = (int)r;  // rows < 2^31
        const int t = ri / H;
        const int h = ri - t * H;
        const int64_t tab = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
        L.pv[p] = tabs[tab].pf16[cg & 15];
      }
    }
  };
  auto load_csr = [&](const TileLoad& L, TileCsr& C) {
    if (cap <= 0) return;
#pragma unroll
    for (int p = 0; p < kUPasses; ++p) {
      int64_t i = (int64_t)(L.rp[p].x > 0 ? L.rp[p].x : 0) + cg;
      i = i < cap ? i : cap - 1;
      C.c[p] = col[i];
      C.v[p] = val[i];
    }
  };
  auto process = [&](int64_t wt, const TileLoad& L, const TileCsr& C) {
    const int64_t r0 = wt * WR;
    if constexpr (PT) {
#pragma unroll
      for (int p = 0; p < kUPasses; ++p)
        if (cg < 16) prow[(p * RW + rw) * 16 + cg] = (uint16_t)L.pv[p];
      if constexpr (G < 16) {  // fewer lanes than poles per row: the rest directly
#pragma unroll
        for (int p = 0; p < kUPasses; ++p) {
          int64_t r = r0 + p * RW + rw;
          r = r < nrows ? r : nrows - 1;
          const int ri = (int)r;
          const int t = ri / H;
          const int h = ri - t * H;
          const int64_t tab = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
          for (int l = cg + G; l < 16; l += G) prow[(p * RW + rw) * 16 + l] = tabs[tab].pf16[l];
        }
      }
      wave_sync();
    }
#pragma unroll
    for (int p = 0; p < kUPasses; ++p) {
      const int rr = p * RW + rw;
      const int64_t r = r0 + rr;
      const int h = (int)(r % H);
      uint32_t res[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t pr = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int e = 2 * j + k;
          const uint32_t c = (L.cw[p] >> (BITS * e)) & ((1u << BITS) - 1u);
          uint16_t v;
          if constexpr (PT) v = prow[rr * 16 + c];
          else if constexpr (KLDS) v = kp[(h * 16 + c) * D + 8 * cg + e];
          else v = tabs[(int64_t)h * D + 8 * cg + e].pf16[c];
          pr |= (uint32_t)v << (16 * k);
        }
        res[j] = pr;
      }
      *reinterpret_cast<uint4*>(seg + rr * D + 8 * cg) = make_uint4(res[0], res[1], res[2], res[3]);
    }
    wave_sync();
#pragma unroll
    for (int p = 0; p < kUPasses; ++p) {
      const int rr = p * RW + rw;
      const int32_t lo = L.rp[p].x > 0 ? L.rp[p].x : 0;
      const int32_t hi = (int64_t)L.rp[p].y < cap ? L.rp[p].y : (int32_t)cap;
      if (lo + cg < hi && C.c[p] < (uint32_t)D) seg[rr * D + C.c[p]] = (uint16_t)C.v[p];
      for (int32_t i = lo + cg + G; i < hi; i += G) {  // rows with more than G outliers
        const uint32_t d = col[i];
        if (d < (uint32_t)D) seg[rr * D + d] = val[i];
      }
    }
    wave_sync();
#pragma unroll
    for (int p = 0; p < kUPasses; ++p) {
      const int rr = p * RW + rw;
      const int64_t r = r0 + rr;
      if (r >= nrows) continue;
      store_stream(out + r * D + 8 * cg, *reinterpret_cast<const uint4*>(seg + rr * D + 8 * cg));
    }
    wave_sync();
  };
  const int64_t wt0 = (int64_t)blockIdx.x * NW + wv;
  if (wt0 >= nwtiles) return;
  TileLoad L0, L1, L2;
  TileCsr C0, C1, C2;
  load_tile(wt0, L0);
  load_tile(wt0 + nwaves, L1);
  load_csr(L0, C0);
  auto step = [&](int64_t wt, const TileLoad& Lc, const TileCsr& Cc, const TileLoad& Ln, TileCsr& Cn,
                  TileLoad& Lw) {
    load_tile(wt + 2 * nwaves, Lw);
    load_csr(Ln, Cn);
    process(wt, Lc, Cc);
  };
  for (int64_t wt = wt0; wt < nwtiles; wt += 3 * nwaves) {
    step(wt, L0, C0, L1, C1, L2);
    if (wt + nwaves >= nwtiles) break;
    step(wt + nwaves, L1, C1, L2, C2, L0);
    if (wt + 2 * nwaves >= nwtiles) break;
    step(wt + 2 * nwaves, L2, C2, L0, C0, L1);
  }
}

// Unpack for D = 128 (16 lanes per row) when H is a power of two dividing the
// rows of a wave tile, with the same three-stage load pipeline as
// unpack_compact_kernel.  A lane's head and token follow from its row by a
// mask and a shift, the tile's rows are addressed from a uniform base row
// (clamped at the end), codes are bit fields of one word, and the K poles sit
// in LDS as [h][level][d] with padded rows (kU128SC, u128_head halfwords) so
// that the heads of a pass and the two halves of a row use different banks.
constexpr int kU128Passes = 2;             // passes of 4 rows per wave tile
constexpr int kU128SC = 130;  // halfwords per (head, level) row of the K poles
// halfwords per head of the K poles (levels rows of kU128SC, skewed by 2)
__host__ __device__ constexpr int u128_head(int levels) { return levels * kU128SC + 2; }

template <bool PT, int BITS>
__global__ void __launch_bounds__(kThreads)
unpack_d128_kernel(const uint8_t* __restrict__ packed, const int32_t* __restrict__ row_ptr,
                   const uint8_t* __restrict__ col, const uint16_t* __restrict__ val, int64_t cap,
                   int64_t nrows, int lgH, hkv_nuq_scales sc, uint16_t* __restrict__ out,
                   int64_t nwtiles) {
  constexpr int D = 128, RW = 4, WR = RW * kU128Passes, RB = D * BITS / 8, NW = kThreads / 64;
  constexpr int NL = 1 << BITS, SH = u128_head(NL);  // pole levels per channel, halfwords per head
  const int H = 1 << lgH;
  extern __shared__ uint16_t dyn[];
  // the wave index through readfirstlane: tile bases are then known to be
  // uniform and stay in scalar registers (loads take a 32-bit lane offset)
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = lane & 15, rw = lane >> 4;
  uint16_t* seg = dyn + wv * (WR * D);
  uint16_t* prow = dyn + NW * WR * D + wv * (WR * 16);  // PT: poles of each row
  uint16_t* kp = dyn + NW * WR * D;                     // K: poles [h][level][d], padded
  const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;
  if constexpr (!PT) {
    for (int i = tid; i < H * D; i += kThreads) {
      const uint4* src = reinterpret_cast<const uint4*>(tabs[i].pf16);
      const uint4 a = src[0], b = src[1];
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      const int h = i >> 7, d = i & (D - 1);
#pragma unroll
      for (int l = 0; l < NL; ++l) kp[h * SH + l * kU128SC + d] = (uint16_t)(w[l >> 1] >> (16 * (l & 1)));
    }
    __syncthreads();
  }
  // The tile's base row (clamped to the last row past the end) and the last
  // valid row offset within it.
  auto tile_base = [&](int64_t wt, int64_t& rbase, int& lim) {
    const int64_t r0 = wt * WR;
    rbase = r0 < nrows ? r0 : nrows - 1;
    const int64_t rest = nrows - 1 - rbase;
    lim = rest < WR - 1 ? (int)rest : WR - 1;
  };
  struct TileLoad {
    uint32_t cw[kU128Passes];
    int2 rp[kU128Passes];
    uint32_t pv[kU128Passes];  // PT: pole cg of the row
  };
  struct TileCsr {
    uint32_t c[kU128Passes], v[kU128Passes];  // entry ra + cg of each pass's row
  };
  const int64_t nwaves = (int64_t)gridDim.x * NW;
  const uint32_t cap32 = (uint32_t)(cap < 0x7fffffff ? cap : 0x7fffffff);  // row_ptr entries are int32
  const int rows32 = (int)sc.rows;  // the host checks H * rows * 80 < 2^31 for this kernel
  auto load_tile = [&](int64_t wt, TileLoad& L) {
    int64_t rbase;
    int lim;
    tile_base(wt, rbase, lim);
    const uint8_t* pk = packed + rbase * RB;
    const int32_t* rp = row_ptr + rbase;
    // PT: token of row o is t0 + (o >> lgH) and its head o & (H - 1) (rbase
    // is a multiple of H for a tile in range; past the end, o = 0 and the
    // loads stay at the last row)
    const int64_t t0 = rbase >> lgH;
    const int64_t p0 = sc.pos_offset + t0;  // position of token t0 without a position array
    const int p0c = p0 < -(int64_t)WR ? -WR : (p0 > (int64_t)rows32 ? rows32 : (int)p0);
#pragma unroll
    for (int p = 0; p < kU128Passes; ++p) {
      // unsigned 32-bit lane offsets from the uniform bases (scalar-base addressing)
      const uint32_t o = (uint32_t)(p * RW + rw < lim ? p * RW + rw : lim);
      if constexpr (BITS == 4) L.cw[p] = *reinterpret_cast<const uint32_t*>(pk + (o * RB + 4u * cg));
      else L.cw[p] = *reinterpret_cast<const uint16_t*>(pk + (o * RB + 2u * cg));
      L.rp[p] = *reinterpret_cast<const int2*>(reinterpret_cast<const char*>(rp) + 4u * o);
      if constexpr (PT) {
        const int k = (int)(o >> lgH), h = (int)(o & (H - 1));
        int pos;
        if (sc.positions) {
          const int64_t ap = sc.positions[t0 + k];
          pos = ap < 0 ? 0 : (ap > rows32 - 1 ? rows32 - 1 : (int)ap);
        } else {
          pos = p0c + k;
          pos = pos < 0 ? 0 : (pos > rows32 - 1 ? rows32 - 1 : pos);
        }
        const uint32_t off = (uint32_t)(h * rows32 + pos) * (uint32_t)sizeof(hkv_table_t) + 32u + 2u * cg;
        L.pv[p] = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(tabs) + off);
      }
    }
  };
  auto load_csr = [&](const TileLoad& L, TileCsr& C) {
    if (cap <= 0) return;
#pragma unroll
    for (int p = 0; p < kU128Passes; ++p) {
      uint32_t i = (uint32_t)(L.rp[p].x > 0 ? L.rp[p].x : 0) + (uint32_t)cg;
      i = i < cap32 ? i : cap32 - 1u;
      C.c[p] = col[i];
      C.v[p] = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const char*>(val) + 2u * i);
    }
  };
  auto process = [&](int64_t wt, const TileLoad& L, const TileCsr& C) {
    int64_t rbase;
    int lim;
    tile_base(wt, rbase, lim);  // rbase = wt * WR: the tile is in range
    if constexpr (PT) {
#pragma unroll
      for (int p = 0; p < kU128Passes; ++p) prow[(p * RW + rw) * 16 + cg] = (uint16_t)L.pv[p];
      wave_sync();
    }
#pragma unroll
    for (int p = 0; p < kU128Passes; ++p) {
      const int rr = p * RW + rw;
      const uint16_t* lb;
      if constexpr (PT) {
        lb = prow + rr * 16;
      } else {
        lb = kp + (rr & (H - 1)) * SH + 8 * cg;  // rbase is a multiple of H
      }
      uint32_t res[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t pr = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int e = 2 * j + k;
          const uint32_t c = (L.cw[p] >> (BITS * e)) & ((1u << BITS) - 1u);
          const uint16_t v = PT ? lb[c] : lb[c * kU128SC + e];
          pr |= (uint32_t)v << (16 * k);
        }
        res[j] = pr;
      }
      *reinterpret_cast<uint4*>(seg + rr * D + 8 * cg) = make_uint4(res[0], res[1], res[2], res[3]);
    }
    wave_sync();
#pragma unroll
    for (int p = 0; p < kU128Passes; ++p) {
      const int rr = p * RW + rw;
      const int32_t lo = L.rp[p].x > 0 ? L.rp[p].x : 0;
      const int32_t hi = (int64_t)L.rp[p].y < cap ? L.rp[p].y : (int32_t)cap;
      if (lo + cg < hi && C.c[p] < (uint32_t)D) seg[rr * D + C.c[p]] = (uint16_t)C.v[p];
      for (int32_t i = lo + cg + 16; i < hi; i += 16) {  // rows with more than 16 outliers
        const uint32_t d = col[i];
        if (d < (uint32_t)D) seg[rr * D + d] = val[i];
      }
    }
    wave_sync();
    uint16_t* ob = out + rbase * D;
#pragma unroll
    for (int p = 0; p < kU128Passes; ++p) {
      const int rr = p * RW + rw;
      if (rr > lim) continue;
      store_stream(ob + (uint32_t)(rr * D + 8 * cg), *reinterpret_cast<const uint4*>(seg + rr * D + 8 * cg));
    }
    wave_sync();
  };
  const int64_t wt0 = (int64_t)blockIdx.x * NW + wv;
  if (wt0 >= nwtiles) return;
  TileLoad L0, L1, L2;
  TileCsr C0, C1, C2;
  load_tile(wt0, L0);
  load_tile(wt0 + nwaves, L1);
  load_csr(L0, C0);
  auto step = [&](int64_t wt, const TileLoad& Lc, const TileCsr& Cc, const TileLoad& Ln, TileCsr& Cn,
                  TileLoad& Lw) {
    load_tile(wt + 2 * nwaves, Lw);
    load_csr(Ln, Cn);
    process(wt, Lc, Cc);
  };
  for (int64_t wt = wt0; wt < nwtiles; wt += 3 * nwaves) {
    step(wt, L0, C0, L1, C1, L2);
    if (wt + nwaves >= nwtiles) break;
    step(wt + nwaves, L1, C1, L2, C2, L0);
    if (wt + 2 * nwaves >= nwtiles) break;
    step(wt + 2 * nwaves, L2, C2, L0, C0, L1);
  }
}

__global__ void write_zero_rowptr(int32_t* row_ptr) { row_ptr[0] = 0; }

bool pow2_G(int D) { return D % 8 == 0 && D >= 8 && D <= 256 && ((D / 8) & (D / 8 - 1)) == 0; }

PackLayout pack_layout(int64_t nrows, int D, int passes) {
  PackLayout L;
  L.tile_rows = (int64_t)(64 / (D / 8)) * passes;
  L.ntiles = (nrows + L.tile_rows - 1) / L.tile_rows;
  L.tile_elems = L.tile_rows * D;
  L.cnt_off = 256;
  L.base_off = L.cnt_off + align256(sizeof(uint32_t) * (size_t)L.ntiles);
  L.ent_off = L.base_off + align256(sizeof(uint32_t) * (size_t)(L.ntiles + 1));
  L.bytes = L.ent_off + sizeof(uint32_t) * (size_t)(L.ntiles * L.tile_elems);
  return L;
}

int num_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

// Persistent grid: as many blocks as fit on the device at once (at most one
// per tile).
template <typename K>
unsigned resident_grid(K kernel, int64_t nblocks, size_t lds = 0) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, lds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  return (unsigned)std::min<int64_t>(nblocks, (int64_t)per_cu * num_cus());
}

struct PackArgs {
  const uint16_t* x;
  int64_t nrows;
  int H;
  hkv_nuq_scales sc;
  uint8_t* pk;
  int32_t* rp;
  uint32_t* sent;
  uint32_t* cnt;
  int64_t ntiles;  // wave tiles
  hipStream_t s;
};

template <int NB, bool PT, int G, int BITS, bool KFIX>
void launch_stage(const PackArgs& a) {
  auto k = pack_stage_kernel<NB, PT, G, BITS, KFIX, pack_passes(PT, NB)>;
  const int64_t nblocks = (a.ntiles + kThreads / 64 - 1) / (kThreads / 64);
  hipLaunchKernelGGL(k, dim3(resident_grid(k, nblocks)), dim3(kThreads), 0, a.s, a.x, a.nrows,
                     a.H, a.sc, a.pk, a.rp, a.sent, a.cnt, a.ntiles);
}

template <int NB, bool PT, int BITS, bool KFIX>
void launch_stage_g(int G, const PackArgs& a) {
  switch (G) {
    case 1: launch_stage<NB, PT, 1, BITS, KFIX>(a); break;
    case 2: launch_stage<NB, PT, 2, BITS, KFIX>(a); break;
    case 4: launch_stage<NB, PT, 4, BITS, KFIX>(a); break;
    case 8: launch_stage<NB, PT, 8, BITS, KFIX>(a); break;
    case 16: launch_stage<NB, PT, 16, BITS, KFIX>(a); break;
    default: launch_stage<NB, PT, 32, BITS, KFIX>(a); break;
  }
}

template <int NB, bool PT, int BITS>
void launch_stage_k(bool kfix, int G, const PackArgs& a) {
  if (kfix) launch_stage_g<NB, PT, BITS, true>(G, a);
  else launch_stage_g<NB, PT, BITS, false>(G, a);
}

template <bool PT, int BITS>
void launch_stage_nb(int nb, bool kfix, int G, const PackArgs& a) {
  switch (nb) {
    case 0: launch_stage_k<0, PT, BITS>(kfix, G, a); break;
    case 1: launch_stage_k<1, PT, BITS>(kfix, G, a); break;
    case 2: launch_stage_k<2, PT, BITS>(kfix, G, a); break;
    case 3: if constexpr (BITS == 4) launch_stage_k<3, PT, BITS>(kfix, G, a); break;
    default: if constexpr (BITS == 4) launch_stage_k<4, PT, BITS>(kfix, G, a); break;
  }
}

template <bool PT, int BITS, bool KLDS>
void launch_unpack_g(int G, unsigned grid, size_t lds, hipStream_t s, const uint8_t* pk,
                     const int32_t* rp, const uint8_t* col, const uint16_t* val, int64_t cap,
                     int64_t nrows, int H, const hkv_nuq_scales& sc, uint16_t* out,
                     int64_t nwtiles) {
  switch (G) {
#define HKV_CASE(g)                                                                            \
  case g:                                                                                      \
    hipLaunchKernelGGL((unpack_compact_kernel<PT, g, BITS, KLDS>), dim3(grid), dim3(kThreads), \
                       lds, s, pk, rp, col, val, cap, nrows, H, sc, out, nwtiles);             \
    break;
    HKV_CASE(1) HKV_CASE(2) HKV_CASE(4) HKV_CASE(8) HKV_CASE(16) HKV_CASE(32)
#undef HKV_CASE
  }
}

}  // namespace

extern "C" size_t hkv_nuq_pack_compact_workspace_bytes(int64_t T, int H, int D) {
  if (T < 0 || H < 1 || !pow2_G(D)) return 0;
  // the larger of the two tilings (more tiles: more counts)
  return std::max(pack_layout(T * H, D, 4).bytes, pack_layout(T * H, D, 8).bytes);
}

extern "C" int hkv_nuq_pack_compact(const void* values, int64_t T, int H, int D, int bits,
                                    const hkv_nuq_scales* scales, void* packed, int32_t* row_ptr,
                                    uint8_t* col, uint16_t* val, int64_t capacity, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  if (!scales || !scales->tables || !scales->poles || !scales->upper || !scales->lower)
    return HKV_ERR_ARG;
  if (bits != 2 && bits != 4) return HKV_ERR_ARG;
  if (scales->levels < 1 || scales->levels > (1 << bits)) return HKV_ERR_ARG;
  if (scales->per_token && scales->rows < 1) return HKV_ERR_SHAPE;
  if (T < 0 || H < 1 || !pow2_G(D)) return HKV_ERR_SHAPE;
  if (T * H * D >= ((int64_t)1 << 31)) return HKV_ERR_SHAPE;  // int32 row_ptr
  if (capacity < 0) return HKV_ERR_ARG;
  if (!row_ptr) return HKV_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nrows = T * H;
  if (nrows == 0) {
    hipLaunchKernelGGL(write_zero_rowptr, dim3(1), dim3(1), 0, s, row_ptr);
    HKV_CHECK_LAUNCH();
    return HKV_OK;
  }
  if (!values || !packed || (capacity > 0 && (!col || !val))) return HKV_ERR_ARG;
  if (((uintptr_t)values & 15u) || ((uintptr_t)packed & 3u)) return HKV_ERR_ARG;
  const PackLayout lay = pack_layout(nrows, D, pack_passes(scales->per_token != 0, nb_for_levels_host(scales->levels)));
  if (!workspace || workspace_bytes < lay.bytes || ((uintptr_t)workspace & 255u))
    return HKV_ERR_WORKSPACE;
  const int G = D / 8, RW = 64 / G;
  char* ws = (char*)workspace;
  PackArgs a;
  a.x = (const uint16_t*)values;
  a.nrows = nrows;
  a.H = H;
  a.sc = *scales;
  a.pk = (uint8_t*)packed;
  a.rp = row_ptr;
  a.sent = (uint32_t*)(ws + lay.ent_off);
  a.cnt = (uint32_t*)(ws + lay.cnt_off);
  a.ntiles = lay.ntiles;
  a.s = s;
  const bool kfix = (RW % H) == 0;
  const int nb = nb_for_levels_host(a.sc.levels);
  if (bits == 4) {
    if (a.sc.per_token) launch_stage_nb<true, 4>(nb, kfix, G, a);
    else launch_stage_nb<false, 4>(nb, kfix, G, a);
  } else {
    if (a.sc.per_token) launch_stage_nb<true, 2>(nb, kfix, G, a);
    else launch_stage_nb<false, 2>(nb, kfix, G, a);
  }
  HKV_CHECK_LAUNCH();
  const uint32_t cap = (uint32_t)std::min<int64_t>(capacity, 0x7fffffff);
  int tpb = 32;
  while (tpb < kCopyMaxTPB && (a.ntiles + tpb - 1) / tpb > kCopyBlocks) tpb *= 2;
  const unsigned cgrid = (unsigned)((a.ntiles + tpb - 1) / tpb);
  hipLaunchKernelGGL(copy_kernel, dim3(cgrid), dim3(kCopyThreads), 0, s, a.cnt, a.ntiles, tpb,
                     lay.tile_rows, (int64_t)D, nrows, a.sent, row_ptr, col, val, cap);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" int hkv_nuq_unpack_compact(const void* packed, const int32_t* row_ptr,
                                      const uint8_t* col, const uint16_t* val, int64_t capacity,
                                      int64_t T, int H, int D, int bits,
                                      const hkv_nuq_scales* scales, void* out, void* stream) {
  if (!scales || !scales->tables) return HKV_ERR_ARG;
  if (bits != 2 && bits != 4) return HKV_ERR_ARG;
  if (scales->per_token && scales->rows < 1) return HKV_ERR_SHAPE;
  if (T < 0 || H < 1 || !pow2_G(D)) return HKV_ERR_SHAPE;
  if (capacity < 0) return HKV_ERR_ARG;
  if (T == 0) return HKV_OK;
  if (!packed || !row_ptr || !out || (capacity > 0 && (!col || !val))) return HKV_ERR_ARG;
  if (((uintptr_t)out & 15u) || ((uintptr_t)packed & 3u)) return HKV_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nrows = T * H;
  const int G = D / 8;
  constexpr int NW = kThreads / 64;
  const int64_t WR = (int64_t)(64 / G) * kUPasses;  // rows per wave tile
  const int64_t nwtiles = (nrows + WR - 1) / WR;
  const unsigned grid =
      (unsigned)std::min<int64_t>((nwtiles + NW - 1) / NW, (int64_t)num_cus() * 8);
  const hkv_nuq_scales sc = *scales;
  const size_t seg_bytes = (size_t)NW * WR * D * 2;
  const size_t kpole_bytes = (size_t)H * 16 * D * 2;
  auto pk = (const uint8_t*)packed;
  auto o = (uint16_t*)out;
  const int lgH = __builtin_ctz((unsigned)H);
  // H a power of two dividing the rows of a wave tile (4 * kU128Passes)
  const bool h_pow2 = (H & (H - 1)) == 0 && (4 * kU128Passes) % H == 0;
  if (D == 128 && h_pow2 &&
      (!sc.per_token || (int64_t)H * sc.rows * (int64_t)sizeof(hkv_table_t) < ((int64_t)1 << 31))) {
    // the specialised kernel (a tile's rows hold whole tokens)
    const int64_t WR1 = 4 * kU128Passes;
    const int64_t nwt1 = (nrows + WR1 - 1) / WR1;
    const size_t seg1 = (size_t)NW * WR1 * D * 2;
    const size_t lds = seg1 + (sc.per_token ? (size_t)NW * WR1 * 16 * 2 : (size_t)H * u128_head(1 << bits) * 2);
#define HKV_D128(PT_, B_)                                                                          \
  hipLaunchKernelGGL((unpack_d128_kernel<PT_, B_>), dim3(resident_grid(unpack_d128_kernel<PT_, B_>, \
                     (nwt1 + NW - 1) / NW, lds)), dim3(kThreads), lds, s, pk, row_ptr,                \
                     col, val, capacity, nrows, lgH, sc, o, nwt1)
    if (sc.per_token) {
      if (bits == 4) HKV_D128(true, 4);
      else HKV_D128(true, 2);
    } else {
      if (bits == 4) HKV_D128(false, 4);
      else HKV_D128(false, 2);
    }
#undef HKV_D128
    HKV_CHECK_LAUNCH();
    return HKV_OK;
  }
#define HKV_UARGS G, grid, lds, s, pk, row_ptr, col, val, capacity, nrows, H, sc, o, nwtiles
  if (sc.per_token) {
    const size_t lds = seg_bytes + (size_t)NW * WR * 16 * 2;
    if (bits == 4) launch_unpack_g<true, 4, false>(HKV_UARGS);
    else launch_unpack_g<true, 2, false>(HKV_UARGS);
  } else if (seg_bytes + kpole_bytes <= 48 * 1024) {
    const size_t lds = seg_bytes + kpole_bytes;
    if (bits == 4) launch_unpack_g<false, 4, true>(HKV_UARGS);
    else launch_unpack_g<false, 2, true>(HKV_UARGS);
  } else {
    const size_t lds = seg_bytes;
    if (bits == 4) launch_unpack_g<false, 4, false>(HKV_UARGS);
    else launch_unpack_g<false, 2, false>(HKV_UARGS);
  }
#undef HKV_UARGS
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
