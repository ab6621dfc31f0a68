// nuq_unpack.hip -- compact unpack: bit-packed nuq codes + CSR outliers
// (the format written by nuq_compact.hip) -> fp16, one tensor per call or a
// batch of tensors per launch.
#include "nuq_launch.h"

#include <vector>

namespace {

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
  // Whole rounds of three tiles with no exit between the steps (an exit
  // there leaves a join at the loop head through which the compiler waits
  // for every outstanding access, the last tile's stores included, before
  // the next loads), then the last one or two tiles.  At each round's start
  // L0, L1 hold tiles wt, wt + nwaves and C0 tile wt's entries.
  int64_t wt = wt0;
  for (; wt + 2 * nwaves < nwtiles; wt += 3 * nwaves) {
    step(wt, L0, C0, L1, C1, L2);
    step(wt + nwaves, L1, C1, L2, C2, L0);
    step(wt + 2 * nwaves, L2, C2, L0, C0, L1);
  }
  if (wt < nwtiles) {
    load_csr(L1, C1);
    process(wt, L0, C0);
    if (wt + nwaves < nwtiles) process(wt + nwaves, L1, C1);
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

// The body, for block blk of nblk blocks working on one tensor.
template <bool PT, int BITS>
HKV_DEV void unpack_d128_body(const uint8_t* __restrict__ packed, const int32_t* __restrict__ row_ptr,
                              const uint8_t* __restrict__ col, const uint16_t* __restrict__ val,
                              int64_t cap, int64_t nrows, int lgH, const hkv_nuq_scales& sc,
                              uint16_t* __restrict__ out, int64_t nwtiles, int blk, int nblk) {
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
  const int64_t nwaves = (int64_t)nblk * NW;
  // The CSR entry, position and output accesses below are unconditional: a
  // branch around any of them makes the compiler's waits allow for the path
  // without it, and a wait for an earlier load then also waits for the
  // previous tile's stores.  With no entries the entry loads read row_ptr's
  // first bytes (it has at least two entries).
  const uint8_t* colp = cap > 0 ? col : reinterpret_cast<const uint8_t*>(row_ptr);
  const char* valp = cap > 0 ? reinterpret_cast<const char*>(val) : reinterpret_cast<const char*>(row_ptr);
  // row_ptr entries are int32
  const uint32_t cap32 = cap <= 0 ? 1u : (uint32_t)(cap < 0x7fffffff ? cap : 0x7fffffff);
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
        // without a position array the load reads row_ptr's first 8 bytes
        const int64_t ap = sc.positions ? sc.positions[t0 + k]
                                        : *reinterpret_cast<const int64_t*>(row_ptr);
        int pos;
        if (sc.positions) {
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
#pragma unroll
    for (int p = 0; p < kU128Passes; ++p) {
      uint32_t i = (uint32_t)(L.rp[p].x > 0 ? L.rp[p].x : 0) + (uint32_t)cg;
      i = i < cap32 ? i : cap32 - 1u;
      C.c[p] = colp[i];
      C.v[p] = *reinterpret_cast<const uint16_t*>(valp + 2u * i);
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
      // a row past the end stores row lim's values again (same lane column,
      // same data), so the store needs no branch
      const int rr = p * RW + rw;
      const int rs = rr > lim ? lim : rr;
      store_stream(ob + (uint32_t)(rs * D + 8 * cg), *reinterpret_cast<const uint4*>(seg + rs * D + 8 * cg));
    }
    wave_sync();
  };
  const int64_t wt0 = (int64_t)blk * NW + wv;
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
  // Whole rounds of three tiles, then the last one or two (as in
  // unpack_compact_kernel).
  int64_t wt = wt0;
  for (; wt + 2 * nwaves < nwtiles; wt += 3 * nwaves) {
    step(wt, L0, C0, L1, C1, L2);
    step(wt + nwaves, L1, C1, L2, C2, L0);
    step(wt + 2 * nwaves, L2, C2, L0, C0, L1);
  }
  if (wt < nwtiles) {
    load_csr(L1, C1);
    process(wt, L0, C0);
    if (wt + nwaves < nwtiles) process(wt + nwaves, L1, C1);
  }
}

template <bool PT, int BITS>
__global__ void __launch_bounds__(kThreads)
unpack_d128_kernel(const uint8_t* __restrict__ packed, const int32_t* __restrict__ row_ptr,
                   const uint8_t* __restrict__ col, const uint16_t* __restrict__ val, int64_t cap,
                   int64_t nrows, int lgH, hkv_nuq_scales sc, uint16_t* __restrict__ out,
                   int64_t nwtiles) {
  unpack_d128_body<PT, BITS>(packed, row_ptr, col, val, cap, nrows, lgH, sc, out, nwtiles,
                             (int)blockIdx.x, (int)gridDim.x);
}

// One tensor of a batched unpack launch (kernel argument, by value).
struct UnpackItem {
  const uint8_t* packed;
  const int32_t* row_ptr;
  const uint8_t* col;
  const uint16_t* val;
  uint16_t* out;
  hkv_nuq_scales sc;
  int64_t cap;
  int64_t nrows;
  int64_t nwtiles;
  uint32_t blk0;  // the item's first block
  uint32_t nblk;  // its blocks
};
struct UnpackBatch {
  UnpackItem it[kBatchItems];
  int32_t n;
  int32_t lgH;
};

// Batched unpack: the launch's blocks are split among the tensors in
// proportion to their rows (every block works on one tensor, so the K poles
// it stages in LDS are that tensor's); no block depends on another.
template <bool PT, int BITS>
__global__ void __launch_bounds__(kThreads)
unpack_d128_batch_kernel(const UnpackBatch B) {
  int j = 0;
  while (j + 1 < B.n && blockIdx.x >= B.it[j + 1].blk0) ++j;
  const UnpackItem& it = B.it[j];
  unpack_d128_body<PT, BITS>(it.packed, it.row_ptr, it.col, it.val, it.cap, it.nrows, B.lgH, it.sc,
                             it.out, it.nwtiles, (int)(blockIdx.x - it.blk0), (int)it.nblk);
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

extern "C" int hkv_nuq_unpack_compact_batch(const hkv_unpack_item* items, int n, void* stream) {
  if (n < 0 || (n > 0 && !items)) return HKV_ERR_ARG;
  // argument checks first: nothing is launched if any item is bad
  for (int i = 0; i < n; ++i) {
    const hkv_unpack_item& a = items[i];
    const hkv_nuq_scales* sc = &a.scales;
    if (!sc->tables) return HKV_ERR_ARG;
    if (a.bits != 2 && a.bits != 4) return HKV_ERR_ARG;
    if (sc->per_token && sc->rows < 1) return HKV_ERR_SHAPE;
    if (a.T < 0 || a.H < 1 || !pow2_G(a.D)) return HKV_ERR_SHAPE;
    if (a.capacity < 0) return HKV_ERR_ARG;
    if (a.T == 0) continue;
    if (!a.packed || !a.row_ptr || !a.out || (a.capacity > 0 && (!a.col || !a.val))) return HKV_ERR_ARG;
    if (((uintptr_t)a.out & 15u) || ((uintptr_t)a.packed & 3u)) return HKV_ERR_ARG;
  }
  hipStream_t s = (hipStream_t)stream;
  constexpr int NW = kThreads / 64;
  const int64_t WR1 = 4 * kU128Passes;
  // items the batched D = 128 kernel takes: H a power of two dividing a wave
  // tile's rows, per-token tables addressable in 32 bits
  auto batchable = [&](const hkv_unpack_item& a) {
    const int H = a.H;
    return a.T > 0 && a.D == 128 && (H & (H - 1)) == 0 && (4 * kU128Passes) % H == 0 &&
           (!a.scales.per_token ||
            (int64_t)H * a.scales.rows * (int64_t)sizeof(hkv_table_t) < ((int64_t)1 << 31));
  };
  std::vector<char> done((size_t)n, 0);
  for (int i0 = 0; i0 < n; ++i0) {
    if (done[i0]) continue;
    const hkv_unpack_item& a0 = items[i0];
    // the single-tensor path: shapes the batched kernel does not take, and
    // per-token tensors, whose pole rows are read through L2 (the rows of a
    // whole batch in flight at once overflow it: 46 us a tensor batched
    // against 42.7 us alone for V nuq2 at 131072 x 4 x 128)
    if (!batchable(a0) || a0.scales.per_token) {
      done[i0] = 1;
      const int st = hkv_nuq_unpack_compact(a0.packed, a0.row_ptr, a0.col, a0.val, a0.capacity, a0.T,
                                            a0.H, a0.D, a0.bits, &a0.scales, a0.out, stream);
      if (st != HKV_OK) return st;
      continue;
    }
    const int pt = a0.scales.per_token != 0, bits = a0.bits, H = a0.H;
    std::vector<int> grp;
    for (int i = i0; i < n; ++i)
      if (!done[i] && batchable(items[i]) && !items[i].scales.per_token &&
          items[i].bits == bits && items[i].H == H) {
        grp.push_back(i);
        done[i] = 1;
      }
    const size_t lds = (size_t)NW * WR1 * 128 * 2 +
                       (pt ? (size_t)NW * WR1 * 16 * 2 : (size_t)H * u128_head(1 << bits) * 2);
    for (size_t g0 = 0; g0 < grp.size(); g0 += kBatchItems) {
      const size_t g1 = std::min(grp.size(), g0 + kBatchItems);
      UnpackBatch b;
      b.n = (int)(g1 - g0);
      b.lgH = __builtin_ctz((unsigned)H);
      int64_t tiles = 0;
      for (size_t g = g0; g < g1; ++g) tiles += (items[grp[g]].T * H + WR1 - 1) / WR1;
      int per_cu = 0;
      const void* kfn = pt ? (bits == 4 ? (const void*)unpack_d128_batch_kernel<true, 4>
                                        : (const void*)unpack_d128_batch_kernel<true, 2>)
                           : (bits == 4 ? (const void*)unpack_d128_batch_kernel<false, 4>
                                        : (const void*)unpack_d128_batch_kernel<false, 2>);
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kfn, kThreads, lds) != hipSuccess ||
          per_cu < 1)
        per_cu = 1;
      const int64_t resident = (int64_t)per_cu * num_cus();
      uint32_t blk = 0;
      for (size_t g = g0; g < g1; ++g) {
        const hkv_unpack_item& a = items[grp[g]];
        UnpackItem& u = b.it[g - g0];
        u.packed = (const uint8_t*)a.packed;
        u.row_ptr = a.row_ptr;
        u.col = a.col;
        u.val = a.val;
        u.out = (uint16_t*)a.out;
        u.sc = a.scales;
        u.cap = a.capacity;
        u.nrows = a.T * H;
        u.nwtiles = (u.nrows + WR1 - 1) / WR1;
        // blocks in proportion to the item's tiles, at most one per NW tiles
        int64_t nb = (resident * u.nwtiles + tiles - 1) / tiles;
        nb = std::max<int64_t>(1, std::min<int64_t>(nb, (u.nwtiles + NW - 1) / NW));
        u.blk0 = blk;
        u.nblk = (uint32_t)nb;
        blk += (uint32_t)nb;
      }
      if (pt) {
        if (bits == 4) hipLaunchKernelGGL((unpack_d128_batch_kernel<true, 4>), dim3(blk), dim3(kThreads), lds, s, b);
        else hipLaunchKernelGGL((unpack_d128_batch_kernel<true, 2>), dim3(blk), dim3(kThreads), lds, s, b);
      } else {
        if (bits == 4) hipLaunchKernelGGL((unpack_d128_batch_kernel<false, 4>), dim3(blk), dim3(kThreads), lds, s, b);
        else hipLaunchKernelGGL((unpack_d128_batch_kernel<false, 2>), dim3(blk), dim3(kThreads), lds, s, b);
      }
      HKV_CHECK_LAUNCH();
    }
  }
  return HKV_OK;
}
