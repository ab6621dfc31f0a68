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
// Pack runs as two kernels.  pack_stage_kernel streams the fp16 input once:
// it writes the packed codes, each row's outlier offset within its tile (into
// row_ptr), the tile's outliers into the tile's own region of a staging
// buffer, and the tile's outlier count.  compact_kernel then turns the tile
// counts into tile offsets, adds them to row_ptr and copies the staged
// outliers into the dense col/val arrays.  No block ever waits on another:
// on gfx950 the eight XCDs' L2 caches are not coherent, so a single-pass scan
// whose tiles wait on their predecessors pays a memory round trip per step.
#include "nuq_core.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPasses = 8;  // passes of kThreads*8 elements per tile

// Workspace: header, per-tile counts, then the staging columns and values,
// each region 256-byte aligned.  Staging holds a whole tile per tile, so no
// input can overflow it.
struct PackLayout {
  int64_t ntiles, tile_elems;
  size_t cnt_off, col_off, val_off, bytes;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// KFIX: the rows per pass are a multiple of H, so a thread's head is fixed
// (rl % H) and its token advances by R / H per pass (no 64-bit division in
// the loop).
template <int NB, bool PT, int G, int BITS, bool KFIX>
__global__ void __launch_bounds__(kThreads)
pack_stage_kernel(const uint16_t* __restrict__ x, int64_t nrows, int H, hkv_nuq_scales sc,
                  uint8_t* __restrict__ packed, int32_t* __restrict__ row_ptr,
                  uint8_t* __restrict__ scol, uint16_t* __restrict__ sval,
                  uint32_t* __restrict__ tile_cnt, uint32_t ntiles) {
  constexpr int R = kThreads / G;   // rows per pass
  constexpr int TR = R * kPasses;   // rows per tile
  constexpr int D = 8 * G;
  constexpr int RB = D * BITS / 8;  // packed bytes per row
  constexpr int NW = kThreads / 64;
  // Per-token tables of the tile's rows are staged in LDS when they fit in
  // 16 KiB (D >= 128); otherwise each row reads its table through L1.
  constexpr bool STAGE = PT && TR * 80 <= 16384;
  __shared__ uint32_t s_wave[kPasses][NW];
  __shared__ uint4 s_tab[STAGE ? TR * 5 : 1];

  const int tid = threadIdx.x, cg = tid % G, rl = tid / G;
  const int wv = tid >> 6, lane = tid & 63;
  const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;
  const SlowInfo si = slow_info(sc);
  const int hfix = KFIX ? rl % H : 0;

  Search2<NB> S[PT ? 1 : 4];
  if constexpr (!PT && KFIX) {
    const int64_t tab0 = (int64_t)hfix * D + 8 * cg;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      load_search_pair<NB>(tabs + tab0 + 2 * j, tabs + tab0 + 2 * j + 1, S[j]);
  }

  for (uint32_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t r0 = (int64_t)tile * TR;
    const int64_t t0 = KFIX ? r0 / H : 0;  // token of row r0 (H divides r0)
    uint32_t xs[kPasses][4];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int64_t r = r0 + p * R + rl;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (r < nrows) v = *reinterpret_cast<const uint4*>(x + r * D + 8 * cg);
      xs[p][0] = v.x; xs[p][1] = v.y; xs[p][2] = v.z; xs[p][3] = v.w;
    }
    if constexpr (STAGE) {
      for (int i = tid; i < TR * 5; i += kThreads) {
        const int rr = i / 5, part = i - rr * 5;
        const int64_t r = r0 + rr;
        if (r < nrows) {
          const int64_t t = r / H;
          const int h = (int)(r - t * H);
          const int64_t tab = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
          s_tab[i] = reinterpret_cast<const uint4*>(tabs + tab)[part];
        }
      }
      __syncthreads();
    }

    uint32_t mk[kPasses], excl[kPasses];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int rr = p * R + rl;
      const int64_t r = r0 + rr;
      mk[p] = 0;
      if (r < nrows) {
        int64_t t;
        int h;
        if constexpr (KFIX) {
          t = t0 + p * (R / H) + rl / H;
          h = hfix;
        } else {
          t = r / H;
          h = (int)(r - t * H);
        }
        const uint4 xv = make_uint4(xs[p][0], xs[p][1], xs[p][2], xs[p][3]);
        uint32_t c[4], om[4];
        if constexpr (PT) {
          const int64_t tab = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
          if constexpr (STAGE) load_search_bcast<NB>(reinterpret_cast<const hkv_table_t*>(s_tab + rr * 5), S[0]);
          else load_search_bcast<NB>(tabs + tab, S[0]);
          quant8<NB, PT>(xv, S, si, RowTab{tab}, c, om);
        } else {
          const int64_t tab0 = (int64_t)h * D + 8 * cg;
          if constexpr (!KFIX) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              load_search_pair<NB>(tabs + tab0 + 2 * j, tabs + tab0 + 2 * j + 1, S[j]);
          }
          quant8<NB, PT>(xv, S, si, ChanTab{tab0}, c, om);
        }
        if constexpr (BITS == 4) {
          *reinterpret_cast<uint32_t*>(packed + r * RB + 4 * cg) = pack_nibbles(c);
        } else {
          *reinterpret_cast<uint16_t*>(packed + r * RB + 2 * cg) = (uint16_t)pack_crumbs(c);
        }
        mk[p] = mask_bits(om);
      }
      uint32_t tot;
      excl[p] = wave_excl_count(__builtin_popcount(mk[p]), &tot);
      if (lane == 0) s_wave[p][wv] = tot;
    }
    __syncthreads();

    // Offsets within the tile in (pass, wave, lane) order = (row, col) order.
    uint32_t total = 0;
    const int64_t sbase = r0 * D;  // the tile's staging region
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      uint32_t before = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) before += w < wv ? s_wave[p][w] : 0u;
      uint32_t pos = total + before + excl[p];
#pragma unroll
      for (int w = 0; w < NW; ++w) total += s_wave[p][w];
      const int64_t r = r0 + p * R + rl;
      if (r >= nrows) continue;
      if (cg == 0) row_ptr[r] = (int32_t)pos;
      uint32_t m = mk[p];
      while (m) {
        const int e = __builtin_ctz(m);
        m &= m - 1u;
        const uint32_t w = pick4(xs[p][0], xs[p][1], xs[p][2], xs[p][3], e >> 1);
        scol[sbase + pos] = (uint8_t)(8 * cg + e);
        sval[sbase + pos] = (uint16_t)(w >> (16 * (e & 1)));
        ++pos;
      }
    }
    if (tid == 0) tile_cnt[tile] = total;
    __syncthreads();  // s_wave / s_tab are reused by the next tile
  }
}

// Tile offsets from the tile counts, then the dense CSR.  One wave per tile
// (kCompactTiles per block); a block first sums the counts of all tiles before
// its own with every thread loading in parallel.
constexpr int kCompactTiles = kThreads / 64;
constexpr int kCopyUnroll = 4;

__global__ void __launch_bounds__(kThreads)
compact_kernel(const uint32_t* __restrict__ tile_cnt, uint32_t ntiles, int64_t TR, int64_t D,
               int64_t nrows, const uint8_t* __restrict__ scol, const uint16_t* __restrict__ sval,
               int32_t* __restrict__ row_ptr, uint8_t* __restrict__ col,
               uint16_t* __restrict__ val, uint32_t cap) {
  __shared__ uint32_t s_red[kThreads / 64];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t t0 = blockIdx.x * kCompactTiles;
  uint32_t acc = 0;
  for (uint32_t i = tid; i < t0; i += kThreads) acc += tile_cnt[i];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (lane == 0) s_red[wv] = acc;
  __syncthreads();
  uint32_t base = 0;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) base += s_red[w];
  const uint32_t tile = t0 + wv;
  if (tile >= ntiles) return;
  // counts of the block's earlier tiles, and this tile's
  const uint32_t mine = lane < kCompactTiles && t0 + lane < ntiles ? tile_cnt[t0 + lane] : 0u;
#pragma unroll
  for (int w = 0; w < kCompactTiles; ++w) {
    const uint32_t c = __shfl(mine, w, 64);
    if (w < wv) base += c;
  }
  const uint32_t n = __shfl(mine, wv, 64);
  const int64_t r0 = (int64_t)tile * TR;
  for (int64_t i = lane; i < TR; i += 64) {
    const int64_t r = r0 + i;
    if (r < nrows) row_ptr[r] += (int32_t)base;
  }
  if (tile == ntiles - 1 && lane == 0) row_ptr[nrows] = (int32_t)(base + n);
  const int64_t src = r0 * D;
  for (uint32_t i0 = 0; i0 < n; i0 += 64 * kCopyUnroll) {
    uint8_t cv[kCopyUnroll];
    uint16_t vv[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const uint32_t i = i0 + u * 64 + lane;
      if (i < n) { cv[u] = scol[src + i]; vv[u] = sval[src + i]; }
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const uint32_t i = i0 + u * 64 + lane;
      if (i < n && base + i < cap) { col[base + i] = cv[u]; val[base + i] = vv[u]; }
    }
  }
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

HKV_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

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

  const int64_t nwaves = (int64_t)gridDim.x * NW;
  for (int64_t wt = (int64_t)blockIdx.x * NW + wv; wt < nwtiles; wt += nwaves) {
    const int64_t r0 = wt * WR;
    uint32_t cw[kUPasses];
    int32_t ra[kUPasses], rb[kUPasses];
#pragma unroll
    for (int p = 0; p < kUPasses; ++p) {
      const int64_t r = r0 + p * RW + rw;
      cw[p] = 0;
      ra[p] = rb[p] = 0;
      if (r < nrows) {
        if constexpr (BITS == 4) cw[p] = *reinterpret_cast<const uint32_t*>(packed + r * RB + 4 * cg);
        else cw[p] = *reinterpret_cast<const uint16_t*>(packed + r * RB + 2 * cg);
        ra[p] = row_ptr[r];
        rb[p] = row_ptr[r + 1];
      }
    }
    if constexpr (PT) {
#pragma unroll
      for (int p = 0; p < kUPasses; ++p) {
        const int64_t r = r0 + p * RW + rw;
        if (r < nrows && cg < 2) {
          const int64_t t = r / H;
          const int h = (int)(r - t * H);
          const int64_t tab = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
          const uint4 v = reinterpret_cast<const uint4*>(tabs[tab].pf16)[cg];
          *reinterpret_cast<uint4*>(prow + (p * RW + rw) * 16 + 8 * cg) = v;
        }
      }
      wave_sync();
    }
#pragma unroll
    for (int p = 0; p < kUPasses; ++p) {
      const int rr = p * RW + rw;
      const int64_t r = r0 + rr;
      if (r >= nrows) continue;
      const int h = (int)(r % H);
      uint32_t res[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t pr = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int e = 2 * j + k;
          const uint32_t c = (cw[p] >> (BITS * e)) & ((1u << BITS) - 1u);
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
      const int32_t lo = ra[p] > 0 ? ra[p] : 0;
      const int32_t hi = (int64_t)rb[p] < cap ? rb[p] : (int32_t)cap;
      for (int32_t i = lo + cg; i < hi; i += G) {
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
      *reinterpret_cast<uint4*>(out + r * D + 8 * cg) =
          *reinterpret_cast<const uint4*>(seg + rr * D + 8 * cg);
    }
    wave_sync();
  }
}

__global__ void write_zero_rowptr(int32_t* row_ptr) { row_ptr[0] = 0; }

bool pow2_G(int D) { return D % 8 == 0 && D >= 8 && D <= 256 && ((D / 8) & (D / 8 - 1)) == 0; }

PackLayout pack_layout(int64_t nrows, int D) {
  PackLayout L;
  const int64_t TR = (int64_t)(kThreads / (D / 8)) * kPasses;
  L.ntiles = (nrows + TR - 1) / TR;
  L.tile_elems = TR * D;
  L.cnt_off = 256;
  L.col_off = L.cnt_off + align256(sizeof(uint32_t) * (size_t)L.ntiles);
  L.val_off = L.col_off + align256((size_t)(L.ntiles * L.tile_elems));
  L.bytes = L.val_off + sizeof(uint16_t) * (size_t)(L.ntiles * L.tile_elems);
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
unsigned resident_grid(K kernel, int64_t ntiles) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  return (unsigned)std::min<int64_t>(ntiles, (int64_t)per_cu * num_cus());
}

struct PackArgs {
  const uint16_t* x;
  int64_t nrows;
  int H;
  hkv_nuq_scales sc;
  uint8_t* pk;
  int32_t* rp;
  uint8_t* scol;
  uint16_t* sval;
  uint32_t* cnt;
  uint32_t ntiles;
  hipStream_t s;
};

template <int NB, bool PT, int G, int BITS, bool KFIX>
void launch_stage(const PackArgs& a) {
  auto k = pack_stage_kernel<NB, PT, G, BITS, KFIX>;
  hipLaunchKernelGGL(k, dim3(resident_grid(k, a.ntiles)), dim3(kThreads), 0, a.s, a.x, a.nrows,
                     a.H, a.sc, a.pk, a.rp, a.scol, a.sval, a.cnt, a.ntiles);
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
  return pack_layout(T * H, D).bytes;
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
  const PackLayout lay = pack_layout(nrows, D);
  if (!workspace || workspace_bytes < lay.bytes || ((uintptr_t)workspace & 255u))
    return HKV_ERR_WORKSPACE;
  const int G = D / 8, R = kThreads / G;
  char* ws = (char*)workspace;
  PackArgs a;
  a.x = (const uint16_t*)values;
  a.nrows = nrows;
  a.H = H;
  a.sc = *scales;
  a.pk = (uint8_t*)packed;
  a.rp = row_ptr;
  a.scol = (uint8_t*)(ws + lay.col_off);
  a.sval = (uint16_t*)(ws + lay.val_off);
  a.cnt = (uint32_t*)(ws + lay.cnt_off);
  a.ntiles = (uint32_t)lay.ntiles;
  a.s = s;
  const bool kfix = (R % H) == 0;
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
  const unsigned cgrid = (unsigned)((lay.ntiles + kCompactTiles - 1) / kCompactTiles);
  hipLaunchKernelGGL(compact_kernel, dim3(cgrid), dim3(kThreads), 0, s, a.cnt, a.ntiles,
                     (int64_t)R * kPasses, (int64_t)D, nrows, a.scol, a.sval, row_ptr, col, val,
                     cap);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" int hkv_nuq_pack_compact_status(const void* workspace, void* stream) {
  // The two-kernel pack has no device-side failure mode; kept for callers
  // that check it.
  (void)stream;
  return workspace ? 0 : HKV_ERR_ARG;
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
