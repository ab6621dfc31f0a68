// gather.hip -- gather + dequantise selected pages of the compact format into
// an fp16 staging buffer, per KV head, over a ragged batch of sequences.
//
// The compact-format counterpart of unpack_to_staging
// (src/kvquant/compact_pool.py:492-537, kernels :292-395): there the kept
// blocks are dequantised for all heads (the union of the heads' selections);
// here each head's own selection is gathered, so only the selected
// (page, head) pairs are read and written.
//
// Input: the compact K or V of the concatenated token stream of B sequences
// (sequence b owns pages [off[b], off[b+1]) of page_size tokens, tokens
// t = page * page_size + j), the selection sel (rows, H) int64 of pages local
// to each sequence (rows out_off[b] .. out_off[b+1]-1 belong to sequence b, as
// hkv_quest_select_ragged writes them).  Output row i, slot j, head h of
// staging (rows, page_size, H, D) is token (off[b] + sel[i][h]) * page_size + j
// of head h, dequantised: per-channel scales (K) by (h, d); per-token scales (V)
// by row min(sel[i][h] * page_size + j, rows - 1), the token's position within
// its sequence.  Pages outside [0, off[b+1] - off[b]) give zero rows.
//
// One wave per (row, head) item: lane l dequantises slot l/4, channels
// [32(l%4), +32) through LUTs in LDS (K: the per-channel poles of every head,
// staged once per block; V: the slots' per-token poles) into the wave's LDS
// tile of the item (16 slots x 128 channels), the four lanes of a slot patch
// the slot's CSR outliers into the tile (its first 16 entries requested
// together), and the lanes write the tile's rows with 128-bit stores.  The
// items of a wave are pipelined: the selection entry of the item after next
// and the codes and row offsets of the next item are in flight while an
// item is dequantised.
#include "hkv_common.h"

namespace {

constexpr int kGT = 512;  // 8 waves share the block's K LUT
constexpr int kGW = kGT / 64;
constexpr int kGD = 128;        // head dim
constexpr int kGPS = 16;        // page size (tokens)
constexpr int kMaxSeqsG = 64;
constexpr int kGTile = kGPS * kGD;  // u16 per wave tile
constexpr int kGCsr = 4;            // CSR entries per lane requested with the item
constexpr int kGHeavy = 16;         // slots with more entries recorded per wave

struct GSegs {
  int64_t off[kMaxSeqsG + 1];
  int64_t out_off[kMaxSeqsG + 1];
  int nseg;
};

struct GArgs {
  const uint8_t* packed;
  const int32_t* row_ptr;
  const uint8_t* col;
  const uint16_t* val;
  int64_t cap;
  const hkv_table_t* tabs;
  int64_t rows;           // per-token scale rows (V)
  int64_t T;
  int H;
  const int64_t* sel;
  int64_t nrows;          // selection rows
  uint16_t* out;          // (nrows, kGPS, H, kGD)
};

// K LUT index of (head, channel, level), skewed per 32-channel group as in the
// decode kernel (conflict-free gathers for 32 or 64 banks).
HKV_DEV int glut_index(int h, int ch, int c) { return h * (kGD * 16 + 64) + ch * 16 + 16 * (ch >> 5) + c; }

HKV_DEV void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Where item x (selection row i = x / H, head h) reads from: its sequence b,
// whether its page is valid for the lane's slot, and the compact row r.
struct GItem {
  int64_t i, r, lp;
  int h;
  bool page_ok, ok;
};

HKV_DEV GItem item_at(const GArgs& A, const GSegs& sg, int64_t x, int64_t lp, int row) {
  GItem g;
  g.i = x / A.H;
  g.h = (int)(x - g.i * A.H);
  int b = 0;  // sequence of selection row i (uniform)
  while (b + 1 < sg.nseg && sg.out_off[b + 1] <= g.i) ++b;
  const int64_t P = sg.off[b + 1] - sg.off[b];
  g.lp = lp;
  g.page_ok = lp >= 0 && lp < P;
  const int64_t t = (sg.off[b] + (g.page_ok ? lp : 0)) * kGPS + row;
  g.ok = g.page_ok && t < A.T;
  g.r = (g.ok ? t : 0) * A.H + g.h;
  return g;
}

// The loads of an item that follow from its selection entry: the lane's
// codes, its slot's row offsets and (V) four of its slot's poles.
template <int NB, bool PT>
struct GLoads {
  uint32_t w[NB];
  int2 rb;
  uint2 tv;
};

template <int NB, bool PT>
HKV_DEV void fetch_item(const GArgs& A, const GItem& g, int row, int q, GLoads<NB, PT>& L) {
  if constexpr (NB == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(A.packed + g.r * (kGD / 2) + q * 16);
    L.w[0] = v.x; L.w[1] = v.y; L.w[2] = v.z; L.w[3] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(A.packed + g.r * (kGD / 4) + q * 8);
    L.w[0] = v.x; L.w[1] = v.y;
  }
  L.rb = *reinterpret_cast<const int2*>(A.row_ptr + g.r);
  if constexpr (PT) {
    const int64_t pos = (g.page_ok ? g.lp : 0) * kGPS + row;
    const int64_t vrow = pos < A.rows ? pos : A.rows - 1;
    L.tv = *reinterpret_cast<const uint2*>(A.tabs[(int64_t)g.h * A.rows + vrow].pf16 + 4 * q);
  } else {
    L.tv = make_uint2(0u, 0u);
  }
}

// Slots with more than 4 * kGCsr CSR entries, recorded by a wave for a pass
// after its item loop (their remaining entries are loaded there, so the item
// loop issues a fixed number of loads per item and every wait in it is exact).
struct GHeavy {
  int64_t x[kGHeavy];
  int slot[kGHeavy];
};

// Dequantise, patch and write item x (g; its loads L in flight); `prefetch`
// issues the loads of the items ahead once this item's CSR entries are
// requested.
template <int NB, bool PT, typename Pre>
HKV_DEV void gather_item(const GArgs& A, int64_t x, const GItem& g, const GLoads<NB, PT>& L, int row,
                         int q, uint16_t* tile, uint16_t* vl, const uint16_t* klut, GHeavy& hv,
                         int& nheavy, Pre prefetch) {
  // this slot's CSR entries [a, e); the first 4 x kGCsr are requested at once
  // (clamped indexes: the loads are unconditional)
  const int64_t a = L.rb.x < 0 ? 0 : L.rb.x;
  int64_t e = L.rb.y < A.cap ? L.rb.y : A.cap;
  if (!g.ok) e = a;
  // (with no CSR capacity col / val point at 4 readable bytes, and e = 0)
  uint32_t ce[kGCsr];  // val | col << 16
#pragma unroll
  for (int u = 0; u < kGCsr; ++u) {
    const int64_t k = a + q + 4 * u;
    const int64_t kc = k < e ? k : (e > 0 ? e - 1 : 0);
    ce[u] = (uint32_t)A.val[kc] | ((uint32_t)A.col[kc] << 16);
  }
  prefetch();
  if constexpr (PT) {
    *reinterpret_cast<uint2*>(vl + row * 16 + 4 * q) = L.tv;
    wave_lds_sync();
  }
  uint32_t o[16];
#pragma unroll
  for (int e2 = 0; e2 < 16; ++e2) {
    uint32_t pr = 0;
#pragma unroll
    for (int hl = 0; hl < 2; ++hl) {
      const int c = 2 * e2 + hl;  // channel 32q + c
      uint32_t code;
      if constexpr (NB == 4) code = (L.w[c >> 3] >> (4 * (c & 7))) & 15u;
      else code = (L.w[c >> 4] >> (2 * (c & 15))) & 3u;
      uint16_t v;
      if constexpr (PT) v = vl[row * 16 + (int)code];
      else v = klut[glut_index(g.h, 32 * q + c, (int)code)];
      pr |= (uint32_t)v << (16 * hl);
    }
    o[e2] = g.ok ? pr : 0u;
  }
  uint4* trow = reinterpret_cast<uint4*>(tile + row * kGD + 32 * q);
#pragma unroll
  for (int k = 0; k < 4; ++k) trow[k] = make_uint4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
  wave_lds_sync();  // the slot's other lanes have written their channels
#pragma unroll
  for (int u = 0; u < kGCsr; ++u)
    if (a + q + 4 * u < e) tile[row * kGD + ((ce[u] >> 16) & (kGD - 1))] = (uint16_t)ce[u];
  // slots with more entries: recorded (the first kGHeavy of the wave)
  const bool heavy = q == 0 && e - a > 4 * kGCsr;
  const uint64_t hb = __ballot(heavy);
  if (hb) {  // uniform
    const int rank = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(hb >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)hb, 0u));
    if (heavy && nheavy + rank < kGHeavy) {
      hv.x[nheavy + rank] = x;
      hv.slot[nheavy + rank] = row;
    }
    nheavy += __builtin_popcountll(hb);
  }
  wave_lds_sync();
  uint4* dst = reinterpret_cast<uint4*>(A.out + ((g.i * kGPS + row) * A.H + g.h) * kGD + 32 * q);
  // plain stores: a store instruction covers 16-byte pieces of several
  // lines, which L2 merges (streaming stores would write them out partial)
#pragma unroll
  for (int k = 0; k < 4; ++k) dst[k] = trow[k];
  wave_lds_sync();  // the tile and the V LUT are rewritten by the next item
}

template <int NB, bool PT>
__global__ void __launch_bounds__(kGT)
gather_pages_kernel(GArgs A, const GSegs sg) {
  // [kGW][kGTile] output tiles, then K: [H][kGD*16+64] LUT; V: [kGW][16][16]
  extern __shared__ __align__(16) uint16_t g_lds[];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int H = A.H;
  uint16_t* tile = g_lds + wv * kGTile;
  uint16_t* lut = g_lds + kGW * kGTile;
  if constexpr (!PT) {
    for (int i = tid; i < H * kGD * 16; i += kGT) {
      const int h = i / (kGD * 16), d = (i / 16) % kGD, l = i % 16;
      lut[glut_index(h, d, l)] = A.tabs[(int64_t)h * kGD + d].pf16[l];
    }
    __syncthreads();
  }
  uint16_t* vl = lut + wv * (kGPS * 16);
  __shared__ GHeavy s_heavy[kGW];
  GHeavy& hv = s_heavy[wv];
  int nheavy = 0;  // wave-uniform
  const int row = lane >> 2, q = lane & 3;
  const int64_t items = A.nrows * H;
  const int64_t S = (int64_t)gridDim.x * kGW;
  const int64_t xfirst = (int64_t)blockIdx.x * kGW + wv;
  int64_t x0 = xfirst;
  if (x0 >= items) return;  // the whole wave (no block barrier follows)
  auto clampx = [&](int64_t x) { return x < items ? x : items - 1; };
  // The wave's items in chunks of 64: one lane loads the selection entry of
  // each item of the chunk, and the items read theirs by readlane (no memory
  // wait).  Within a chunk, two register sets: the loads of the next item go
  // into the set that is not being used (no pending load is copied; past the
  // chunk's end they repeat its last item).
  for (int64_t xc = xfirst; xc < items; xc += 64 * S) {
    const int64_t selb = A.sel[clampx(xc + (int64_t)lane * S)];
    const int nk = (int)((items - xc + S - 1) / S < 64 ? (items - xc + S - 1) / S : 64);
    auto sel_k = [&](int k) {
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)selb, k);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)selb >> 32), k);
      return (int64_t)(((uint64_t)hi << 32) | lo);
    };
    auto item_k = [&](int k) {
      const int kk = k < nk ? k : nk - 1;
      return item_at(A, sg, xc + (int64_t)kk * S, sel_k(kk), row);
    };
    GItem g0 = item_k(0), g1;
    GLoads<NB, PT> l0, l1;
    fetch_item<NB, PT>(A, g0, row, q, l0);
    for (int k = 0;;) {
      gather_item<NB, PT>(A, xc + (int64_t)k * S, g0, l0, row, q, tile, vl, lut, hv, nheavy, [&] {
        g1 = item_k(k + 1);
        fetch_item<NB, PT>(A, g1, row, q, l1);
      });
      if (++k >= nk) break;
      gather_item<NB, PT>(A, xc + (int64_t)k * S, g1, l1, row, q, tile, vl, lut, hv, nheavy, [&] {
        g0 = item_k(k + 1);
        fetch_item<NB, PT>(A, g0, row, q, l0);
      });
      if (++k >= nk) break;
    }
  }
  if (nheavy == 0) return;
  // The remaining entries of the recorded slots (all slots of the wave's
  // items if more were heavy than recorded), stored into the written rows
  // once the rows' stores are complete.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  wave_lds_sync();
  auto patch = [&](int64_t x, int slot, int first, int step) {
    const GItem g = item_at(A, sg, x, A.sel[x], slot);
    if (!g.ok) return;
    const int2 rb = *reinterpret_cast<const int2*>(A.row_ptr + g.r);
    const int64_t a = (rb.x < 0 ? 0 : rb.x) + 4 * kGCsr;
    const int64_t e = rb.y < A.cap ? rb.y : A.cap;
    uint16_t* orow = A.out + ((g.i * kGPS + slot) * A.H + g.h) * kGD;
    for (int64_t k = a + first; k < e; k += step) orow[A.col[k] & (kGD - 1)] = A.val[k];
  };
  if (nheavy <= kGHeavy) {
    for (int j = 0; j < nheavy; ++j) patch(hv.x[j], hv.slot[j], lane, 64);
  } else {
    for (int64_t x = xfirst; x < items; x += S) patch(x, row, q, 4);
  }
}

int gather_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

}  // namespace

extern "C" int hkv_nuq_gather_pages(const void* packed, const int32_t* row_ptr, const uint8_t* col,
                                    const uint16_t* val, int64_t capacity, int64_t T, int H, int D,
                                    int bits, const hkv_nuq_scales* scales, int page_size, int B,
                                    const int64_t* page_offsets, const int64_t* out_offsets,
                                    const int64_t* sel, void* out, void* stream) {
  if (!scales) return HKV_ERR_ARG;
  if (D != kGD || page_size != kGPS) return HKV_ERR_SHAPE;
  if (B < 1 || B > kMaxSeqsG || H < 1 || T < 0) return HKV_ERR_SHAPE;
  if (bits != 2 && bits != 4) return HKV_ERR_ARG;
  if (!page_offsets || !out_offsets) return HKV_ERR_ARG;
  if (T * H * D >= ((int64_t)1 << 31)) return HKV_ERR_SHAPE;
  GSegs sg;
  sg.nseg = B;
  if (page_offsets[0] != 0 || out_offsets[0] != 0) return HKV_ERR_ARG;
  for (int b = 0; b <= B; ++b) {
    if (b > 0 && (page_offsets[b] < page_offsets[b - 1] || out_offsets[b] < out_offsets[b - 1]))
      return HKV_ERR_ARG;
    sg.off[b] = page_offsets[b];
    sg.out_off[b] = out_offsets[b];
  }
  if (page_offsets[B] * page_size > T) return HKV_ERR_SHAPE;
  const int64_t nrows = out_offsets[B];
  if (nrows == 0) return HKV_OK;
  if (T < 1) return HKV_ERR_SHAPE;
  if (!packed || !row_ptr || !scales->tables || !sel || !out || capacity < 0) return HKV_ERR_ARG;
  if (capacity > 0 && (!col || !val)) return HKV_ERR_ARG;
  const bool pt = scales->per_token != 0;
  if (pt && scales->rows < 1) return HKV_ERR_ARG;
  if (((uintptr_t)packed & 15u) || ((uintptr_t)out & 15u) || ((uintptr_t)row_ptr & 3u))
    return HKV_ERR_ARG;
  const size_t lds = sizeof(uint16_t) * kGW * kGTile +
                     (pt ? sizeof(uint16_t) * kGW * kGPS * 16 : sizeof(uint16_t) * H * (kGD * 16 + 64));
  if (lds > 64 * 1024) return HKV_ERR_SHAPE;
  GArgs a;
  a.packed = (const uint8_t*)packed;
  a.row_ptr = row_ptr;
  // no CSR capacity: the kernel's clamped CSR loads read row_ptr's first
  // bytes instead (their results are never applied)
  a.col = capacity > 0 ? col : (const uint8_t*)row_ptr;
  a.val = capacity > 0 ? val : (const uint16_t*)row_ptr;
  a.cap = capacity;
  a.tabs = (const hkv_table_t*)scales->tables;
  a.rows = scales->rows;
  a.T = T;
  a.H = H;
  a.sel = sel;
  a.nrows = nrows;
  a.out = (uint16_t*)out;
  const int64_t items = nrows * H;
  hipStream_t s = (hipStream_t)stream;
  // a resident grid (the items are strided over its waves)
  auto launch = [&](auto kernel) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kGT, lds) != hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    const unsigned grid =
        (unsigned)std::min<int64_t>((items + kGW - 1) / kGW, (int64_t)gather_cus() * per_cu);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kGT), lds, s, a, sg);
  };
  if (bits == 4) {
    if (pt) launch(gather_pages_kernel<4, true>);
    else launch(gather_pages_kernel<4, false>);
  } else {
    if (pt) launch(gather_pages_kernel<2, true>);
    else launch(gather_pages_kernel<2, false>);
  }
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
