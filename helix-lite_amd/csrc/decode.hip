// decode.hip -- decode attention over Quest-selected pages (batch 1).
//
// 1. hkv_decode_attn: fused dequant + sparse attention from the compact format.
//    Replaces the reference's decode path unpack_to_staging +
//    flash_attn_varlen_func over an fp16 staging copy
//    (src/kvquant/compact_backend.py:233-299): the selected pages are read
//    straight from the compact format (bit-packed nuq2/nuq4 codes + CSR
//    outliers over rows t*H + h, as written by hkv_nuq_pack_compact),
//    dequantised in LDS and fed to MFMA.  For query head hq (KV head
//    g = hq / group): softmax(q . K^T * scale) . V over the tokens of the pages
//    sel[0..nsel)[g] (page p = tokens [16p, 16p+16), tokens >= T masked), fp32
//    softmax -- the restatement of src/quest/reference.py:136-168 with the
//    standard GQA head map.
//
//    Work: grid (splits, H); a split is a run of pps consecutive selected
//    pages of one KV head; wave w of the block takes pages w, w+4, ... of the
//    split (at most 64, one page id per lane).  Per page a wave
//      - dequantises the 16 rows' K and V codes through LUTs in LDS (K: the
//        per-channel poles of head g, staged once per block in a bank-swizzled
//        [channel][level] layout; V: the rows' per-token poles, row
//        min(t, rows-1)) into padded fp16 tiles [16 keys][136],
//      - writes the rows' CSR outliers over the tiles,
//      - S^T = K Q^T with 8 v_mfma_f32_16x16x16f16 (lane l: query head l%16
//        of the group, keys 4*(l/16)..+3), online softmax per query head,
//      - O^T += V^T P^T with 8 more MFMAs, P straight from S's registers.
//    Global loads run three pages ahead of the math in a software pipeline:
//    while page i is computed, the CSR entries of page i+1 (whose row_ptr
//    arrived during page i-1) and the codes, pole rows and row_ptr of page
//    i+2 are in flight, so no global latency sits between two pages.
//    The 4 waves' (m, l, O) are merged through LDS into one partial per split.
//
// 2. hkv_selected_attention: the same attention over dense K/V pages
//    (P, page, H, D) in fp16/fp32/bf16 -- the drop-in for selected_attention
//    (src/quest/reference.py:136-168), any page size, head dims <= 512.
//
// merge_kernel combines the splits of either kernel (flash-decoding):
// out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s, m in log2 units.
#include "hkv_common.h"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kDT = 256;        // threads per block
constexpr int kW = kDT / 64;    // waves per block
constexpr int kHD = 128;        // head dim of the fused kernel
constexpr int kPS = 16;         // tokens per page
constexpr int kTS = kHD + 8;    // padded tile row (halves)
constexpr int kMaxPPS = 256;    // pages per split: at most 64 per wave
constexpr int kSlots = 3;       // CSR entries per lane per side kept in registers
constexpr int kKLut = kHD * 16 + 16 * 4;  // halves of the swizzled K LUT
constexpr float kLog2e = 1.4426950408889634f;

// K LUT index of (channel, level).  A lane dequantises channels
// [32q, 32q+32) of one row (q = lane % 4); for a fixed channel offset the
// 16 lanes of one q read one channel's 8 words, and the 16-half skew per
// q puts the four q groups on disjoint banks (32 or 64 banks).
HKV_DEV int klut_index(int ch, int c) { return ch * 16 + 16 * (ch >> 5) + c; }

// nuq2 pair tables: one 32-bit word holds the two fp16 values of a pair of
// adjacent channels' codes, so a lane makes one table read (and one address)
// per two codes and stores the word as it is.  K: pair p = channels (2p,
// 2p+1) of the block's KV head, entry x = c0 | c1 << 2 (the pair's 4 code
// bits) -> pole(2p, c0) | pole(2p+1, c1) << 16, at word kpair_index(p, x)
// (the 16-word skew per 16 pairs puts the four channel groups of a wave on
// disjoint banks).  V: per row, entry x -> pole(c0) | pole(c1) << 16 of the
// row's per-token poles.
HKV_DEV int kpair_index(int p, int x) { return p * 16 + 16 * (p >> 4) + x; }
constexpr int kKPair = 64 * 16 + 16 * 4;  // words
constexpr int kKLutWords = kKPair > kKLut / 2 ? kKPair : kKLut / 2;

struct Side {  // one of K / V in the compact format, or in the paged pool
  const uint8_t* packed;   // compact: (T, H, D*bits/8); paged: (NB, H, 16, D*bits/8)
  const int32_t* row_ptr;  // compact: (T*H + 1)
  const uint8_t* col;      // compact: (cap)
  const uint16_t* val;     // compact: (cap)
  int64_t cap;             // compact: CSR entries; paged: entries per page-head
  const hkv_table_t* tabs; // decision tables: pf16 are the dequantised poles
  int64_t rows;            // per-token scale rows (V); unused for K
  const int32_t* ocnt;     // paged: (NB, H) outliers per page-head
  const uint32_t* oent;    // paged: (NB, H, cap) value | channel << 16 | slot << 24
  const int32_t* ovf;      // paged: (NB, H) overflow chunk (entries cap..), -1 none; or NULL
  const uint32_t* ovf_ent; // paged: (chunks, 16 * 128 - cap)
};

struct DecodeArgs {
  const uint16_t* q;  // (Hq, D) fp16
  Side k, v;
  int H, group;
  int64_t T, npages;
  const int64_t* sel;  // (nsel, H)
  int64_t nsel;
  const int64_t* bt;   // paged: logical page -> pool block (npages entries)
  int64_t nblocks;     // paged: blocks in the pool
  int pps;             // pages per split
  float scale;
  float* part_m;       // (splits, Hq)
  float* part_l;       // (splits, Hq)
  float* part_o;       // (splits, Hq, D)
};

HKV_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Loads of one page that depend only on its id.  Lane l covers row l/4 and
// channels [32(l%4), +32): NB dwords of codes per side (nuq4: 4, nuq2: 2),
// row_ptr[r] and row_ptr[r+1] of its row, and levels 4(l%4)..+3 of its row's
// V poles.  Every load is unconditional from an in-bounds address (row 0 for
// rows past the context, whose data the math ignores), so no load result is
// moved or combined before it is used: the loads stay in flight across the
// pipeline stages.  Offsets fit in 32 bits (T*H*D < 2^31 is checked).
template <int KB, int VB>
struct PageLoad {
  uint32_t kc[KB], vc[VB];
  uint2 vtab;
  int2 kr, vr;
};

// The page's CSR entries: lane l holds entries a + l%4 + 4s (s < kSlots) of
// its row (index clamped into [0, cap); whether an entry belongs to the row is
// decided from row_ptr when it is used).
struct PageOutl {
  uint32_t kval[kSlots], kcol[kSlots], vval[kSlots], vcol[kSlots];
};

template <int NB>
HKV_DEV void load_codes(const uint8_t* packed, int r, int q, uint32_t (&w)[NB]) {
  const uint8_t* base = packed + (uint32_t)(r * (kHD * NB / 8) + q * (32 * NB / 8));
  if constexpr (NB == 4) {
    const uint4 v = *reinterpret_cast<const uint4*>(base);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(base);
    w[0] = v.x; w[1] = v.y;
  }
}

// PG (paged pool): p is the logical page, b its pool block; the codes of row
// l/4 are row l/4 of page-head block (b, g), and kr / vr hold the page-head's
// outlier count and index (count, b * H + g) instead of row_ptr entries.
template <int KB, int VB, bool PG>
HKV_DEV void load_page(const DecodeArgs& A, int p, int b, int g, int lane, PageLoad<KB, VB>& L) {
  const int row = lane >> 2, q = lane & 3;
  const int t = p < 0 ? 0 : p * kPS + row;
  if constexpr (PG) {
    const int ph = p < 0 ? 0 : b * A.H + g;
    const int r = ph * kPS + row;
    L.kr = make_int2(A.k.ocnt[ph], ph);
    L.vr = make_int2(A.v.ocnt[ph], ph);
    load_codes<KB>(A.k.packed, r, q, L.kc);
    load_codes<VB>(A.v.packed, r, q, L.vc);
  } else {
    const int tc = t < (int)A.T ? t : 0;
    const int r = tc * A.H + g;
    L.kr = *reinterpret_cast<const int2*>(A.k.row_ptr + (uint32_t)r);
    L.vr = *reinterpret_cast<const int2*>(A.v.row_ptr + (uint32_t)r);
    load_codes<KB>(A.k.packed, r, q, L.kc);
    load_codes<VB>(A.v.packed, r, q, L.vc);
  }
  const int vrow = t < (int)A.v.rows ? t : (int)A.v.rows - 1;
  // nuq4: levels 4q..4q+3 of the row; nuq2: its 4 levels, in every lane
  L.vtab = *reinterpret_cast<const uint2*>(A.v.tabs[(uint32_t)(g * (int)A.v.rows + vrow)].pf16 +
                                           (VB == 2 ? 0 : 4 * q));
}

HKV_DEV int csr_slot(int a, int sub, int s, int cap) {
  const int i = (a < 0 ? 0 : a) + sub + 4 * s;
  return i < cap ? i : cap - 1;
}

// PG: lane l holds entries l + 64 s (s < kSlots) of the page-head in
// kval[s] / vval[s], the index clamped to the page-head's last entry (or 0):
// the loads stay unconditional, and those past the count read a line
// already fetched, so only the entries' own lines come from HBM.
template <int KB, int VB, bool PG>
HKV_DEV void load_outl(const DecodeArgs& A, const PageLoad<KB, VB>& L, int lane, PageOutl& O) {
  const int kcap = (int)A.k.cap, vcap = (int)A.v.cap;
  if constexpr (PG) {
    const int kl = (L.kr.x < kcap ? L.kr.x : kcap) - 1, vl = (L.vr.x < vcap ? L.vr.x : vcap) - 1;
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      const int i = lane + 64 * s;
      if (kcap > 0) O.kval[s] = A.k.oent[(int64_t)L.kr.y * kcap + (i < kl ? i : (kl > 0 ? kl : 0))];
      if (vcap > 0) O.vval[s] = A.v.oent[(int64_t)L.vr.y * vcap + (i < vl ? i : (vl > 0 ? vl : 0))];
    }
    return;
  }
  const int sub = lane & 3;
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    if (kcap > 0) {
      const uint32_t i = (uint32_t)csr_slot(L.kr.x, sub, s, kcap);
      O.kval[s] = A.k.val[i];
      O.kcol[s] = A.k.col[i];
    }
    if (vcap > 0) {
      const uint32_t i = (uint32_t)csr_slot(L.vr.x, sub, s, vcap);
      O.vval[s] = A.v.val[i];
      O.vcol[s] = A.v.col[i];
    }
  }
}

// Dequantise the lane's 32 codes into tile row l/4, channels [32(l%4), +32).
// FULL: every row of the page is a token of the context (no masking).
template <int NB, bool FULL, typename Lut>
HKV_DEV void dequant_rows(const uint32_t (&w)[NB], bool valid, int lane, uint16_t* tile, Lut lut) {
  const int row = lane >> 2, c0 = 32 * (lane & 3);
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // 8 channels per 128-bit LDS store
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t pr = 0;
#pragma unroll
      for (int e2 = 0; e2 < 2; ++e2) {
        const int e = 8 * k + 2 * j + e2;  // channel c0 + e
        uint32_t code;
        if constexpr (NB == 4) code = (w[e >> 3] >> (4 * (e & 7))) & 15u;
        else code = (w[e >> 4] >> (2 * (e & 15))) & 3u;
        pr |= (uint32_t)lut(c0 + e, code) << (16 * e2);
      }
      h[j] = (FULL || valid) ? pr : 0u;  // rows past the context read as zeros
    }
    *reinterpret_cast<uint4*>(tile + row * kTS + c0 + 8 * k) = make_uint4(h[0], h[1], h[2], h[3]);
  }
}

// nuq2 through a pair table: the lane's 16 pairs (channels [32(l%4), +32) of
// row l/4) read lut[pstride * k + x] for pair k with code bits x.
template <int PSTRIDE>
HKV_DEV void dequant_pairs(const uint32_t (&w)[2], bool valid, int lane, uint16_t* tile,
                           const uint32_t* lut) {
  const int row = lane >> 2, c0 = 32 * (lane & 3);
#pragma unroll
  for (int k4 = 0; k4 < 4; ++k4) {  // 8 channels per 128-bit LDS store
    uint32_t h[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = 4 * k4 + j;
      const uint32_t x = (w[k >> 3] >> (4 * (k & 7))) & 15u;
      const uint32_t v = lut[PSTRIDE * k + (int)x];
      h[j] = valid ? v : 0u;  // rows past the context read as zeros
    }
    *reinterpret_cast<uint4*>(tile + row * kTS + c0 + 8 * k4) = make_uint4(h[0], h[1], h[2], h[3]);
  }
}

// CSR entries beyond the kSlots held in registers (rows with > 4*kSlots
// outliers): read directly.
HKV_DEV void patch_rest(const Side& sd, int2 rb, int lane, uint16_t* tile) {
  const int row = lane >> 2;
  int64_t i = (int64_t)(rb.x < 0 ? 0 : rb.x) + 4 * kSlots + (lane & 3);
  const int64_t e = rb.y < sd.cap ? rb.y : sd.cap;
  for (; i < e; i += 4) {
    const uint32_t d = sd.col[i];
    if (d < (uint32_t)kHD) tile[row * kTS + d] = sd.val[i];
  }
}

// Page-head entries past those held in registers (PG): the inline ones from
// index 64 * kSlots, then those of the page-head's overflow chunk.
HKV_DEV void patch_rest_paged(const Side& sd, int2 cr, int lane, uint16_t* tile, int64_t t0, int64_t T) {
  const int cap = (int)sd.cap;
  const int ov = (cr.x > cap && sd.ovf) ? sd.ovf[cr.y] : -1;
  const int room = cap + (ov >= 0 ? kPS * kHD - cap : 0);
  const int n = cr.x < room ? cr.x : room;
  const int first = cap < 64 * kSlots ? cap : 64 * kSlots;
  for (int i = first + lane; i < n; i += 64) {
    const uint32_t e = i < cap ? sd.oent[(int64_t)cr.y * cap + i]
                               : sd.ovf_ent[(int64_t)ov * (kPS * kHD - cap) + (i - cap)];
    const uint32_t slot = e >> 24, ch = (e >> 16) & 255u;
    if (slot < (uint32_t)kPS && t0 + (int64_t)slot < T && ch < (uint32_t)kHD) tile[slot * kTS + ch] = (uint16_t)e;
  }
}

// One block: split `split` of the selection (pages split * pps ..) for KV
// head blockIdx.y.
template <int KB, int VB, bool PG>
HKV_DEV void decode_body(const DecodeArgs& A, int64_t split) {
  // K: the nuq4 table (halves) or the nuq2 pair table (words); V: the wave's
  // page, [row][level] halves (nuq4) or [row][pair entry] words (nuq2)
  __shared__ __align__(16) uint32_t s_klut_w[kKLutWords];
  __shared__ __align__(16) uint32_t s_vlut_w[kW][kPS * 16];
  uint16_t* s_klut = reinterpret_cast<uint16_t*>(s_klut_w);
  __shared__ __align__(16) uint16_t s_tiles[kW][2][kPS * kTS];
  __shared__ float s_m[kW][16], s_l[kW][16];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = blockIdx.y, H = A.H, group = A.group;
  const int64_t j0 = split * A.pps;
  const int64_t j1 = j0 + A.pps < A.nsel ? j0 + A.pps : A.nsel;

  if constexpr (KB == 2) {
    for (int i = tid; i < 64 * 16; i += kDT) {
      const int pp = i >> 4, x = i & 15;
      const uint32_t lo = A.k.tabs[(int64_t)g * kHD + 2 * pp].pf16[x & 3];
      const uint32_t hi = A.k.tabs[(int64_t)g * kHD + 2 * pp + 1].pf16[x >> 2];
      s_klut_w[kpair_index(pp, x)] = lo | hi << 16;
    }
  } else {
    for (int i = tid; i < kHD * 16; i += kDT) {
      const int d = i >> 4, l = i & 15;
      s_klut[klut_index(d, l)] = A.k.tabs[(int64_t)g * kHD + d].pf16[l];
    }
  }

  // the wave's page ids, one per lane (-1: none / out of range)
  const int64_t nw64 = j1 - j0 > wv ? (j1 - j0 - wv + kW - 1) / kW : 0;
  const int nslots = (int)nw64;  // <= kMaxPPS / kW = 64
  int my_p = -1, my_b = 0;  // logical page and (PG) its pool block
  if (lane < nslots) {
    const int64_t s = A.sel[(j0 + wv + (int64_t)kW * lane) * H + g];
    my_p = (s >= 0 && s < A.npages) ? (int)s : -1;
    if constexpr (PG) {
      if (my_p >= 0) {
        const int64_t b = A.bt[my_p];
        if (b >= 0 && b < A.nblocks) my_b = (int)b;
        else my_p = -1;  // a page without a block is skipped
      }
    }
  }
  // Only valid ids are visited: they move, in order, to the wave's first nw
  // lanes (one ds_permute over a permutation of the 64 lanes: the invalid
  // ids go to the lanes after them).  A selection with holes (the union of
  // the heads' pages written with -1 in place of the pages left out) then
  // costs no pipeline steps for its holes.
  const uint64_t vm = __builtin_amdgcn_ballot_w64(my_p >= 0);
  const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(vm >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)vm, 0u));
  const int nw = __builtin_popcountll(vm);
  const int dst = (my_p >= 0 ? below : nw + (lane - below)) << 2;
  my_p = __builtin_amdgcn_ds_permute(dst, my_p);
  if constexpr (PG) my_b = __builtin_amdgcn_ds_permute(dst, my_b);
  auto page_at = [&](int i) -> int { return i < nw ? __builtin_amdgcn_readlane(my_p, i) : -1; };
  auto block_at = [&](int i) -> int { return PG && i < nw ? __builtin_amdgcn_readlane(my_b, i) : 0; };

  // B operand of S^T = K Q^T: lane l holds q[qh = l%16][16i + 4(l/16) .. +3]
  const int qh = lane & 15, kg = lane >> 4;
  half4_t qb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (qh < group) {
      const uint2 v = *reinterpret_cast<const uint2*>(
          A.q + (int64_t)(g * group + qh) * kHD + 16 * i + 4 * kg);
      qb[i] = __builtin_bit_cast(half4_t, v);
    } else {
      qb[i] = (half4_t){0, 0, 0, 0};
    }
  }
  float4_t o[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) o[t] = (float4_t){0.f, 0.f, 0.f, 0.f};
  float m = -__builtin_inff(), lsum = 0.0f;
  const float sl2 = A.scale * kLog2e;
  __syncthreads();  // K LUT

  uint16_t* kt = s_tiles[wv][0];
  uint16_t* vt = s_tiles[wv][1];
  uint16_t* vl = reinterpret_cast<uint16_t*>(s_vlut_w[wv]);
  uint32_t* vlw = s_vlut_w[wv];

  auto compute = [&](const PageLoad<KB, VB>& L, const PageOutl& Ob, int p) {
    const int64_t t0 = (int64_t)p * kPS;
    const int row = lane >> 2;
    const bool valid = t0 + row < A.T;
    const int q = lane & 3;
    if constexpr (VB == 2) {
      // the row's pair entries 4q .. 4q + 3 (c1 = q): pole(c0) | pole(q) << 16
      const uint32_t p01 = L.vtab.x, p23 = L.vtab.y;
      const uint32_t pq = ((q < 2 ? p01 : p23) >> (16 * (q & 1))) << 16;
      *reinterpret_cast<uint4*>(vlw + row * 16 + 4 * q) =
          make_uint4((p01 & 0xffffu) | pq, (p01 >> 16) | pq, (p23 & 0xffffu) | pq, (p23 >> 16) | pq);
    } else {
      *reinterpret_cast<uint2*>(vl + row * 16 + 4 * q) = L.vtab;
    }
    wave_sync();
    if constexpr (KB == 2) {
      dequant_pairs<16>(L.kc, valid, lane, kt, s_klut_w + kpair_index(16 * q, 0));
    } else {
      dequant_rows<KB, false>(L.kc, valid, lane, kt,
                              [&](int ch, uint32_t c) { return s_klut[klut_index(ch, (int)c)]; });
    }
    if constexpr (VB == 2) {
      dequant_pairs<0>(L.vc, valid, lane, vt, vlw + row * 16);
    } else {
      dequant_rows<VB, false>(L.vc, valid, lane, vt, [&](int, uint32_t c) { return vl[row * 16 + (int)c]; });
    }
    wave_sync();
    if constexpr (PG) {
      // the page-head's entries (rows past the context are masked below)
      // the counts are the same in every lane: slots past them are skipped
      const int kn = __builtin_amdgcn_readfirstlane(L.kr.x < (int)A.k.cap ? L.kr.x : (int)A.k.cap);
      const int vn = __builtin_amdgcn_readfirstlane(L.vr.x < (int)A.v.cap ? L.vr.x : (int)A.v.cap);
#pragma unroll
      for (int s = 0; s < kSlots; ++s) {
        if (64 * s >= (kn > vn ? kn : vn)) break;
        const int i = lane + 64 * s;
        if (i < kn) {
          const uint32_t e = Ob.kval[s], sl = e >> 24, ch = (e >> 16) & 255u;
          if (sl < (uint32_t)kPS && t0 + (int64_t)sl < A.T && ch < (uint32_t)kHD) kt[sl * kTS + ch] = (uint16_t)e;
        }
        if (i < vn) {
          const uint32_t e = Ob.vval[s], sl = e >> 24, ch = (e >> 16) & 255u;
          if (sl < (uint32_t)kPS && t0 + (int64_t)sl < A.T && ch < (uint32_t)kHD) vt[sl * kTS + ch] = (uint16_t)e;
        }
      }
      // past the registers: more inline entries, or an overflow chunk
      if (L.kr.x > (kn < 64 * kSlots ? kn : 64 * kSlots)) patch_rest_paged(A.k, L.kr, lane, kt, t0, A.T);
      if (L.vr.x > (vn < 64 * kSlots ? vn : 64 * kSlots)) patch_rest_paged(A.v, L.vr, lane, vt, t0, A.T);
    } else if (valid) {
      const int sub = lane & 3;
      const int ka = L.kr.x < 0 ? 0 : L.kr.x, va = L.vr.x < 0 ? 0 : L.vr.x;
      const int ke = L.kr.y < (int)A.k.cap ? L.kr.y : (int)A.k.cap;
      const int ve = L.vr.y < (int)A.v.cap ? L.vr.y : (int)A.v.cap;
#pragma unroll
      for (int s = 0; s < kSlots; ++s) {
        if (ka + sub + 4 * s < ke && Ob.kcol[s] < (uint32_t)kHD)
          kt[row * kTS + Ob.kcol[s]] = (uint16_t)Ob.kval[s];
        if (va + sub + 4 * s < ve && Ob.vcol[s] < (uint32_t)kHD)
          vt[row * kTS + Ob.vcol[s]] = (uint16_t)Ob.vval[s];
      }
      if (ke - ka > 4 * kSlots) patch_rest(A.k, L.kr, lane, kt);
      if (ve - va > 4 * kSlots) patch_rest(A.v, L.vr, lane, vt);
    }
    wave_sync();

    // S^T (16 keys x 16 query heads)
    float4_t s = (float4_t){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const half4_t a = __builtin_bit_cast(
          half4_t, *reinterpret_cast<const uint2*>(kt + qh * kTS + 16 * i + 4 * kg));
      s = __builtin_amdgcn_mfma_f32_16x16x16f16(a, qb[i], s, 0, 0, 0);
    }
    // lane holds keys 4*kg + r of query head qh
    float x[4];
    float mp = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = t0 + 4 * kg + r < A.T;
      x[r] = ok ? s[r] * sl2 : -__builtin_inff();
      mp = x[r] > mp ? x[r] : mp;
    }
    mp = fmaxf(mp, __shfl_xor(mp, 16, 64));
    mp = fmaxf(mp, __shfl_xor(mp, 32, 64));
    const float mn = fmaxf(m, mp);  // finite: a valid page holds a token < T
    const float alpha = exp2f(m - mn);
    m = mn;
    half4_t pb;
    float ps = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float e = exp2f(x[r] - mn);
      ps += e;
      pb[r] = (_Float16)e;
    }
    lsum = lsum * alpha + ps;
#pragma unroll
    for (int t = 0; t < 8; ++t) o[t] *= alpha;
    // O^T (128 ch x 16 heads) += V^T P^T: A[ch][key] = vt[key][ch]
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      half4_t a;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        a[r] = __builtin_bit_cast(_Float16, vt[(4 * kg + r) * kTS + 16 * t + qh]);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb, o[t], 0, 0, 0);
    }
    wave_sync();  // the tiles and the V LUT are rewritten by the next page
  };

  // three-stage pipeline over the wave's pages, unrolled by 3 so that every
  // in-flight load keeps its registers (no copies of pending loads)
  PageLoad<KB, VB> L0, L1, L2;
  PageOutl O0, O1, O2;
  load_page<KB, VB, PG>(A, page_at(0), block_at(0), g, lane, L0);
  load_page<KB, VB, PG>(A, page_at(1), block_at(1), g, lane, L1);
  load_outl<KB, VB, PG>(A, L0, lane, O0);
  auto step = [&](int i, const PageLoad<KB, VB>& Lc, const PageOutl& Oc, const PageLoad<KB, VB>& Ln,
                  PageOutl& On, PageLoad<KB, VB>& Lw) {
    load_page<KB, VB, PG>(A, page_at(i + 2), block_at(i + 2), g, lane, Lw);
    if (i + 1 < nw) load_outl<KB, VB, PG>(A, Ln, lane, On);
    const int p = page_at(i);
    if (p >= 0) compute(Lc, Oc, p);
  };
  for (int i = 0; i < nw; i += 3) {
    step(i, L0, O0, L1, O1, L2);
    if (i + 1 >= nw) break;
    step(i + 1, L1, O1, L2, O2, L0);
    if (i + 2 >= nw) break;
    step(i + 2, L2, O2, L0, O0, L1);
  }

  // wave partials: m (replicated over the 4 lane groups), l summed over them
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  __syncthreads();
  float* s_o = reinterpret_cast<float*>(&s_tiles[0][0][0]);  // [kW][16][kHD]
  if (kg == 0) { s_m[wv][qh] = m; s_l[wv][qh] = lsum; }
  // O^T tile t: lane holds channel 16t + 4kg + r of head qh
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) s_o[(wv * 16 + qh) * kHD + 16 * t + 4 * kg + r] = o[t][r];
  __syncthreads();
  const int Hq = H * group;
  for (int i = tid; i < group * kHD; i += kDT) {
    const int hh = i / kHD, d = i % kHD;
    float M = -__builtin_inff();
    for (int w = 0; w < kW; ++w) M = fmaxf(M, s_m[w][hh]);
    float acc = 0.0f, L = 0.0f;
    if (M != -__builtin_inff()) {
      for (int w = 0; w < kW; ++w) {
        const float f = exp2f(s_m[w][hh] - M);
        acc += f * s_o[(w * 16 + hh) * kHD + d];
        L += f * s_l[w][hh];
      }
    }
    const int64_t hq = (int64_t)g * group + hh;
    A.part_o[(split * Hq + hq) * kHD + d] = acc;
    if (d == 0) {
      A.part_m[split * Hq + hq] = M;
      A.part_l[split * Hq + hq] = L;
    }
  }
}

template <int KB, int VB, bool PG>
__global__ void __launch_bounds__(kDT) __attribute__((amdgpu_waves_per_eu(3, 3)))
decode_kernel(DecodeArgs A) {
  decode_body<KB, VB, PG>(A, blockIdx.x);
}

// Batched form: B sequences of one compact-format tensor (or of one paged
// pool), each with its own query, length, selection rows and splits.
// Sequence b owns the kernel's blocks [split0[b], split0[b+1]); base[b] is
// its first token in the compact tensor (a multiple of 16) or its first
// block-table entry in the paged form.
constexpr int kMaxDecSeqs = 64;
struct DecSegs {
  int64_t split0[kMaxDecSeqs + 1];
  int64_t base[kMaxDecSeqs];
  int64_t T[kMaxDecSeqs];
  int64_t sel0[kMaxDecSeqs];
  int64_t nsel[kMaxDecSeqs];
  int nseg;
};

template <int KB, int VB, bool PG>
__global__ void __launch_bounds__(kDT) __attribute__((amdgpu_waves_per_eu(3, 3)))
decode_batch_kernel(DecodeArgs A, DecSegs S) {
  int b = 0;
  while (b + 1 < S.nseg && S.split0[b + 1] <= (int64_t)blockIdx.x) ++b;
  // the sequence's view: its query, tokens, selection and partials
  DecodeArgs a = A;
  const int Hq = A.H * A.group;
  a.q = A.q + (int64_t)b * Hq * kHD;
  a.T = S.T[b];
  a.npages = (S.T[b] + kPS - 1) / kPS;
  a.sel = A.sel + S.sel0[b] * A.H;
  a.nsel = S.nsel[b];
  if constexpr (PG) {
    a.bt = A.bt + S.base[b];
  } else {
    const int64_t r0 = S.base[b] * A.H;  // first row of the sequence
    a.k.packed = A.k.packed + r0 * (kHD * KB / 8);
    a.k.row_ptr = A.k.row_ptr + r0;
    a.v.packed = A.v.packed + r0 * (kHD * VB / 8);
    a.v.row_ptr = A.v.row_ptr + r0;
  }
  a.part_m = A.part_m + S.split0[b] * Hq;
  a.part_l = A.part_l + S.split0[b] * Hq;
  a.part_o = A.part_o + S.split0[b] * Hq * kHD;
  decode_body<KB, VB, PG>(a, (int64_t)blockIdx.x - S.split0[b]);
}

// Union of the heads' selected pages per sequence (the reference's decode
// attends every query head over it: src/kvquant/quest_selector.py:80, then
// all heads of each kept block, src/kvquant/compact_pool.py:492-537).
// Sequence b's selection is rows row0[b] .. row0[b+1]-1 of sel (rows, H),
// page ids local to the sequence; its union goes to rows page0[b] .. of out
// (all H columns), ascending, -1 after it.  Three launches over the whole
// batch: mark (a flag byte per selected page), count (set flags per chunk of
// kUnionChunk pages), write (each chunk's pages at the offset its sequence's
// earlier chunks give, through LDS so the rows are written coalesced; the
// chunk's rows past the union get -1; the flags are cleared).  The flags
// (one byte per page of all sequences) are zero on entry and left zero.
constexpr int kUnionThreads = 256;
constexpr int kUnionPer = 8;                                 // pages per thread
constexpr int kUnionChunk = kUnionThreads * kUnionPer;       // pages per block
struct UnionSegs {
  int64_t row0[kMaxDecSeqs + 1];
  int64_t page0[kMaxDecSeqs + 1];
  int64_t chunk0[kMaxDecSeqs + 1];  // sequence b's chunks are chunk0[b] .. chunk0[b+1]-1
  int nseg;
};

__global__ void __launch_bounds__(256)
union_mark_kernel(const int64_t* __restrict__ sel, int H, UnionSegs S, uint8_t* __restrict__ flags) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= S.row0[S.nseg] * H) return;
  const int64_t r = i / H;
  int b = 0;
  while (b + 1 < S.nseg && S.row0[b + 1] <= r) ++b;
  const int64_t p = sel[i], P = S.page0[b + 1] - S.page0[b];
  if (p >= 0 && p < P) flags[S.page0[b] + p] = 1;
}

// Block = chunk c of sequence b: its pages [q0, q1) of the sequence and the
// thread's flag mask (page q0 + kUnionPer * tid + i at bit i).
struct UnionChunk {
  int b;
  int64_t p0, P, q0, q1;
};
HKV_DEV UnionChunk union_chunk(const UnionSegs& S) {
  UnionChunk u;
  u.b = 0;
  while (u.b + 1 < S.nseg && S.chunk0[u.b + 1] <= (int64_t)blockIdx.x) ++u.b;
  u.p0 = S.page0[u.b];
  u.P = S.page0[u.b + 1] - u.p0;
  u.q0 = ((int64_t)blockIdx.x - S.chunk0[u.b]) * kUnionChunk;
  u.q1 = u.q0 + kUnionChunk < u.P ? u.q0 + kUnionChunk : u.P;
  return u;
}
HKV_DEV uint32_t union_mask(const uint8_t* flags, const UnionChunk& u) {
  const int64_t t0 = u.q0 + (int64_t)kUnionPer * threadIdx.x;
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < kUnionPer; ++i)
    if (t0 + i < u.q1 && flags[u.p0 + t0 + i]) m |= 1u << i;
  return m;
}
HKV_DEV uint32_t union_block_sum(uint32_t v, uint32_t* red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  __syncthreads();
  if (lane == 0) red[wv] = v;
  __syncthreads();
  uint32_t t = 0;
  for (int w = 0; w < kUnionThreads / 64; ++w) t += red[w];
  return t;
}

__global__ void __launch_bounds__(kUnionThreads)
union_count_kernel(const uint8_t* __restrict__ flags, UnionSegs S, uint32_t* __restrict__ cnt) {
  __shared__ uint32_t red[kUnionThreads / 64];
  const UnionChunk u = union_chunk(S);
  const uint32_t t = union_block_sum((uint32_t)__builtin_popcount(union_mask(flags, u)), red);
  if (threadIdx.x == 0) cnt[blockIdx.x] = t;
}

__global__ void __launch_bounds__(kUnionThreads)
union_write_kernel(uint8_t* __restrict__ flags, UnionSegs S, const uint32_t* __restrict__ cnt, int H,
                   int64_t* __restrict__ out) {
  __shared__ uint32_t red[kUnionThreads / 64];
  __shared__ uint32_t lst[kUnionChunk];  // the chunk's union pages, in order
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const UnionChunk u = union_chunk(S);
  // pages of the sequence's earlier chunks, and of all its chunks
  const int64_t c0 = S.chunk0[u.b], c = (int64_t)blockIdx.x;
  uint32_t before = 0, all = 0;
  for (int64_t i = c0 + tid; i < S.chunk0[u.b + 1]; i += kUnionThreads) {
    before += i < c ? cnt[i] : 0u;
    all += cnt[i];
  }
  before = union_block_sum(before, red);
  all = union_block_sum(all, red);
  // the chunk's pages in order: exclusive scan of the threads' counts
  const uint32_t m = union_mask(flags, u);
  const uint32_t k = (uint32_t)__builtin_popcount(m);
  uint32_t x = k;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  __syncthreads();
  if (lane == 63) red[wv] = x;
  __syncthreads();
  uint32_t pre = x - k, tot = 0;
  for (int w = 0; w < kUnionThreads / 64; ++w) {
    pre += w < wv ? red[w] : 0u;
    tot += red[w];
  }
  const int64_t t0 = u.q0 + (int64_t)kUnionPer * tid;
#pragma unroll
  for (int i = 0; i < kUnionPer; ++i) {
    if ((m >> i) & 1u) {
      lst[pre++] = (uint32_t)(t0 + i);
      flags[u.p0 + t0 + i] = 0;
    }
  }
  __syncthreads();
  // rows before + j of the sequence, every column, written consecutively
  int64_t* o = out + (u.p0 + (int64_t)before) * H;
  for (int64_t e = tid; e < (int64_t)tot * H; e += kUnionThreads) o[e] = (int64_t)lst[e / H];
  // this chunk's share of the rows after the union: [q0, q1) past `all`
  const int64_t r0 = u.q0 > (int64_t)all ? u.q0 : (int64_t)all;
  for (int64_t e = r0 * H + tid; e < u.q1 * H; e += kUnionThreads) out[u.p0 * H + e] = -1;
}

// ------------------------------------------------ dense pages (any dtype)

constexpr int kDenseKeys = 1024;  // keys per split of the dense kernel
constexpr int kDenseMaxD = 512;

struct DenseArgs {
  const void* q;       // (Hq, D)
  const void* k;       // (P, S, Hk, D)
  const void* v;       // (P, S, Hv, Dv)
  int q_dt, kv_dt;
  int64_t P;
  int S, Hk, Hv, D, Dv, Hq, head_map;  // head_map 0: K head h, V head h % Hv; 1: h / (Hq/Hk)
  const int64_t* sel;  // (nsel, ncols)
  int64_t nsel;
  int ncols;           // Hq (column per query head) or Hk (column per KV head)
  int pps;
  float scale;
  float *part_m, *part_l, *part_o;
};

__global__ void __launch_bounds__(kDT)
dense_attn_kernel(DenseArgs A) {
  __shared__ float s_q[kDenseMaxD];
  __shared__ float s_s[kDenseKeys];
  __shared__ float s_red[kW];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int h = blockIdx.y;
  const int kh = A.head_map == 0 ? h : h / (A.Hq / A.Hk);
  const int vh = A.head_map == 0 ? h % A.Hv : kh;
  const int col = A.ncols == A.Hq ? h : kh;
  const int64_t j0 = (int64_t)blockIdx.x * A.pps;
  const int64_t j1 = j0 + A.pps < A.nsel ? j0 + A.pps : A.nsel;
  const int nk = (int)(j1 - j0) * A.S;  // <= kDenseKeys
  for (int d = tid; d < A.D; d += kDT) s_q[d] = load_scale(A.q, A.q_dt, (int64_t)h * A.D + d);
  __syncthreads();
  // scores: one wave per key, lanes over channels
  const float sl2 = A.scale * kLog2e;
  for (int kk = wv; kk < nk; kk += kW) {
    const int64_t p = A.sel[(j0 + kk / A.S) * A.ncols + col];
    float sc = -__builtin_inff();
    if (p >= 0 && p < A.P) {  // uniform per wave
      const int64_t base = ((p * A.S + kk % A.S) * A.Hk + kh) * A.D;
      float acc = 0.0f;
      for (int d = lane; d < A.D; d += 64) acc += s_q[d] * load_scale(A.k, A.kv_dt, base + d);
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
      sc = acc * sl2;
    }
    if (lane == 0) s_s[kk] = sc;
  }
  __syncthreads();
  float mx = -__builtin_inff();
  for (int kk = tid; kk < nk; kk += kDT) mx = fmaxf(mx, s_s[kk]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) s_red[wv] = mx;
  __syncthreads();
  float M = s_red[0];
  for (int w = 1; w < kW; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();
  float ls = 0.0f;
  for (int kk = tid; kk < nk; kk += kDT) {
    const float e = M == -__builtin_inff() ? 0.0f : exp2f(s_s[kk] - M);
    s_s[kk] = e;
    ls += e;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ls += __shfl_xor(ls, off, 64);
  if (lane == 0) s_red[wv] = ls;
  __syncthreads();
  float L = 0.0f;
  for (int w = 0; w < kW; ++w) L += s_red[w];
  for (int d = tid; d < A.Dv; d += kDT) {
    float acc = 0.0f;
    for (int kk = 0; kk < nk; ++kk) {
      const float pk = s_s[kk];
      if (pk == 0.0f) continue;
      const int64_t p = A.sel[(j0 + kk / A.S) * A.ncols + col];
      const int64_t base = ((p * A.S + kk % A.S) * A.Hv + vh) * A.Dv;
      acc += pk * load_scale(A.v, A.kv_dt, base + d);
    }
    A.part_o[((int64_t)blockIdx.x * A.Hq + h) * A.Dv + d] = acc;
  }
  if (tid == 0) {
    A.part_m[(int64_t)blockIdx.x * A.Hq + h] = M;
    A.part_l[(int64_t)blockIdx.x * A.Hq + h] = L;
  }
}

// ------------------------------------------------------------------ merge

// Block (query head, 16-channel slice); thread (d, sub) sums the splits
// s = sub (mod 16) of channel d, then the 16 partial sums are added in LDS.
// Every block first reduces M = max_s m_s and L = sum_s 2^(m_s - M) l_s.
constexpr int kMergeCh = 16;
constexpr int kMergeSub = kDT / kMergeCh;

HKV_DEV void merge_body(const float* __restrict__ pm, const float* __restrict__ pl,
                       const float* __restrict__ po, int64_t splits, int Hq, int Dv, void* out, int odt) {
  __shared__ float s_red[kW];
  __shared__ float s_acc[kDT];
  const int hq = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int d = blockIdx.y * kMergeCh + (tid % kMergeCh), sub = tid / kMergeCh;
  // Up to kMergeRegs splits a thread: their partial outputs and maxima are
  // requested first (clamped indexes, unconditional), so the max and sum
  // passes below overlap them instead of following them.
  constexpr int kMergeRegs = 16;
  const bool in_regs = splits <= (int64_t)kMergeRegs * kMergeSub;
  const int dc = d < Dv ? d : Dv - 1;
  float pov[kMergeRegs], pmv[kMergeRegs];
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < kMergeRegs; ++i) {
      int64_t s = sub + (int64_t)i * kMergeSub;
      s = s < splits ? s : splits - 1;
      pmv[i] = pm[s * Hq + hq];
      pov[i] = po[(s * Hq + hq) * Dv + dc];
    }
  }
  float mx = -__builtin_inff();
  for (int64_t s = tid; s < splits; s += kDT) mx = fmaxf(mx, pm[s * Hq + hq]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  if (lane == 0) s_red[wv] = mx;
  __syncthreads();
  float M = s_red[0];
  for (int w = 1; w < kW; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();
  float ls = 0.0f;
  if (M != -__builtin_inff())
    for (int64_t s = tid; s < splits; s += kDT) {
      const float ms = pm[s * Hq + hq];
      if (ms != -__builtin_inff()) ls += exp2f(ms - M) * pl[s * Hq + hq];
    }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ls += __shfl_xor(ls, off, 64);
  if (lane == 0) s_red[wv] = ls;
  __syncthreads();
  float L = 0.0f;
  for (int w = 0; w < kW; ++w) L += s_red[w];
  float acc = 0.0f;
  if (in_regs) {
    if (d < Dv && M != -__builtin_inff()) {
#pragma unroll
      for (int i = 0; i < kMergeRegs; ++i) {
        if (sub + (int64_t)i * kMergeSub < splits) {
          const float w = pmv[i] == -__builtin_inff() ? 0.0f : exp2f(pmv[i] - M);
          acc += w * pov[i];
        }
      }
    }
  } else if (d < Dv && M != -__builtin_inff()) {
#pragma unroll 4
    for (int64_t s = sub; s < splits; s += kMergeSub) {
      const float ms = pm[s * Hq + hq];
      const float w = ms == -__builtin_inff() ? 0.0f : exp2f(ms - M);
      acc += w * po[(s * Hq + hq) * Dv + d];
    }
  }
  s_acc[tid] = acc;
  __syncthreads();
  if (sub == 0 && d < Dv) {
    float a = 0.0f;
    for (int u = 0; u < kMergeSub; ++u) a += s_acc[tid + u * kMergeCh];
    const float r = L > 0.0f ? a / L : 0.0f;
    if (odt == HKV_DT_F32) ((float*)out)[(int64_t)hq * Dv + d] = r;
    else if (odt == HKV_DT_BF16) {
      const uint32_t b = __builtin_bit_cast(uint32_t, r);
      const uint32_t rb = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;  // nearest even
      ((uint16_t*)out)[(int64_t)hq * Dv + d] = (r != r) ? (uint16_t)0x7fc0u : (uint16_t)rb;
    } else ((uint16_t*)out)[(int64_t)hq * Dv + d] = f2h(r);
  }
}

__global__ void __launch_bounds__(kDT)
merge_kernel(const float* __restrict__ pm, const float* __restrict__ pl,
             const float* __restrict__ po, int64_t splits, int Hq, int Dv, void* out, int odt) {
  merge_body(pm, pl, po, splits, Hq, Dv, out, odt);
}

// Batched: blockIdx.z = sequence b merges its splits [split0[b], split0[b+1])
// into out + b * Hq * Dv.
struct MergeSegs {
  int64_t split0[kMaxDecSeqs + 1];
};

__global__ void __launch_bounds__(kDT)
merge_batch_kernel(const float* __restrict__ pm, const float* __restrict__ pl,
                   const float* __restrict__ po, MergeSegs S, int Hq, int Dv, void* out, int odt) {
  const int b = blockIdx.z;
  const int64_t s0 = S.split0[b];
  const size_t esz = odt == HKV_DT_F32 ? 4 : 2;
  merge_body(pm + s0 * Hq, pl + s0 * Hq, po + s0 * Hq * Dv, S.split0[b + 1] - s0, Hq, Dv,
             static_cast<char*>(out) + (size_t)b * Hq * Dv * esz, odt);
}

void launch_merge(const float* pm, const float* pl, const float* po, int64_t splits, int Hq, int Dv,
                  void* out, int odt, hipStream_t s) {
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)Hq, (unsigned)((Dv + kMergeCh - 1) / kMergeCh)),
                     dim3(kDT), 0, s, pm, pl, po, splits, Hq, Dv, out, odt);
}

int64_t n_splits(int64_t nsel, int pps) { return nsel == 0 ? 1 : (nsel + pps - 1) / pps; }

template <int KB, int VB, bool PG = false>
void launch_decode(const DecodeArgs& a, int64_t splits, hipStream_t s) {
  hipLaunchKernelGGL((decode_kernel<KB, VB, PG>), dim3((unsigned)splits, (unsigned)a.H), dim3(kDT),
                     0, s, a);
}

template <int KB, int VB, bool PG = false>
void launch_decode_batch(const DecodeArgs& a, const DecSegs& sg, hipStream_t s) {
  hipLaunchKernelGGL((decode_batch_kernel<KB, VB, PG>), dim3((unsigned)sg.split0[sg.nseg], (unsigned)a.H),
                     dim3(kDT), 0, s, a, sg);
}

}  // namespace

extern "C" int hkv_paged_decode_attn(const void* q, int Hq, int64_t T, const int64_t* block_table,
                                     const hkv_paged_side* ks, const void* k_tables,
                                     const hkv_paged_side* vs, const void* v_tables, int64_t v_rows,
                                     const int64_t* sel, int64_t nsel, int pages_per_split,
                                     float scale, void* out, int out_dtype, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (!ks || !vs) return HKV_ERR_ARG;
  const int H = ks->heads;
  const int64_t num_blocks = ks->num_blocks;
  const int k_bits = ks->bits, v_bits = vs->bits, k_cap = ks->cap, v_cap = vs->cap;
  if (vs->heads != H || vs->num_blocks != num_blocks) return HKV_ERR_SHAPE;
  if (H < 1 || H > 16 || Hq < H || Hq % H || Hq / H > 16 || T < 1 || nsel < 0 || num_blocks < 1)
    return HKV_ERR_SHAPE;
  if (pages_per_split < 1 || pages_per_split > kMaxPPS) return HKV_ERR_ARG;
  if ((k_bits != 2 && k_bits != 4) || (v_bits != 2 && v_bits != 4)) return HKV_ERR_ARG;
  if (out_dtype != HKV_DT_F16 && out_dtype != HKV_DT_F32) return HKV_ERR_DTYPE;
  if (v_rows < 1 || k_cap < 0 || v_cap < 0 || k_cap > kPS * kHD || v_cap > kPS * kHD) return HKV_ERR_ARG;
  // page-head blocks and their rows are addressed in 32 bits
  if (num_blocks * H * kPS * kHD >= ((int64_t)1 << 31) || (int64_t)H * v_rows >= ((int64_t)1 << 31) ||
      T >= ((int64_t)1 << 31) - kPS)
    return HKV_ERR_SHAPE;
  if (!q || !block_table || !ks->codes || !ks->ocnt || !k_tables || !vs->codes || !vs->ocnt ||
      !v_tables || !out)
    return HKV_ERR_ARG;
  if ((k_cap > 0 && !ks->oent) || (v_cap > 0 && !vs->oent)) return HKV_ERR_ARG;
  if ((ks->ovf && !ks->ovf_ent) || (vs->ovf && !vs->ovf_ent)) return HKV_ERR_ARG;
  if (nsel > 0 && !sel) return HKV_ERR_ARG;
  if ((((uintptr_t)ks->codes | (uintptr_t)vs->codes) & 15u) || ((uintptr_t)q & 7u)) return HKV_ERR_ARG;
  const size_t need = hkv_decode_workspace_bytes(nsel, Hq, pages_per_split);
  if (!workspace || workspace_bytes < need) return HKV_ERR_WORKSPACE;
  const int64_t splits = n_splits(nsel, pages_per_split);
  if (splits > 0x7fffffff) return HKV_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  float* pm = (float*)workspace;
  float* pl = pm + splits * Hq;
  float* po = pl + splits * Hq;
  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.k = Side{ks->codes, nullptr, nullptr, nullptr, k_cap, (const hkv_table_t*)k_tables, 0, ks->ocnt,
             ks->oent, ks->ovf, ks->ovf_ent};
  a.v = Side{vs->codes, nullptr, nullptr, nullptr, v_cap, (const hkv_table_t*)v_tables, v_rows,
             vs->ocnt, vs->oent, vs->ovf, vs->ovf_ent};
  a.H = H;
  a.group = Hq / H;
  a.T = T;
  a.npages = (T + kPS - 1) / kPS;
  a.sel = sel;
  a.nsel = nsel;
  a.bt = block_table;
  a.nblocks = num_blocks;
  a.pps = pages_per_split;
  a.scale = scale;
  a.part_m = pm;
  a.part_l = pl;
  a.part_o = po;
  if (k_bits == 4 && v_bits == 4) launch_decode<4, 4, true>(a, splits, s);
  else if (k_bits == 4) launch_decode<4, 2, true>(a, splits, s);
  else if (v_bits == 4) launch_decode<2, 4, true>(a, splits, s);
  else launch_decode<2, 2, true>(a, splits, s);
  HKV_CHECK_LAUNCH();
  launch_merge(pm, pl, po, splits, Hq, kHD, out, out_dtype, s);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" size_t hkv_decode_workspace_bytes(int64_t nsel, int Hq, int pages_per_split) {
  if (nsel < 0 || Hq < 1 || pages_per_split < 1) return 0;
  return sizeof(float) * (size_t)n_splits(nsel, pages_per_split) * Hq * (2 + kHD);
}

extern "C" int hkv_decode_attn(const void* q, int Hq, int H, int D, int64_t T,
                               const void* k_packed, const int32_t* k_row_ptr,
                               const uint8_t* k_col, const uint16_t* k_val, int64_t k_cap,
                               int k_bits, const void* k_tables,
                               const void* v_packed, const int32_t* v_row_ptr,
                               const uint8_t* v_col, const uint16_t* v_val, int64_t v_cap,
                               int v_bits, const void* v_tables, int64_t v_rows,
                               const int64_t* sel, int64_t nsel, int pages_per_split, float scale,
                               void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                               void* stream) {
  if (D != kHD) return HKV_ERR_SHAPE;
  if (H < 1 || H > 65535 || Hq < H || Hq % H || Hq / H > 16 || T < 1 || nsel < 0)
    return HKV_ERR_SHAPE;
  if (pages_per_split < 1 || pages_per_split > kMaxPPS) return HKV_ERR_ARG;
  if ((k_bits != 2 && k_bits != 4) || (v_bits != 2 && v_bits != 4)) return HKV_ERR_ARG;
  if (out_dtype != HKV_DT_F16 && out_dtype != HKV_DT_F32) return HKV_ERR_DTYPE;
  if (v_rows < 1 || k_cap < 0 || v_cap < 0) return HKV_ERR_ARG;
  if (T * H * D >= ((int64_t)1 << 31) || (int64_t)H * v_rows >= ((int64_t)1 << 31))
    return HKV_ERR_SHAPE;
  if (!q || !k_packed || !k_row_ptr || !k_tables || !v_packed || !v_row_ptr || !v_tables || !out)
    return HKV_ERR_ARG;
  if ((k_cap > 0 && (!k_col || !k_val)) || (v_cap > 0 && (!v_col || !v_val))) return HKV_ERR_ARG;
  if (nsel > 0 && !sel) return HKV_ERR_ARG;
  if ((((uintptr_t)k_packed | (uintptr_t)v_packed) & 15u) || ((uintptr_t)q & 7u))
    return HKV_ERR_ARG;
  const size_t need = hkv_decode_workspace_bytes(nsel, Hq, pages_per_split);
  if (!workspace || workspace_bytes < need) return HKV_ERR_WORKSPACE;
  const int64_t splits = n_splits(nsel, pages_per_split);
  if (splits > 0x7fffffff) return HKV_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  float* pm = (float*)workspace;
  float* pl = pm + splits * Hq;
  float* po = pl + splits * Hq;
  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.k = Side{(const uint8_t*)k_packed, k_row_ptr, k_col, k_val, k_cap, (const hkv_table_t*)k_tables, 0,
             nullptr, nullptr};
  a.v = Side{(const uint8_t*)v_packed, v_row_ptr, v_col, v_val, v_cap, (const hkv_table_t*)v_tables,
             v_rows, nullptr, nullptr};
  a.bt = nullptr;
  a.nblocks = 0;
  a.H = H;
  a.group = Hq / H;
  a.T = T;
  a.npages = (T + kPS - 1) / kPS;
  a.sel = sel;
  a.nsel = nsel;
  a.pps = pages_per_split;
  a.scale = scale;
  a.part_m = pm;
  a.part_l = pl;
  a.part_o = po;
  if (k_bits == 4 && v_bits == 4) launch_decode<4, 4>(a, splits, s);
  else if (k_bits == 4) launch_decode<4, 2>(a, splits, s);
  else if (v_bits == 4) launch_decode<2, 4>(a, splits, s);
  else launch_decode<2, 2>(a, splits, s);
  HKV_CHECK_LAUNCH();
  launch_merge(pm, pl, po, splits, Hq, kHD, out, out_dtype, s);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" size_t hkv_decode_batch_workspace_bytes(int B, const int64_t* sel_offsets, int Hq,
                                                   int pages_per_split) {
  if (B < 1 || B > kMaxDecSeqs || !sel_offsets || Hq < 1 || pages_per_split < 1) return 0;
  int64_t splits = 0;
  for (int b = 0; b < B; ++b) {
    const int64_t n = sel_offsets[b + 1] - sel_offsets[b];
    if (n < 0) return 0;
    splits += n_splits(n, pages_per_split);
  }
  return sizeof(float) * (size_t)splits * Hq * (2 + kHD);
}

extern "C" int hkv_decode_attn_batch(const void* q, int B, int Hq, int H, int D, int64_t T,
                                     const int64_t* tok_offsets, const int64_t* seq_lens,
                                     const void* k_packed, const int32_t* k_row_ptr,
                                     const uint8_t* k_col, const uint16_t* k_val, int64_t k_cap,
                                     int k_bits, const void* k_tables,
                                     const void* v_packed, const int32_t* v_row_ptr,
                                     const uint8_t* v_col, const uint16_t* v_val, int64_t v_cap,
                                     int v_bits, const void* v_tables, int64_t v_rows,
                                     const int64_t* sel, const int64_t* sel_offsets,
                                     int pages_per_split, float scale, void* out, int out_dtype,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (D != kHD) return HKV_ERR_SHAPE;
  if (B < 1 || B > kMaxDecSeqs) return HKV_ERR_SHAPE;
  if (H < 1 || H > 65535 || Hq < H || Hq % H || Hq / H > 16 || T < 1) return HKV_ERR_SHAPE;
  if (pages_per_split < 1 || pages_per_split > kMaxPPS) return HKV_ERR_ARG;
  if ((k_bits != 2 && k_bits != 4) || (v_bits != 2 && v_bits != 4)) return HKV_ERR_ARG;
  if (out_dtype != HKV_DT_F16 && out_dtype != HKV_DT_F32) return HKV_ERR_DTYPE;
  if (v_rows < 1 || k_cap < 0 || v_cap < 0) return HKV_ERR_ARG;
  if (T * H * D >= ((int64_t)1 << 31) || (int64_t)H * v_rows >= ((int64_t)1 << 31))
    return HKV_ERR_SHAPE;
  if (!q || !k_packed || !k_row_ptr || !k_tables || !v_packed || !v_row_ptr || !v_tables || !out ||
      !tok_offsets || !seq_lens || !sel_offsets)
    return HKV_ERR_ARG;
  if ((k_cap > 0 && (!k_col || !k_val)) || (v_cap > 0 && (!v_col || !v_val))) return HKV_ERR_ARG;
  if ((((uintptr_t)k_packed | (uintptr_t)v_packed) & 15u) || ((uintptr_t)q & 7u))
    return HKV_ERR_ARG;
  DecSegs sg;
  sg.nseg = B;
  sg.split0[0] = 0;
  if (sel_offsets[0] < 0) return HKV_ERR_ARG;
  for (int b = 0; b < B; ++b) {
    const int64_t t0 = tok_offsets[b], n = seq_lens[b], ns = sel_offsets[b + 1] - sel_offsets[b];
    if (t0 < 0 || t0 % kPS || n < 1 || t0 + n > T || ns < 0) return HKV_ERR_ARG;
    if (ns > 0 && !sel) return HKV_ERR_ARG;
    sg.base[b] = t0;
    sg.T[b] = n;
    sg.sel0[b] = sel_offsets[b];
    sg.nsel[b] = ns;
    sg.split0[b + 1] = sg.split0[b] + n_splits(ns, pages_per_split);
  }
  const int64_t splits = sg.split0[B];
  if (splits > 0x7fffffff) return HKV_ERR_SHAPE;
  const size_t need = hkv_decode_batch_workspace_bytes(B, sel_offsets, Hq, pages_per_split);
  if (!workspace || workspace_bytes < need) return HKV_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  float* pm = (float*)workspace;
  float* pl = pm + splits * Hq;
  float* po = pl + splits * Hq;
  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.k = Side{(const uint8_t*)k_packed, k_row_ptr, k_col, k_val, k_cap, (const hkv_table_t*)k_tables, 0,
             nullptr, nullptr};
  a.v = Side{(const uint8_t*)v_packed, v_row_ptr, v_col, v_val, v_cap, (const hkv_table_t*)v_tables,
             v_rows, nullptr, nullptr};
  a.bt = nullptr;
  a.nblocks = 0;
  a.H = H;
  a.group = Hq / H;
  a.T = T;
  a.npages = (T + kPS - 1) / kPS;
  a.sel = sel;
  a.nsel = 0;
  a.pps = pages_per_split;
  a.scale = scale;
  a.part_m = pm;
  a.part_l = pl;
  a.part_o = po;
  if (k_bits == 4 && v_bits == 4) launch_decode_batch<4, 4>(a, sg, s);
  else if (k_bits == 4) launch_decode_batch<4, 2>(a, sg, s);
  else if (v_bits == 4) launch_decode_batch<2, 4>(a, sg, s);
  else launch_decode_batch<2, 2>(a, sg, s);
  HKV_CHECK_LAUNCH();
  MergeSegs ms;
  for (int b = 0; b <= B; ++b) ms.split0[b] = sg.split0[b];
  hipLaunchKernelGGL(merge_batch_kernel, dim3((unsigned)Hq, (unsigned)((kHD + kMergeCh - 1) / kMergeCh), (unsigned)B),
                     dim3(kDT), 0, s, pm, pl, po, ms, Hq, kHD, out, out_dtype);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" int hkv_paged_decode_attn_batch(const void* q, int B, int Hq, const int64_t* seq_lens,
                                           const int64_t* block_table, const int64_t* bt_offsets,
                                           const hkv_paged_side* ks, const void* k_tables,
                                           const hkv_paged_side* vs, const void* v_tables,
                                           int64_t v_rows, const int64_t* sel,
                                           const int64_t* sel_offsets, int pages_per_split,
                                           float scale, void* out, int out_dtype, void* workspace,
                                           size_t workspace_bytes, void* stream) {
  if (!ks || !vs) return HKV_ERR_ARG;
  const int H = ks->heads;
  const int64_t num_blocks = ks->num_blocks;
  const int k_bits = ks->bits, v_bits = vs->bits, k_cap = ks->cap, v_cap = vs->cap;
  if (B < 1 || B > kMaxDecSeqs) return HKV_ERR_SHAPE;
  if (vs->heads != H || vs->num_blocks != num_blocks) return HKV_ERR_SHAPE;
  if (H < 1 || H > 16 || Hq < H || Hq % H || Hq / H > 16 || num_blocks < 1) return HKV_ERR_SHAPE;
  if (pages_per_split < 1 || pages_per_split > kMaxPPS) return HKV_ERR_ARG;
  if ((k_bits != 2 && k_bits != 4) || (v_bits != 2 && v_bits != 4)) return HKV_ERR_ARG;
  if (out_dtype != HKV_DT_F16 && out_dtype != HKV_DT_F32) return HKV_ERR_DTYPE;
  if (v_rows < 1 || k_cap < 0 || v_cap < 0 || k_cap > kPS * kHD || v_cap > kPS * kHD) return HKV_ERR_ARG;
  if (num_blocks * H * kPS * kHD >= ((int64_t)1 << 31) || (int64_t)H * v_rows >= ((int64_t)1 << 31))
    return HKV_ERR_SHAPE;
  if (!q || !block_table || !ks->codes || !ks->ocnt || !k_tables || !vs->codes || !vs->ocnt ||
      !v_tables || !out || !seq_lens || !bt_offsets || !sel_offsets)
    return HKV_ERR_ARG;
  if ((k_cap > 0 && !ks->oent) || (v_cap > 0 && !vs->oent)) return HKV_ERR_ARG;
  if ((ks->ovf && !ks->ovf_ent) || (vs->ovf && !vs->ovf_ent)) return HKV_ERR_ARG;
  if ((((uintptr_t)ks->codes | (uintptr_t)vs->codes) & 15u) || ((uintptr_t)q & 7u)) return HKV_ERR_ARG;
  DecSegs sg;
  sg.nseg = B;
  sg.split0[0] = 0;
  if (sel_offsets[0] < 0) return HKV_ERR_ARG;
  for (int b = 0; b < B; ++b) {
    const int64_t n = seq_lens[b], ns = sel_offsets[b + 1] - sel_offsets[b];
    if (n < 1 || n >= ((int64_t)1 << 31) - kPS || bt_offsets[b] < 0 || ns < 0) return HKV_ERR_ARG;
    if (ns > 0 && !sel) return HKV_ERR_ARG;
    sg.base[b] = bt_offsets[b];
    sg.T[b] = n;
    sg.sel0[b] = sel_offsets[b];
    sg.nsel[b] = ns;
    sg.split0[b + 1] = sg.split0[b] + n_splits(ns, pages_per_split);
  }
  const int64_t splits = sg.split0[B];
  if (splits > 0x7fffffff) return HKV_ERR_SHAPE;
  const size_t need = hkv_decode_batch_workspace_bytes(B, sel_offsets, Hq, pages_per_split);
  if (!workspace || workspace_bytes < need) return HKV_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  float* pm = (float*)workspace;
  float* pl = pm + splits * Hq;
  float* po = pl + splits * Hq;
  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.k = Side{ks->codes, nullptr, nullptr, nullptr, k_cap, (const hkv_table_t*)k_tables, 0, ks->ocnt,
             ks->oent, ks->ovf, ks->ovf_ent};
  a.v = Side{vs->codes, nullptr, nullptr, nullptr, v_cap, (const hkv_table_t*)v_tables, v_rows,
             vs->ocnt, vs->oent, vs->ovf, vs->ovf_ent};
  a.H = H;
  a.group = Hq / H;
  a.T = 0;
  a.npages = 0;
  a.sel = sel;
  a.nsel = 0;
  a.bt = block_table;
  a.nblocks = num_blocks;
  a.pps = pages_per_split;
  a.scale = scale;
  a.part_m = pm;
  a.part_l = pl;
  a.part_o = po;
  if (k_bits == 4 && v_bits == 4) launch_decode_batch<4, 4, true>(a, sg, s);
  else if (k_bits == 4) launch_decode_batch<4, 2, true>(a, sg, s);
  else if (v_bits == 4) launch_decode_batch<2, 4, true>(a, sg, s);
  else launch_decode_batch<2, 2, true>(a, sg, s);
  HKV_CHECK_LAUNCH();
  MergeSegs ms;
  for (int b = 0; b <= B; ++b) ms.split0[b] = sg.split0[b];
  hipLaunchKernelGGL(merge_batch_kernel, dim3((unsigned)Hq, (unsigned)((kHD + kMergeCh - 1) / kMergeCh), (unsigned)B),
                     dim3(kDT), 0, s, pm, pl, po, ms, Hq, kHD, out, out_dtype);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

// Workspace: the flags (one byte per page) at its start, the per-chunk
// counts (at most total_pages / kUnionChunk + kMaxDecSeqs + 1 chunks) at its
// end.  A buffer reused by calls over different page counts keeps every
// call's counts past every call's flags: a call over P pages needs its size
// W >= align256(P) + 4 n(P) with n growing with P, so the flags of any call
// end below W - 4 n(P) for every P it can hold.
static size_t union_counts(int64_t total_pages) { return (size_t)total_pages / kUnionChunk + kMaxDecSeqs + 1; }

extern "C" size_t hkv_union_pages_workspace_bytes(int64_t total_pages) {
  if (total_pages < 0) return 0;
  const size_t f = ((size_t)total_pages + 255) & ~(size_t)255;
  return f + sizeof(uint32_t) * union_counts(total_pages);
}

extern "C" int hkv_union_pages_ragged(const int64_t* sel, int H, int B, const int64_t* row_offsets,
                                      const int64_t* page_offsets, int64_t* out, void* flags,
                                      size_t flags_bytes, void* stream) {
  if (B < 1 || B > kMaxDecSeqs || H < 1) return HKV_ERR_SHAPE;
  if (!row_offsets || !page_offsets || !out || !flags) return HKV_ERR_ARG;
  UnionSegs sg;
  sg.nseg = B;
  if (row_offsets[0] != 0 || page_offsets[0] != 0) return HKV_ERR_ARG;
  sg.chunk0[0] = 0;
  for (int b = 0; b <= B; ++b) {
    if (b > 0 && (row_offsets[b] < row_offsets[b - 1] || page_offsets[b] < page_offsets[b - 1]))
      return HKV_ERR_ARG;
    sg.row0[b] = row_offsets[b];
    sg.page0[b] = page_offsets[b];
    if (b > 0)
      sg.chunk0[b] = sg.chunk0[b - 1] + (page_offsets[b] - page_offsets[b - 1] + kUnionChunk - 1) / kUnionChunk;
  }
  if (sg.row0[B] > 0 && !sel) return HKV_ERR_ARG;
  if (flags_bytes < hkv_union_pages_workspace_bytes(sg.page0[B])) return HKV_ERR_WORKSPACE;
  const int64_t chunks = sg.chunk0[B];
  if (chunks > 0x7fffffff) return HKV_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  uint8_t* fl = (uint8_t*)flags;
  uint32_t* cnt = (uint32_t*)(fl + ((flags_bytes - sizeof(uint32_t) * union_counts(sg.page0[B])) & ~(size_t)3));
  const int64_t n = sg.row0[B] * H;
  if (n > 0) {
    hipLaunchKernelGGL(union_mark_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, sel, H, sg, fl);
    HKV_CHECK_LAUNCH();
  }
  if (chunks > 0) {
    hipLaunchKernelGGL(union_count_kernel, dim3((unsigned)chunks), dim3(kUnionThreads), 0, s, fl, sg, cnt);
    HKV_CHECK_LAUNCH();
    hipLaunchKernelGGL(union_write_kernel, dim3((unsigned)chunks), dim3(kUnionThreads), 0, s, fl, sg, cnt, H, out);
    HKV_CHECK_LAUNCH();
  }
  return HKV_OK;
}

extern "C" size_t hkv_selected_attention_workspace_bytes(int64_t nsel, int page_size, int Hq,
                                                         int Dv) {
  if (nsel < 0 || page_size < 1 || page_size > kDenseKeys || Hq < 1 || Dv < 1) return 0;
  const int pps = kDenseKeys / page_size;
  return sizeof(float) * (size_t)n_splits(nsel, pps) * Hq * (2 + (size_t)Dv);
}

extern "C" int hkv_selected_attention(const void* q, int q_dtype, int Hq, int D, const void* k_pages,
                                      const void* v_pages, int kv_dtype, int64_t P, int page_size,
                                      int Hk, int Hv, int Dv, const int64_t* sel, int64_t nsel,
                                      int sel_cols, int head_map, float scale, void* out,
                                      int out_dtype, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  auto okdt = [](int d) { return d == HKV_DT_F16 || d == HKV_DT_F32 || d == HKV_DT_BF16; };
  if (!okdt(q_dtype) || !okdt(kv_dtype) || !okdt(out_dtype)) return HKV_ERR_DTYPE;
  if (Hq < 1 || Hk < 1 || Hv < 1 || D < 1 || Dv < 1 || D > kDenseMaxD || Dv > kDenseMaxD ||
      P < 0 || nsel < 0 || page_size < 1 || page_size > kDenseKeys || Hq > 65535)
    return HKV_ERR_SHAPE;
  if (head_map == 0) {
    if (Hk != Hq) return HKV_ERR_SHAPE;
  } else if (head_map == 1) {
    if (Hq % Hk || Hv != Hk) return HKV_ERR_SHAPE;
  } else {
    return HKV_ERR_ARG;
  }
  if (sel_cols != Hq && sel_cols != Hk) return HKV_ERR_SHAPE;
  if (!q || !out || (nsel > 0 && (!sel || !k_pages || !v_pages))) return HKV_ERR_ARG;
  const size_t need = hkv_selected_attention_workspace_bytes(nsel, page_size, Hq, Dv);
  if (!workspace || workspace_bytes < need) return HKV_ERR_WORKSPACE;
  const int pps = kDenseKeys / page_size;
  const int64_t splits = n_splits(nsel, pps);
  if (splits > 0x7fffffff) return HKV_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  DenseArgs a;
  a.q = q;
  a.k = k_pages;
  a.v = v_pages;
  a.q_dt = q_dtype;
  a.kv_dt = kv_dtype;
  a.P = P;
  a.S = page_size;
  a.Hk = Hk;
  a.Hv = Hv;
  a.D = D;
  a.Dv = Dv;
  a.Hq = Hq;
  a.head_map = head_map;
  a.sel = sel;
  a.nsel = nsel;
  a.ncols = sel_cols;
  a.pps = pps;
  a.scale = scale;
  a.part_m = (float*)workspace;
  a.part_l = a.part_m + splits * Hq;
  a.part_o = a.part_l + splits * Hq;
  hipLaunchKernelGGL(dense_attn_kernel, dim3((unsigned)splits, (unsigned)Hq), dim3(kDT), 0, s, a);
  HKV_CHECK_LAUNCH();
  launch_merge(a.part_m, a.part_l, a.part_o, splits, Hq, Dv, out, out_dtype, s);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
