// paged.hip -- the paged compact KV pool: slot-mapped writes of bit-packed
// nuq codes with per-page outlier lists and K page statistics, and the
// gather-dequant of kept blocks.
//
// The reference's pool (src/kvquant/compact_pool.py:398-537) stores one byte
// per code plus dense fp16 outlier values and a u8 mask per element, (L, NB,
// BS, H, D), and plans a bit-packed layout with outliers kept beside the
// block table (compact_pool.py:11-12, vllm_integration.md:51-55).  This pool
// is that plan, laid out for per-head page reads.  Per layer and side (K or
// V), D = 128, page (block) size 16:
//   codes  (NB, H, 16, D*bits/8) u8   page-head blocks: the 16 slots of one
//                                     head are contiguous (nuq4 1 KiB, nuq2
//                                     512 B), little-endian codes in a byte
//   ocnt   (NB, H) int32              outliers recorded for the page-head
//   oent   (NB, H, cap) u32           its outliers, (slot, channel) ascending:
//                                     fp16 value | channel << 16 | slot << 24
//   kmin / kmax (NB, H, D) fp16       K only: min / max over the page-head's
//                                     written slots of the dequantised values
//                                     (the outlier's value, else the fp16
//                                     pole), a zero stored as +0
//   status int32                      bit 0 set when a page-head's outliers
//                                     exceeded cap (ocnt then still counts
//                                     them all; the first cap are kept)
//
// Write (hkv_paged_write, the counterpart of CompactKVPool.write_kv,
// compact_pool.py:447-489 with K10/K11 :160-287): token t goes to slot
// slot_mapping[t] (skipped if < 0 or past the pool).  A run is a maximal
// stretch of consecutive tokens whose slots are consecutive within one page;
// each run is written by one wave per head.  A run starting at slot w0 keeps
// the page-head's entries of slots < w0 and replaces the rest (a rewrite of
// earlier slots, e.g. a rollback, truncates the page there); its statistics
// restart when w0 = 0 and otherwise fold into the page's.  The tokens a call
// writes into one page must form one run (vLLM's slot mappings do: a
// sequence's new tokens take consecutive slots).
#include "nuq_core.h"

#include <algorithm>

namespace {

constexpr int kPD = 128;       // head dim
constexpr int kPBS = 16;       // page (block) size
constexpr int kPT = 256;       // threads per block
constexpr int kPW = kPT / 64;  // waves per block
constexpr uint32_t kInf2 = 0x7c007c00u, kNInf2 = 0xfc00fc00u;

HKV_DEV void pwave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

HKV_DEV uint32_t pk_min(uint32_t a, uint32_t b) { return as_u32(__builtin_elementwise_min(as_h2(a), as_h2(b))); }
HKV_DEV uint32_t pk_max(uint32_t a, uint32_t b) { return as_u32(__builtin_elementwise_max(as_h2(a), as_h2(b))); }

struct PagedWriteArgs {
  const uint16_t* x;   // (T, H, 128) fp16
  int64_t T;
  int H;
  hkv_nuq_scales sc;   // tables required; V: row of token t = h * rows + clamp(pos(t))
  const int64_t* slots;
  int64_t nslots;      // NB * 16
  uint8_t* codes;
  int32_t* ocnt;
  uint32_t* oent;
  int cap;
  uint16_t* kmin;
  uint16_t* kmax;
  int32_t* status;
  int64_t nunits;      // ceil(T / 16) * H
  int32_t* ovf;        // (NB, H) overflow chunk of the page-head, -1: none
  uint32_t* ovf_ent;   // (n_chunks, 16 * 128 - cap)
  int32_t* ovf_next;   // chunks handed out so far
  int n_chunks;
};

// Entry i of a page-head's list: the first cap inline, the rest in its
// overflow chunk (ovf >= 0).
HKV_DEV uint32_t* entry_ptr(uint32_t* oent, uint32_t* ovf_ent, int64_t ph, int cap, int ovf, int i) {
  return i < cap ? oent + ph * cap + i : ovf_ent + (int64_t)ovf * (kPBS * kPD - cap) + (i - cap);
}

// Codes and outlier flags of one lane's 8 channels (quant8_packed with the
// per-pair outlier masks and codes kept for the statistics): returns true on
// the fast (decision-table) path.  om[j]: 0xffff in a 16-bit lane whose
// element is an outlier; on the exact path also code[j] (codes of the pair
// in bits 0..3 / 16..19).
template <int NB, bool PT, int BITS, typename TabFn, bool XMIN>
HKV_DEV bool quant8_paged(const uint4 xv, const Search2<NB>* S, const SlowInfo& si, TabFn tab,
                          uint32_t xmin, uint32_t* packed, uint32_t* mask8, uint32_t om[4],
                          uint32_t code[4]) {
  const uint32_t x[4] = {xv.x, xv.y, xv.z, xv.w};
  uint32_t uns = 0;
  if constexpr (PT || XMIN) {
    u2_t mg = __builtin_bit_cast(u2_t, x[0] & 0x7fff7fffu);
#pragma unroll
    for (int j = 1; j < 4; ++j) mg = __builtin_elementwise_max(mg, __builtin_bit_cast(u2_t, x[j] & 0x7fff7fffu));
    if constexpr (PT) {
      uns = unsafe2<NB>(__builtin_bit_cast(uint32_t, mg), S[0]);
    } else {
      const s2_t d = as_s2(xmin) - as_s2(__builtin_bit_cast(uint32_t, mg));
      uns = as_u32(d) & 0x80008000u;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) uns |= unsafe2<NB>(x[j], S[j]);
  }
  if (__builtin_expect(uns == 0, 1)) {
    uint32_t M = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      om[j] = as_u32(as_s2(outlier2_sign<NB>(x[j], S[PT ? 0 : j])) >> (s2_t){15, 15});
      M = place(posm(j), om[j], M);
    }
    *mask8 = (M | (M >> 16)) & 0xffu;
    if constexpr ((BITS == 2 && NB == 2) || (BITS == 4 && NB == 4)) {
      uint32_t A = 0, B = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t m[NB];
        search_masks<NB>(x[j], S[PT ? 0 : j], m);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          if constexpr (BITS == 2) A = place_not(pos2(j, b), m[b], A);
          else if (j < 2) A = place_not(pos4(j, b), m[b], A);
          else B = place_not(pos4(j, b), m[b], B);
        }
      }
      if constexpr (BITS == 2) *packed = A | (A >> 16);
      else *packed = ((A & 0xffffu) | (B & 0xffff0000u)) | __builtin_amdgcn_alignbit(B, A, 16);
    } else {
      uint32_t c[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = search2<NB>(x[j], S[PT ? 0 : j]);
      *packed = BITS == 4 ? pack_nibbles(c) : pack_crumbs(c);
    }
    return true;
  }
#pragma unroll 1
  for (int j = 0; j < 4; ++j) {
    int o0, o1;
    const int c0 = slow_one((uint16_t)(x[j] & 0xffffu), si, tab(2 * j), &o0);
    const int c1 = slow_one((uint16_t)(x[j] >> 16), si, tab(2 * j + 1), &o1);
    code[j] = (uint32_t)c0 | ((uint32_t)c1 << 16);
    om[j] = (o0 ? 0xffffu : 0u) | (o1 ? 0xffff0000u : 0u);
  }
  *packed = BITS == 4 ? pack_nibbles(code) : pack_crumbs(code);
  *mask8 = mask_bits(om);
  return false;
}

// fp16 pole of `code` in table `t` (the dequantised value of a code).
HKV_DEV uint32_t pole16(const hkv_table_t* tabs, int64_t t, uint32_t code) {
  return tabs[t].pf16[code & 15u];
}

// Quantise-then-dequantise of the two fp16 lanes of x under the pair's
// tables (the fast path applies: |x| within the tables' safe range), with
// ±inf sentinels passed through: an outlier keeps its value, any other
// element becomes its fp16 pole.
template <int NB>
HKV_DEV uint32_t qd2(uint32_t x, const Search2<NB>& s, const hkv_table_t* tabs, int64_t t0, int64_t t1) {
  const uint32_t o = outlier2<NB>(x, s);
  const uint32_t c = search2<NB>(x, s);
  uint32_t r = x;
  const uint32_t lo = x & 0xffffu, hi = x >> 16;
  if (lo != 0x7c00u && lo != 0xfc00u && !(o & 0xffffu)) r = (r & 0xffff0000u) | pole16(tabs, t0, c);
  if (hi != 0x7c00u && hi != 0xfc00u && !(o >> 16)) r = (r & 0xffffu) | (pole16(tabs, t1, c >> 16) << 16);
  return r;
}

HKV_DEV uint32_t pos_zero2(uint32_t v) {  // -0 -> +0 in both halves
  if ((v & 0xffffu) == 0x8000u) v &= 0xffff0000u;
  if ((v >> 16) == 0x8000u) v &= 0xffffu;
  return v;
}

// One wave per (16-token group, head) unit: the runs that start in the
// group, written for the wave's head.  STATS (K): page min / max of the
// dequantised values.
template <int NB, bool PT, int BITS, bool STATS>
__global__ void __launch_bounds__(kPT) __attribute__((amdgpu_waves_per_eu(PT ? 5 : 3)))
paged_write_kernel(PagedWriteArgs A) {
  constexpr int RB = kPD * BITS / 8;    // packed bytes per row
  constexpr int TW = 20;                // staged table words per row
  __shared__ __align__(16) uint32_t s_tab[PT ? kPW * kPBS * TW : 1];
  __shared__ __align__(16) uint4 s_x[kPW * 64];

  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = lane & 15, rw = lane >> 4;
  const hkv_table_t* tabs = (const hkv_table_t*)A.sc.tables;
  const SlowInfo si = slow_info(A.sc);
  const int H = A.H;
  uint32_t* wtab = s_tab + (PT ? wv * kPBS * TW : 0);

  // STATS: per channel, the ordered keys of the least / greatest value taken
  // as-is (outliers, and exact-path elements at their dequantised value)
  __shared__ int s_okey[STATS ? kPW * 2 * kPD : 1];
  int* okmin = s_okey + (STATS ? wv * 2 * kPD : 0);
  int* okmax = okmin + kPD;

  Search2<NB> S[PT ? 1 : 4];
  uint32_t xmin = 0;
  int cur_h = -1;
  const int64_t nwaves = (int64_t)gridDim.x * kPW;
  for (int64_t u = (int64_t)blockIdx.x * kPW + wv; u < A.nunits; u += nwaves) {
    const int64_t g = u / H;
    const int h = (int)(u - g * H);
    if constexpr (!PT) {
      if (h != cur_h) {  // uniform: the wave's tables for this head
        cur_h = h;
        const int64_t tab0 = (int64_t)h * kPD + 8 * cg;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          load_search_pair<NB>(tabs + tab0 + 2 * j, tabs + tab0 + 2 * j + 1, S[j]);
        xmin = xsafe_min<NB>(S);
      }
    }
    // slots of tokens 16g - 1 + l (l < 33) and of their predecessors
    const int64_t tok = g * kPBS - 1 + lane;
    int64_t s = -1, sp = -1;
    if (lane < 33 && tok >= 0 && tok < A.T) s = A.slots[tok];
    if (lane < 33 && tok >= 1 && tok - 1 < A.T) sp = A.slots[tok - 1];
    const bool valid = s >= 0 && s < A.nslots;
    const bool contig = lane >= 1 && valid && sp >= 0 && sp < A.nslots && s == sp + 1 && (s % kPBS) != 0;
    uint64_t starts = __builtin_amdgcn_ballot_w64(valid && !contig && lane >= 1 && lane <= kPBS);
    const uint64_t conts = __builtin_amdgcn_ballot_w64(contig);
    while (starts) {
      const int l0 = __builtin_ctzll(starts);
      starts &= starts - 1;
      const int n = 1 + __builtin_ctzll(~(conts >> (l0 + 1)));  // 1..16
      const int64_t t0 = g * kPBS - 1 + l0;
      const int64_t s0 = (int64_t)__builtin_amdgcn_readlane((int)(s & 0xffffffff), l0) |
                         ((int64_t)__builtin_amdgcn_readlane((int)(s >> 32), l0) << 32);
      const int64_t pg = s0 / kPBS;
      const int w0 = (int)(s0 - pg * kPBS);
      const int64_t ph = pg * H + h;
      // entries kept from earlier writes: those of slots < w0
      // the page-head's overflow chunk (kept across writes once allocated)
      int ovf = A.ovf ? A.ovf[ph] : -1;
      const int room = A.cap + (ovf >= 0 ? kPBS * kPD - A.cap : 0);  // entries it can store
      int base = 0;
      if (w0 > 0) {
        const int cnt = A.ocnt[ph];
        const int m = cnt < room ? cnt : room;
        int below = 0;
        for (int i0 = 0; i0 < m; i0 += 64) {
          const int i = i0 + lane;
          const bool lt = i < m && (int)(*entry_ptr(A.oent, A.ovf_ent, ph, A.cap, ovf, i) >> 24) < w0;
          below += __builtin_popcountll(__builtin_amdgcn_ballot_w64(lt));
        }
        base = below == m ? cnt : below;
      }
      if constexpr (PT) {  // the run's per-token tables, in search form
        for (int i = lane; i < n * 3; i += 64) {
          const int rr = i / 3, q = i - rr * 3;
          const int64_t t = t0 + rr;
          const int64_t tab = (int64_t)h * A.sc.rows + clamp_row(token_pos(A.sc, t), A.sc.rows);
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
        pwave_sync();
      }
      uint4 xs[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int rr = p * 4 + rw;
        xs[p] = make_uint4(0u, 0u, 0u, 0u);
        if (rr < n) xs[p] = *reinterpret_cast<const uint4*>(A.x + ((t0 + rr) * H + h) * kPD + 8 * cg);
      }
      // STATS: least / greatest non-outlier input of the lane's channel pairs
      // (fast path); the dequantised value of those is their pole, which is
      // monotone in the input
      uint32_t nmin[4], nmax[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) { nmin[j] = kInf2; nmax[j] = kNInf2; }
      if constexpr (STATS) {
        okmin[lane] = okmin[lane + 64] = 0x7fffffff;
        okmax[lane] = okmax[lane + 64] = (int)0x80000000;
        pwave_sync();
      }
      uint32_t run = 0;
      uint8_t* cpage = A.codes + (ph * kPBS + w0) * RB;
      uint32_t* epage = A.oent + ph * A.cap;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int rr = p * 4 + rw;
        uint32_t m = 0;
        bool fold = false;  // STATS: fold this lane's outliers into the LDS keys
        if (p * 4 < n) {  // uniform
          if (rr < n) {
            const int64_t t = t0 + rr;
            uint32_t pk, om[4], code[4];
            bool fast;
            if constexpr (PT) {
              const uint32_t* tw = wtab + rr * TW;
#pragma unroll
              for (int i = 0; i < (1 << NB) - 1; ++i) S[0].bp[i] = tw[i];
              S[0].lo = tw[15];
              S[0].up = tw[16];
              S[0].xsafe = tw[17];
              const RowTabAt tab{A.sc.rows, A.sc.positions, A.sc.pos_offset, h, t};
              fast = quant8_paged<NB, PT, BITS, RowTabAt, false>(xs[p], S, si, tab, 0, &pk, &m, om, code);
            } else {
              const ChanTab tab{(int64_t)h * kPD + 8 * cg};
              fast = quant8_paged<NB, PT, BITS, ChanTab, true>(xs[p], S, si, tab, xmin, &pk, &m, om, code);
              if constexpr (STATS) {
                const uint32_t x4[4] = {xs[p].x, xs[p].y, xs[p].z, xs[p].w};
                if (fast) {
#pragma unroll
                  for (int j = 0; j < 4; ++j) {
                    nmin[j] = pk_min(nmin[j], bsel(om[j], kInf2, x4[j]));
                    nmax[j] = pk_max(nmax[j], bsel(om[j], kNInf2, x4[j]));
                  }
                } else {  // exact path: fold every dequantised value as-is
#pragma unroll 1
                  for (int e = 0; e < 8; ++e) {
                    const uint32_t w = x4[e >> 1] >> (16 * (e & 1));
                    const bool o = (om[e >> 1] >> (16 * (e & 1))) & 1u;
                    const uint32_t c = (code[e >> 1] >> (16 * (e & 1))) & 15u;
                    const uint16_t r = o ? (uint16_t)w : (uint16_t)pole16(tabs, tab(e), c);
                    atomicMin(&okmin[8 * cg + e], hkey(r));
                    atomicMax(&okmax[8 * cg + e], hkey(r));
                  }
                }
                fold = fast;  // the fast path's outliers are folded as their entries are written
              }
            }
            (void)fast;
            if constexpr (BITS == 4)
              *reinterpret_cast<uint32_t*>(cpage + rr * RB + 4 * cg) = pk;
            else
              *reinterpret_cast<uint16_t*>(cpage + rr * RB + 2 * cg) = (uint16_t)pk;
            s_x[wv * 64 + lane] = xs[p];
          }
          // lanes are in (row, channel) order: the wave's exclusive count is
          // the entry's position in (slot, channel) order
          uint32_t tot;
          const uint32_t pos = run + wave_excl_count_fused(__builtin_popcount(m), &tot);
          run += tot;
          if (ovf == -1 && A.ovf && base + (int)run > A.cap && A.cap < kPBS * kPD) {
            // uniform: the first entry past the inline capacity takes a chunk
            int got = -2;  // -2: the arena is used up (entries past cap are dropped)
            if (lane == 0) {
              const int i = atomicAdd(A.ovf_next, 1);
              if (i < A.n_chunks) {
                got = i;
                A.ovf[ph] = i;
              }
            }
            ovf = __builtin_amdgcn_readfirstlane(got);
          }
          const uint16_t* xl = reinterpret_cast<const uint16_t*>(s_x + wv * 64 + lane);
          const uint32_t tag = ((uint32_t)(w0 + rr) << 24) | ((uint32_t)(8 * cg) << 16);
          uint32_t idx = (uint32_t)base + pos;
          while (m) {
            const int e = __builtin_ctz(m);
            m &= m - 1u;
            const uint16_t v = xl[e];
            const uint32_t ent = (uint32_t)v | (tag + ((uint32_t)e << 16));
            if (idx < (uint32_t)A.cap) epage[idx] = ent;
            else if (ovf >= 0) A.ovf_ent[(int64_t)ovf * (kPBS * kPD - A.cap) + (idx - A.cap)] = ent;
            ++idx;
            if constexpr (STATS) {
              if (fold) {
                atomicMin(&okmin[8 * cg + e], hkey(v));
                atomicMax(&okmax[8 * cg + e], hkey(v));
              }
            }
          }
        }
      }
      if (lane == 0) {
        const int total = base + (int)run;
        A.ocnt[ph] = total;
        if (total > A.cap + (ovf >= 0 ? kPBS * kPD - A.cap : 0)) atomicOr(A.status, 1);
      }
      if constexpr (STATS) {
        // over the four row groups of the wave (lanes cg, cg+16, cg+32, cg+48)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int off = 16; off <= 32; off <<= 1) {
            nmin[j] = pk_min(nmin[j], (uint32_t)__shfl_xor((int)nmin[j], off, 64));
            nmax[j] = pk_max(nmax[j], (uint32_t)__shfl_xor((int)nmax[j], off, 64));
          }
        }
        pwave_sync();  // the LDS keys of every lane's outliers
        if (rw == 0) {
          const int64_t tab0 = (int64_t)h * kPD + 8 * cg;
          uint32_t lo4[4], hi4[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            // the pole of the least / greatest non-outlier, then the values
            // taken as-is (a key of +-2^31 - 1 / -2^31: none)
            const uint32_t a = qd2<NB>(nmin[j], S[j], tabs, tab0 + 2 * j, tab0 + 2 * j + 1);
            const uint32_t b = qd2<NB>(nmax[j], S[j], tabs, tab0 + 2 * j, tab0 + 2 * j + 1);
            const int k0 = okmin[8 * cg + 2 * j], k1 = okmin[8 * cg + 2 * j + 1];
            const int q0 = okmax[8 * cg + 2 * j], q1 = okmax[8 * cg + 2 * j + 1];
            const uint32_t omn = (k0 == 0x7fffffff ? 0x7c00u : (uint32_t)hkey_inv(k0)) |
                                 ((k1 == 0x7fffffff ? 0x7c00u : (uint32_t)hkey_inv(k1)) << 16);
            const uint32_t omx = (q0 == (int)0x80000000 ? 0xfc00u : (uint32_t)hkey_inv(q0)) |
                                 ((q1 == (int)0x80000000 ? 0xfc00u : (uint32_t)hkey_inv(q1)) << 16);
            lo4[j] = pos_zero2(pk_min(a, omn));
            hi4[j] = pos_zero2(pk_max(b, omx));
          }
          uint4* mnp = reinterpret_cast<uint4*>(A.kmin + ph * kPD + 8 * cg);
          uint4* mxp = reinterpret_cast<uint4*>(A.kmax + ph * kPD + 8 * cg);
          if (w0 > 0) {
            const uint4 a = *mnp, b = *mxp;
            const uint32_t oa[4] = {a.x, a.y, a.z, a.w}, ob[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              lo4[j] = pk_min(lo4[j], oa[j]);
              hi4[j] = pk_max(hi4[j], ob[j]);
            }
          }
          *mnp = make_uint4(lo4[0], lo4[1], lo4[2], lo4[3]);
          *mxp = make_uint4(hi4[0], hi4[1], hi4[2], hi4[3]);
        }
      }
      if constexpr (PT) pwave_sync();  // the staged tables are refilled by the next run
    }
  }
}

int paged_num_cus() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
  }
  return n;
}

template <typename K>
unsigned paged_grid(K kernel, int64_t nblocks) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kPT, 0) != hipSuccess || per_cu < 1)
    per_cu = 1;
  const int64_t cap = (int64_t)per_cu * paged_num_cus();
  return (unsigned)std::max<int64_t>(1, std::min<int64_t>(nblocks, cap));
}

template <int NB, bool PT, int BITS, bool STATS>
void launch_write(const PagedWriteArgs& a, hipStream_t s) {
  auto k = paged_write_kernel<NB, PT, BITS, STATS>;
  const unsigned grid = paged_grid(k, (a.nunits + kPW - 1) / kPW);
  hipLaunchKernelGGL(k, dim3(grid), dim3(kPT), 0, s, a);
}

template <bool PT, int BITS, bool STATS>
void launch_write_nb(int nb, const PagedWriteArgs& a, hipStream_t s) {
  switch (nb) {
    case 0: launch_write<0, PT, BITS, STATS>(a, s); break;
    case 1: launch_write<1, PT, BITS, STATS>(a, s); break;
    case 2: launch_write<2, PT, BITS, STATS>(a, s); break;
    case 3: if constexpr (BITS == 4) launch_write<3, PT, BITS, STATS>(a, s); break;
    default: if constexpr (BITS == 4) launch_write<4, PT, BITS, STATS>(a, s); break;
  }
}

// ------------------------------------------------------------------ gather
//
// One wave per (kept block k, head h): the page-head's 16 slots dequantised
// into an LDS tile, its outliers written over it, the rows stored to
// staging[k, slot, h, :].  Per-token (V) scales use row
// min(first_pos[k] + slot, rows - 1).  Block ids outside the pool give zero
// rows.

struct PagedGatherArgs {
  const uint8_t* codes;
  const int32_t* ocnt;
  const uint32_t* oent;
  int cap;
  int64_t NB;
  int H;
  hkv_nuq_scales sc;
  const int64_t* ids;
  const int64_t* first_pos;
  int64_t NK;
  uint16_t* out;   // (NK, 16, H, 128)
  const int32_t* ovf;       // (NB, H) overflow chunk per page-head, or NULL
  const uint32_t* ovf_ent;  // (chunks, 16 * 128 - cap)
};

template <bool PT, int BITS>
__global__ void __launch_bounds__(kPT)
paged_gather_kernel(PagedGatherArgs A) {
  constexpr int RB = kPD * BITS / 8;
  constexpr int NL = 1 << BITS;
  constexpr int SC = kPD + 2;  // halfwords per (level) row of the K poles (skewed)
  extern __shared__ uint16_t dyn[];
  const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = lane & 15, rw = lane >> 4;
  const int H = A.H;
  uint16_t* tile = dyn + wv * (kPBS * kPD);          // [slot][channel]
  uint16_t* prow = dyn + kPW * kPBS * kPD + wv * (kPBS * 16);  // PT: poles of each slot
  uint16_t* kp = dyn + kPW * kPBS * kPD;            // K: [h][level][channel]
  const hkv_table_t* tabs = (const hkv_table_t*)A.sc.tables;
  if constexpr (!PT) {
    for (int i = tid; i < H * kPD; i += kPT) {
      const uint4* src = reinterpret_cast<const uint4*>(tabs[i].pf16);
      const uint4 a = src[0], b = src[1];
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      const int hh = i / kPD, d = i % kPD;
#pragma unroll
      for (int l = 0; l < NL; ++l) kp[(hh * NL + l) * SC + d] = (uint16_t)(w[l >> 1] >> (16 * (l & 1)));
    }
    __syncthreads();
  }
  const int64_t items = A.NK * H;
  const int64_t nwaves = (int64_t)gridDim.x * kPW;
  for (int64_t it = (int64_t)blockIdx.x * kPW + wv; it < items; it += nwaves) {
    const int64_t k = it / H;
    const int h = (int)(it - k * H);
    const int64_t id = A.ids[k];
    uint16_t* ob = A.out + (k * kPBS * H + h) * kPD;
    if (id < 0 || id >= A.NB) {  // uniform
#pragma unroll
      for (int p = 0; p < 4; ++p)
        *reinterpret_cast<uint4*>(ob + (int64_t)(p * 4 + rw) * H * kPD + 8 * cg) = make_uint4(0u, 0u, 0u, 0u);
      continue;
    }
    const int64_t ph = id * H + h;
    const uint8_t* cp = A.codes + ph * kPBS * RB;
    uint32_t cw[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if constexpr (BITS == 4) cw[p] = *reinterpret_cast<const uint32_t*>(cp + (p * 4 + rw) * RB + 4 * cg);
      else cw[p] = *reinterpret_cast<const uint16_t*>(cp + (p * 4 + rw) * RB + 2 * cg);
    }
    const int cnt = A.ocnt[ph];
    const int ov = (cnt > A.cap && A.ovf) ? A.ovf[ph] : -1;
    const int room = A.cap + (ov >= 0 ? kPBS * kPD - A.cap : 0);
    const int m = cnt < room ? cnt : room;
    if constexpr (PT) {
      const int64_t fp = A.first_pos[k];
      for (int i = lane; i < kPBS * 16; i += 64) {
        const int slot = i >> 4, l = i & 15;
        const int64_t tab = (int64_t)h * A.sc.rows + clamp_row(fp + slot, A.sc.rows);
        prow[slot * 16 + l] = tabs[tab].pf16[l];
      }
      pwave_sync();
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int rr = p * 4 + rw;
      const uint16_t* lb = PT ? prow + rr * 16 : kp + h * NL * SC + 8 * cg;
      uint32_t res[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t pr = 0;
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
          const int e = 2 * j + e2;
          const uint32_t c = (cw[p] >> (BITS * e)) & (NL - 1u);
          const uint16_t v = PT ? lb[c] : lb[c * SC + e];
          pr |= (uint32_t)v << (16 * e2);
        }
        res[j] = pr;
      }
      *reinterpret_cast<uint4*>(tile + rr * kPD + 8 * cg) = make_uint4(res[0], res[1], res[2], res[3]);
    }
    pwave_sync();
    for (int i = lane; i < m; i += 64) {
      const uint32_t e = *entry_ptr(const_cast<uint32_t*>(A.oent), const_cast<uint32_t*>(A.ovf_ent),
                                    ph, A.cap, ov, i);
      const uint32_t slot = e >> 24, ch = (e >> 16) & 255u;
      if (slot < (uint32_t)kPBS && ch < (uint32_t)kPD) tile[slot * kPD + ch] = (uint16_t)e;
    }
    pwave_sync();
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int rr = p * 4 + rw;
      *reinterpret_cast<uint4*>(ob + (int64_t)rr * H * kPD + 8 * cg) =
          *reinterpret_cast<const uint4*>(tile + rr * kPD + 8 * cg);
    }
    pwave_sync();
  }
}

}  // namespace

// Shape / pointer checks of a paged side (the host half of every paged call).
static int check_side(const hkv_paged_side* d, bool stats_allowed) {
  if (!d) return HKV_ERR_ARG;
  if (d->bits != 2 && d->bits != 4) return HKV_ERR_ARG;
  if (d->num_blocks < 0 || d->heads < 1 || d->heads > 16 || d->cap < 0 || d->cap > kPBS * kPD ||
      d->n_chunks < 0)
    return HKV_ERR_SHAPE;
  if (d->num_blocks * d->heads * kPBS * kPD >= ((int64_t)1 << 31)) return HKV_ERR_SHAPE;
  if (!d->codes || !d->ocnt || !d->status || (d->cap > 0 && !d->oent)) return HKV_ERR_ARG;
  if (d->ovf && (!d->ovf_next || (d->n_chunks > 0 && !d->ovf_ent))) return HKV_ERR_ARG;
  if ((d->kmin == nullptr) != (d->kmax == nullptr)) return HKV_ERR_ARG;
  if (d->kmin && !stats_allowed) return HKV_ERR_ARG;
  if ((((uintptr_t)d->codes) | ((uintptr_t)d->kmin) | ((uintptr_t)d->kmax)) & 15u) return HKV_ERR_ARG;
  return HKV_OK;
}

extern "C" int hkv_paged_write(const void* values, int64_t T, const hkv_nuq_scales* scales,
                               const int64_t* slot_mapping, const hkv_paged_side* side,
                               void* stream) {
  if (!scales || !scales->tables) return HKV_ERR_ARG;
  int rc = check_side(side, !scales->per_token);
  if (rc != HKV_OK) return rc;
  const int bits = side->bits, H = side->heads;
  if (scales->levels < 1 || scales->levels > (1 << bits)) return HKV_ERR_ARG;
  if (T < 0) return HKV_ERR_SHAPE;
  if (scales->per_token && scales->rows < 1) return HKV_ERR_SHAPE;
  if (T == 0 || side->num_blocks == 0) return HKV_OK;
  if (!values || !slot_mapping) return HKV_ERR_ARG;
  if ((uintptr_t)values & 15u) return HKV_ERR_ARG;
  PagedWriteArgs a;
  a.x = (const uint16_t*)values;
  a.T = T;
  a.H = H;
  a.sc = *scales;
  a.slots = slot_mapping;
  a.nslots = side->num_blocks * kPBS;
  a.codes = side->codes;
  a.ocnt = side->ocnt;
  a.oent = side->oent;
  a.cap = side->cap;
  a.kmin = side->kmin;
  a.kmax = side->kmax;
  a.status = side->status;
  a.nunits = ((T + kPBS - 1) / kPBS) * H;
  a.ovf = side->ovf;
  a.ovf_ent = side->ovf_ent;
  a.ovf_next = side->ovf_next;
  a.n_chunks = side->ovf ? side->n_chunks : 0;
  hipStream_t s = (hipStream_t)stream;
  const int nb = nb_for_levels_host(scales->levels);
  const bool stats = side->kmin != nullptr;
  if (scales->per_token) {
    if (bits == 4) launch_write_nb<true, 4, false>(nb, a, s);
    else launch_write_nb<true, 2, false>(nb < 2 ? nb : 2, a, s);
  } else if (bits == 4) {
    if (stats) launch_write_nb<false, 4, true>(nb, a, s);
    else launch_write_nb<false, 4, false>(nb, a, s);
  } else {
    if (stats) launch_write_nb<false, 2, true>(nb < 2 ? nb : 2, a, s);
    else launch_write_nb<false, 2, false>(nb < 2 ? nb : 2, a, s);
  }
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" int hkv_paged_gather(const hkv_paged_side* side, const hkv_nuq_scales* scales,
                                const int64_t* block_ids, const int64_t* first_pos, int64_t NK,
                                void* staging, void* stream) {
  if (!scales || !scales->tables) return HKV_ERR_ARG;
  int rc = check_side(side, true);
  if (rc != HKV_OK) return rc;
  const int bits = side->bits, H = side->heads;
  if (NK < 0) return HKV_ERR_SHAPE;
  if (scales->per_token && scales->rows < 1) return HKV_ERR_SHAPE;
  if (NK == 0) return HKV_OK;
  if (!block_ids || !staging || (scales->per_token && !first_pos)) return HKV_ERR_ARG;
  if ((uintptr_t)staging & 15u) return HKV_ERR_ARG;
  PagedGatherArgs a;
  a.codes = side->codes;
  a.ocnt = side->ocnt;
  a.oent = side->oent;
  a.cap = side->cap;
  a.NB = side->num_blocks;
  a.H = H;
  a.sc = *scales;
  a.ids = block_ids;
  a.first_pos = first_pos;
  a.NK = NK;
  a.out = (uint16_t*)staging;
  a.ovf = side->ovf;
  a.ovf_ent = side->ovf_ent;
  hipStream_t s = (hipStream_t)stream;
  const int NL = 1 << bits;
  const size_t lds = (size_t)kPW * kPBS * kPD * 2 +
                     (scales->per_token ? (size_t)kPW * kPBS * 16 * 2 : (size_t)H * NL * (kPD + 2) * 2);
  const int64_t items = NK * H;
  const unsigned grid = (unsigned)std::max<int64_t>(
      1, std::min<int64_t>((items + kPW - 1) / kPW, (int64_t)paged_num_cus() * 8));
#define HKV_PG(PT_, B_) \
  hipLaunchKernelGGL((paged_gather_kernel<PT_, B_>), dim3(grid), dim3(kPT), lds, s, a)
  if (scales->per_token) {
    if (bits == 4) HKV_PG(true, 4);
    else HKV_PG(true, 2);
  } else {
    if (bits == 4) HKV_PG(false, 4);
    else HKV_PG(false, 2);
  }
#undef HKV_PG
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
