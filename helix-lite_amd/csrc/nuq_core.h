// nuq_core.h -- per-thread nuq quantisation of 8 consecutive fp16 channels.
//
// Semantics (bit-exact with src/kvquant/triton_batched.py:53-82 / :204-232):
//   outlier = v > upper || v < lower           (fp32 compare)
//   code    = first argmin_l fl32(|v - pole_l|) (strict '<', ascending levels)
// Fast path: decision-table binary search on packed fp16 lanes (2 elements per
// VALU op).  Slow path (|v| beyond the table's safe range, NaN/inf, or a table
// that failed the exactness criterion): the scan itself.
#pragma once

#include "hkv_common.h"

struct SlowInfo {
  const void* poles;
  const void* upper;
  const void* lower;
  int pdt, tdt, L;
};

HKV_DEV SlowInfo slow_info(const hkv_nuq_scales& s) {
  return SlowInfo{s.poles, s.upper, s.lower, s.poles_dtype, s.thr_dtype, s.levels};
}

// The exact-scan inputs of a call site: a SlowInfo itself, or an object
// whose get() loads them where the rare exact scan needs them (so they are
// not held in registers across a kernel's main loop).
HKV_DEV const SlowInfo& slow_get(const SlowInfo& s) { return s; }
template <typename L>
HKV_DEV SlowInfo slow_get(const L& l) {
  return l.get();
}

HKV_DEV int64_t clamp_row(int64_t pos, int64_t rows) {
  return pos > rows - 1 ? rows - 1 : (pos < 0 ? 0 : pos);
}

// Position of token t for per-token scales.
HKV_DEV int64_t token_pos(const hkv_nuq_scales& s, int64_t t) {
  return s.positions ? s.positions[t] : s.pos_offset + t;
}

// Exact scan of one element; returns code and sets *o to the outlier flag.
HKV_DEV int slow_one(uint16_t xb, const SlowInfo& si, int64_t tab, int* o) {
  float v = h2f(xb);
  float up = load_scale(si.upper, si.tdt, tab), lo = load_scale(si.lower, si.tdt, tab);
  *o = (v > up) || (v < lo);
  return scan_code(v, si.poles, si.pdt, tab * si.L, si.L);
}

// Quantise 8 channels.  PT (per-token): S[0] holds the row's table broadcast;
// otherwise S[j] holds the tables of channel pair j.  tab(e) gives the table
// index of element e (0..7); it is evaluated only on the exact-scan path.
// code[j]: codes of elements 2j, 2j+1 in bits 0..3 / 16..19; om[j]: 0xffff lanes
// for outliers.
template <int NB, bool PT, typename TabFn>
HKV_DEV void quant8(const uint4 xv, const Search2<NB>* S, const SlowInfo& si, TabFn tab,
                    uint32_t code[4], uint32_t om[4]) {
  const uint32_t x[4] = {xv.x, xv.y, xv.z, xv.w};
  uint32_t uns = 0;
  if constexpr (PT) {  // one bound: compare the largest magnitude
    u2_t mg = __builtin_bit_cast(u2_t, x[0] & 0x7fff7fffu);
#pragma unroll
    for (int j = 1; j < 4; ++j) mg = __builtin_elementwise_max(mg, __builtin_bit_cast(u2_t, x[j] & 0x7fff7fffu));
    uns = unsafe2<NB>(__builtin_bit_cast(uint32_t, mg), S[0]);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) uns |= unsafe2<NB>(x[j], S[j]);
  }
  if (__builtin_expect(uns == 0, 1)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      code[j] = search2<NB>(x[j], S[PT ? 0 : j]);
      om[j] = outlier2<NB>(x[j], S[PT ? 0 : j]);
    }
  } else {
#pragma unroll 1
    for (int j = 0; j < 4; ++j) {
      int o0, o1;
      int c0 = slow_one((uint16_t)(x[j] & 0xffffu), si, tab(2 * j), &o0);
      int c1 = slow_one((uint16_t)(x[j] >> 16), si, tab(2 * j + 1), &o1);
      code[j] = (uint32_t)c0 | ((uint32_t)c1 << 16);
      om[j] = (o0 ? 0xffffu : 0u) | (o1 ? 0xffff0000u : 0u);
    }
  }
}

// The smallest fast-path bound of four channel-pair tables, in both halves
// (bounds are in [0, 0x7bff], or 0xffff = -1 when a table has no fast path).
template <int NB>
HKV_DEV uint32_t xsafe_min(const Search2<NB>* S) {
  s2_t m = as_s2(S[0].xsafe);
#pragma unroll
  for (int j = 1; j < 4; ++j) m = __builtin_elementwise_min(m, as_s2(S[j].xsafe));
  const short lo = m.x < m.y ? m.x : m.y;
  return (uint32_t)(uint16_t)lo * 0x00010001u;
}

// Per-channel tables: element e of the chunk starting at table index tab0.
struct ChanTab {
  int64_t tab0;
  HKV_DEV int64_t operator()(int e) const { return tab0 + e; }
};
// Per-token tables: one table for the whole row.
struct RowTab {
  int64_t tab;
  HKV_DEV int64_t operator()(int) const { return tab; }
};
// The same, computed from (head, token) where it is needed.
struct RowTabAt {
  int64_t rows;
  const int64_t* positions;
  int64_t pos_offset;
  int h;
  int64_t t;
  HKV_DEV int64_t operator()(int) const {
    const int64_t pos = positions ? positions[t] : pos_offset + t;
    return (int64_t)h * rows + clamp_row(pos, rows);
  }
};

// Two 16-bit lanes holding small values -> two bytes (lane0 -> byte0).
HKV_DEV uint32_t lanes_to_bytes(uint32_t v) { return (v & 0xffu) | ((v >> 8) & 0xff00u); }

// 8 codes (4 regs) -> 32 bits of nibbles, element e at bits 4e..4e+3.
HKV_DEV uint32_t pack_nibbles(const uint32_t c[4]) {
  uint32_t r = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) r |= ((c[j] & 0xfu) | ((c[j] >> 12) & 0xf0u)) << (8 * j);
  return r;
}

// 8 codes -> 16 bits of crumbs, element e at bits 2e..2e+1.
HKV_DEV uint32_t pack_crumbs(const uint32_t c[4]) {
  uint32_t r = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) r |= ((c[j] & 0x3u) | ((c[j] >> 14) & 0xcu)) << (4 * j);
  return r;
}

// 8 outlier lane masks -> 8-bit mask, element e at bit e.
HKV_DEV uint32_t mask_bits(const uint32_t om[4]) {
  uint32_t r = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) r |= ((om[j] & 1u) | ((om[j] >> 15) & 2u)) << (2 * j);
  return r;
}

// ------------------------------------------- packed output by bit placement
//
// The search yields one full-lane mask per code bit (0xffff in a 16-bit lane
// where that bit of the lane's code is 0).  Each bit is moved straight to its
// place in the packed output by one v_bitop3 against a constant position
// mask, so no code is ever formed in a lane and then shifted into place.

// Per bit: p ? v : acc.
HKV_DEV uint32_t place(uint32_t p, uint32_t v, uint32_t acc) {
  return __builtin_amdgcn_bitop3_b32(p, v, acc, 0xCA);
}
// Per bit: p ? ~m : acc.
HKV_DEV uint32_t place_not(uint32_t p, uint32_t m, uint32_t acc) {
  return __builtin_amdgcn_bitop3_b32(p, m, acc, 0x3A);
}

// Masks of the code bits of two fp16 lanes: m[b] is 0xffff in a lane whose
// code has bit b clear (the same binary search as search2).
template <int NB>
HKV_DEV void search_masks(uint32_t x, const Search2<NB>& s, uint32_t m[NB]) {
  if constexpr (NB == 2) {
    m[1] = lt2(x, s.bp[1]);
    m[0] = lt2(x, bsel(m[1], s.bp[0], s.bp[2]));
  } else {
    static_assert(NB == 4, "placement is used for 4 and 16 levels");
    m[3] = lt2(x, s.bp[7]);
    const uint32_t t2 = bsel(m[3], s.bp[3], s.bp[11]);
    const uint32_t a = bsel(m[3], s.bp[1], s.bp[9]);
    const uint32_t b = bsel(m[3], s.bp[5], s.bp[13]);
    const uint32_t q0 = bsel(m[3], s.bp[0], s.bp[8]);
    const uint32_t q1 = bsel(m[3], s.bp[2], s.bp[10]);
    const uint32_t q2 = bsel(m[3], s.bp[4], s.bp[12]);
    const uint32_t q3 = bsel(m[3], s.bp[6], s.bp[14]);
    m[2] = lt2(x, t2);
    const uint32_t t1 = bsel(m[2], a, b);
    const uint32_t r0 = bsel(m[2], q0, q2);
    const uint32_t r1 = bsel(m[2], q1, q3);
    m[1] = lt2(x, t1);
    m[0] = lt2(x, bsel(m[1], r0, r1));
  }
}

// Position masks.  Element e = 2j (low lane of pair j) and e = 2j + 1 (high
// lane).  Packed codes:
//   2-bit: element e's bit b at bit 2e + b of the 16-bit word.  The low lane
//     places it directly (bit 4j + b); the high lane at 16 + 4j + 2 + b,
//     brought down by acc | acc >> 16.
//   4-bit: element e's bit b at bit 4e + b of the 32-bit word, built from two
//     accumulators (pairs 0-1 and 2-3), each a 16-bit half in the same way:
//     low lane at 8(j & 1) + b, high lane at 16 + 8(j & 1) + 4 + b.
// Outlier flags: element e at bit e of the 8-bit mask: low lane at 2j, high
// lane at 16 + 2j + 1.
HKV_DEV constexpr uint32_t pos2(int j, int b) { return (1u << (4 * j + b)) | (1u << (16 + 4 * j + 2 + b)); }
HKV_DEV constexpr uint32_t pos4(int j, int b) {
  return (1u << (8 * (j & 1) + b)) | (1u << (16 + 8 * (j & 1) + 4 + b));
}
HKV_DEV constexpr uint32_t posm(int j) { return (1u << (2 * j)) | (1u << (16 + 2 * j + 1)); }

// Quantise 8 channels straight into packed form: *packed receives the 8
// codes packed at BITS bits (element e at bits BITS*e..; for BITS = 2 only
// the low 16 bits are meaningful), *mask8 the 8-bit outlier mask (element e
// at bit e).  Same semantics and fast/exact split as quant8.
//
// XMIN (per-channel tables): the fast path is taken when the largest |x| of
// the 8 elements is within xmin, the smallest bound of the 8 tables (see
// xsafe_min), instead of comparing each pair with its own bounds.  Never less
// exact: the scan decides whatever the fast path does not.
template <int NB, bool PT, int BITS, typename TabFn, bool XMIN = false, typename SI = SlowInfo>
HKV_DEV void quant8_packed(const uint4 xv, const Search2<NB>* S, const SI& slow, TabFn tab,
                           uint32_t* packed, uint32_t* mask8, uint32_t xmin = 0) {
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
      const uint32_t o = as_u32(as_s2(outlier2_sign<NB>(x[j], S[PT ? 0 : j])) >> (s2_t){15, 15});
      M = place(posm(j), o, M);
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
  } else {
    const SlowInfo si = slow_get(slow);
    uint32_t c[4], om[4];
#pragma unroll 1
    for (int j = 0; j < 4; ++j) {
      int o0, o1;
      int c0 = slow_one((uint16_t)(x[j] & 0xffffu), si, tab(2 * j), &o0);
      int c1 = slow_one((uint16_t)(x[j] >> 16), si, tab(2 * j + 1), &o1);
      c[j] = (uint32_t)c0 | ((uint32_t)c1 << 16);
      om[j] = (o0 ? 0xffffu : 0u) | (o1 ? 0xffff0000u : 0u);
    }
    *packed = BITS == 4 ? pack_nibbles(c) : pack_crumbs(c);
    *mask8 = mask_bits(om);
  }
}

// Wave-wide inclusive prefix sum with the adds fused into DPP (one
// v_add_u32_dpp per step).  Every lane of the wave must be active.  Each step
// reads the previous step's result through DPP, which needs two wait states
// after the VALU write (s_nop 1).
HKV_DEV uint32_t wave_incl_sum_fused(uint32_t v) {
  asm("s_nop 1\n\t"
      "v_add_u32_dpp %0, %0, %0 row_shr:1 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_add_u32_dpp %0, %0, %0 row_shr:2 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_add_u32_dpp %0, %0, %0 row_shr:4 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_add_u32_dpp %0, %0, %0 row_shr:8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
      "s_nop 1\n\t"
      "v_add_u32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_add_u32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
      "s_nop 1"
      : "+v"(v));
  return v;
}

HKV_DEV uint32_t wave_excl_count_fused(uint32_t cnt, uint32_t* total) {
  const uint32_t inc = wave_incl_sum_fused(cnt);
  *total = (uint32_t)__builtin_amdgcn_readlane((int)inc, 63);
  return inc - cnt;
}
