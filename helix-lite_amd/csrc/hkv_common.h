// hkv_common.h -- device helpers shared by the helix-kv HIP kernels (gfx950).
//
// fp16 lanes are processed two at a time in 32-bit registers (packed 16-bit
// VALU ops); all float math that defines a result bit-for-bit is binary32 with
// explicit rounding (no fast-math, no contraction where it would matter).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/helix_kv.h"

#define HKV_DEV __device__ __forceinline__

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef short s2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u2_t __attribute__((ext_vector_type(2)));

HKV_DEV h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
HKV_DEV s2_t as_s2(uint32_t v) { return __builtin_bit_cast(s2_t, v); }
HKV_DEV uint32_t as_u32(h2_t v) { return __builtin_bit_cast(uint32_t, v); }
HKV_DEV uint32_t as_u32(s2_t v) { return __builtin_bit_cast(uint32_t, v); }
HKV_DEV uint32_t as_u32(u2_t v) { return __builtin_bit_cast(uint32_t, v); }

// ---------------------------------------------------------------- fp16 scalar

HKV_DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// float -> fp16 round-to-nearest-even (v_cvt_f16_f32 in the default mode).
HKV_DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Signed ordered key of an fp16 pattern: increasing in value, -0 just below +0.
HKV_DEV int32_t hkey(uint16_t h) {
  return (h & 0x8000u) ? -(int32_t)(h & 0x7fffu) - 1 : (int32_t)h;
}
HKV_DEV uint16_t hkey_inv(int32_t k) {
  return k >= 0 ? (uint16_t)k : (uint16_t)((((-(k + 1)) & 0x7fff)) | 0x8000);
}

HKV_DEV float load_scale(const void* p, int dt, int64_t i) {
  switch (dt) {
    case HKV_DT_F32: return ((const float*)p)[i];
    case HKV_DT_BF16: {
      uint32_t b = (uint32_t)((const uint16_t*)p)[i] << 16;
      return __builtin_bit_cast(float, b);
    }
    default: return h2f(((const uint16_t*)p)[i]);
  }
}

// ------------------------------------------------------- nearest-pole scan

// Strict-'<' ascending scan over fp32 |v - pole|; the lowest index wins ties.
// This is the defining semantics; the decision-table path below reproduces it.
HKV_DEV int scan_code(float v, const void* poles, int dt, int64_t base, int L) {
  float best = __builtin_inff();
  int idx = 0;
  for (int l = 0; l < L; ++l) {
    float d = __builtin_fabsf(__fsub_rn(v, load_scale(poles, dt, base + l)));
    if (d < best) { best = d; idx = l; }
  }
  return idx;
}

// -------------------------------------------------- packed fp16 comparisons

// Per 16-bit lane: 0xffff where a < b, 0 otherwise, for a, b finite fp16 (or
// b = +-inf).  The sign of the fp16 difference equals the sign of the exact
// difference; equal operands give +0.  Callers avoid the one case where a
// zero difference is -0 (a = -0, b = +0) by storing zero breakpoints as -0,
// zero lower thresholds as -0 and zero upper thresholds as +0.
HKV_DEV uint32_t lt2(uint32_t a, uint32_t b) {
  h2_t d = as_h2(a) - as_h2(b);
  return as_u32(as_s2(as_u32(d)) >> (s2_t){15, 15});
}

// Bitwise select: m ? a : b per bit, as one v_bfi_b32.  Written as inline
// asm: when m is a per-16-bit sign splat, the compiler otherwise rewrites the
// and/or form into per-half selects (two shifts, two v_cndmask and a v_perm).
HKV_DEV uint32_t bsel(uint32_t m, uint32_t a, uint32_t b) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(a), "v"(b));
  return r;
}

// Streaming (non-temporal) stores for outputs that are not re-read by the
// same kernel: the lines are written through L2 without displacing the
// kernel's input working set.
typedef unsigned int hkv_v4u __attribute__((ext_vector_type(4)));
HKV_DEV void store_stream(void* p, uint4 v) {
  const hkv_v4u x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<hkv_v4u*>(p));
}
HKV_DEV void store_stream(uint32_t* p, uint32_t v) { __builtin_nontemporal_store(v, p); }
HKV_DEV void store_stream(uint16_t* p, uint16_t v) { __builtin_nontemporal_store(v, p); }

// Streaming (non-temporal) loads for inputs read once: a large stream does
// not displace the kernel's small re-read working set (tables, counters).
template <typename LT>
HKV_DEV LT load_stream(const LT* p) {
  if constexpr (sizeof(LT) == 16) {
    return __builtin_bit_cast(LT, __builtin_nontemporal_load(reinterpret_cast<const hkv_v4u*>(p)));
  } else if constexpr (sizeof(LT) == 8) {
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(LT, __builtin_nontemporal_load(reinterpret_cast<const v2u*>(p)));
  } else if constexpr (sizeof(LT) == 4) {
    return __builtin_bit_cast(LT, __builtin_nontemporal_load(reinterpret_cast<const unsigned int*>(p)));
  } else {
    static_assert(sizeof(LT) == 2, "2, 4, 8 or 16 bytes");
    return __builtin_bit_cast(LT, __builtin_nontemporal_load(reinterpret_cast<const unsigned short*>(p)));
  }
}

// Pack the low halves of a and b into one register (a -> lane 0, b -> lane 1).
HKV_DEV uint32_t pack_lo(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }

// ------------------------------------------------------ decision tables

// Device image of one decision table (80 bytes; identical to the oracle's
// record and to HKV_TABLE_BYTES in the public header).
struct __attribute__((packed, aligned(16))) hkv_table_t {
  uint16_t bp[16];    // bp[c-1]: smallest fp16 x with code(x) >= c; +inf if none
  uint16_t pf16[16];  // fp16 value of each pole (dequantised value of a code)
  uint16_t lo, up;    // outlier iff x < lo || x > up
  uint16_t xsafe;     // fast path valid iff |x| <= xsafe
  uint16_t flags;     // bit 0: fast path usable
  uint16_t levels;
  uint16_t pad[3];
};
static_assert(sizeof(hkv_table_t) == 80, "table layout");

// Packed search state for two lanes (two tables, or one table broadcast).
template <int NB>  // number of search steps: levels <= 2^NB
struct Search2 {
  uint32_t bp[(1 << NB) - 1];  // breakpoint pairs
  uint32_t lo, up, xsafe;
};

// Code of two fp16 lanes by binary search over sorted breakpoints.  Returns the
// two codes in the low bits of each 16-bit lane.
//
// The code bits are the complements of the comparison masks.  v_bitop3 merges
// two masks at once: bitop3(A, B, K, 0x1B) is, per bit, K ? ~A : ~B.
HKV_DEV uint32_t not_sel(uint32_t a, uint32_t b, uint32_t k) { return __builtin_amdgcn_bitop3_b32(a, b, k, 0x1B); }

template <int NB>
HKV_DEV uint32_t search2(uint32_t x, const Search2<NB>& s) {
  if constexpr (NB == 0) {
    return 0u;
  } else if constexpr (NB == 1) {
    uint32_t m0 = lt2(x, s.bp[0]);
    return ~m0 & 0x00010001u;
  } else if constexpr (NB == 2) {
    uint32_t m1 = lt2(x, s.bp[1]);
    uint32_t t = bsel(m1, s.bp[0], s.bp[2]);
    uint32_t m0 = lt2(x, t);
    return not_sel(m1, m0, 0x00020002u) & 0x00030003u;
  } else if constexpr (NB == 3) {
    uint32_t m2 = lt2(x, s.bp[3]);
    uint32_t t1 = bsel(m2, s.bp[1], s.bp[5]);
    uint32_t q0 = bsel(m2, s.bp[0], s.bp[4]);
    uint32_t q1 = bsel(m2, s.bp[2], s.bp[6]);
    uint32_t m1 = lt2(x, t1);
    uint32_t t0 = bsel(m1, q0, q1);
    uint32_t m0 = lt2(x, t0);
    return ~((m2 & 0x00040004u) | (m1 & 0x00020002u) | (m0 & 0x00010001u)) & 0x00070007u;
  } else {
    static_assert(NB == 4, "at most 16 levels");
    uint32_t m3 = lt2(x, s.bp[7]);
    uint32_t t2 = bsel(m3, s.bp[3], s.bp[11]);
    uint32_t a = bsel(m3, s.bp[1], s.bp[9]);
    uint32_t b = bsel(m3, s.bp[5], s.bp[13]);
    uint32_t q0 = bsel(m3, s.bp[0], s.bp[8]);
    uint32_t q1 = bsel(m3, s.bp[2], s.bp[10]);
    uint32_t q2 = bsel(m3, s.bp[4], s.bp[12]);
    uint32_t q3 = bsel(m3, s.bp[6], s.bp[14]);
    uint32_t m2 = lt2(x, t2);
    uint32_t t1 = bsel(m2, a, b);
    uint32_t r0 = bsel(m2, q0, q2);
    uint32_t r1 = bsel(m2, q1, q3);
    uint32_t m1 = lt2(x, t1);
    uint32_t t0 = bsel(m1, r0, r1);
    uint32_t m0 = lt2(x, t0);
    return (not_sel(m3, m2, 0x00080008u) & 0x000c000cu) | (not_sel(m1, m0, 0x00020002u) & 0x00030003u);
  }
}

// Outlier mask (0xffff per lane) for two fp16 lanes: x < lo || x > up.
template <int NB>
HKV_DEV uint32_t outlier2(uint32_t x, const Search2<NB>& s) {
  return lt2(x, s.lo) | lt2(s.up, x);
}

// Outlier flags of two fp16 lanes in the sign bits (bit 15: lane 0, bit 31:
// lane 1; other bits are garbage): the sign of x - lo or of up - x.
template <int NB>
HKV_DEV uint32_t outlier2_sign(uint32_t x, const Search2<NB>& s) {
  const h2_t d1 = as_h2(x) - as_h2(s.lo), d2 = as_h2(s.up) - as_h2(x);
  return as_u32(d1) | as_u32(d2);
}

// Nonzero if some lane of x has |x| > xsafe (fast path not applicable).
// xsafe lanes are in [0, 0x7bff] or 0xffff (= -1: never applicable).
template <int NB>
HKV_DEV uint32_t unsafe2(uint32_t x, const Search2<NB>& s) {
  s2_t d = as_s2(s.xsafe) - as_s2(x & 0x7fff7fffu);
  return as_u32(d) & 0x80008000u;
}

// Load the search fields of one table into both lanes (broadcast).
template <int NB>
HKV_DEV void load_search_bcast(const hkv_table_t* t, Search2<NB>& s) {
  const uint4* p = reinterpret_cast<const uint4*>(t);
  uint4 a = p[0], b = p[1], c = p[4];
  uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < (1 << NB) - 1; ++i) {
    uint32_t h = (w[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
    s.bp[i] = h | (h << 16);
  }
  // record bytes 64..79: lo, up, xsafe, flags, levels, pad
  uint32_t lo = c.x & 0xffffu, up = c.x >> 16;
  uint32_t xs = c.y & 0xffffu, fl = c.y >> 16;
  if (!(fl & 1u)) xs = 0xffffu;
  s.lo = lo | (lo << 16);
  s.up = up | (up << 16);
  s.xsafe = xs | (xs << 16);
}

// Load two tables into the two lanes (lane 0 <- t0, lane 1 <- t1).
template <int NB>
HKV_DEV void load_search_pair(const hkv_table_t* t0, const hkv_table_t* t1, Search2<NB>& s) {
  const uint4* p0 = reinterpret_cast<const uint4*>(t0);
  const uint4* p1 = reinterpret_cast<const uint4*>(t1);
  uint4 a0 = p0[0], b0 = p0[1], c0 = p0[4];
  uint4 a1 = p1[0], b1 = p1[1], c1 = p1[4];
  uint32_t w0[8] = {a0.x, a0.y, a0.z, a0.w, b0.x, b0.y, b0.z, b0.w};
  uint32_t w1[8] = {a1.x, a1.y, a1.z, a1.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
  for (int i = 0; i < (1 << NB) - 1; ++i) {
    uint32_t h0 = (w0[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
    uint32_t h1 = (w1[i >> 1] >> ((i & 1) * 16)) & 0xffffu;
    s.bp[i] = h0 | (h1 << 16);
  }
  uint32_t xs0 = (c0.y >> 16) & 1u ? (c0.y & 0xffffu) : 0xffffu;
  uint32_t xs1 = (c1.y >> 16) & 1u ? (c1.y & 0xffffu) : 0xffffu;
  s.lo = (c0.x & 0xffffu) | (c1.x << 16);
  s.up = (c0.x >> 16) | (c1.x & 0xffff0000u);
  s.xsafe = xs0 | (xs1 << 16);
}

// ------------------------------------------------------------ misc helpers

HKV_DEV int nb_for_levels(int L) { return L <= 1 ? 0 : L <= 2 ? 1 : L <= 4 ? 2 : L <= 8 ? 3 : 4; }
inline int nb_for_levels_host(int L) { return L <= 1 ? 0 : L <= 2 ? 1 : L <= 4 ? 2 : L <= 8 ? 3 : 4; }

template <typename T>
HKV_DEV T wave_shfl_xor(T v, int m) {
  return __shfl_xor(v, m, 64);
}

#define HKV_CHECK_LAUNCH()                          \
  do {                                              \
    hipError_t e_ = hipGetLastError();              \
    if (e_ != hipSuccess) return HKV_ERR_LAUNCH;    \
  } while (0)
