// quest.hip -- Quest page metadata, upper-bound scoring and top-K selection.
//
// Reference semantics: src/quest/reference.py:38-133 (stats, bound, top-K with
// sinks), src/quest/triton_kernels.py:25-57 (fused bound, fp16 out),
// src/kvquant/quest_selector.py:64-78 (selector path).
//
// Canonical bound evaluation (fixed so that the selected page sets are exact):
// channels in chunks of 8, one lane per chunk; a lane sums its chunk left to
// right (positive part sum_d clamp(q,0)*kmax and negative part
// sum_d clamp(q,max=0)*kmin kept apart, products rounded before the add); the
// chunk sums are combined by a xor-butterfly over the row's lanes (offsets
// n/2 ... 1); bound = pos + neg, then + 0.0f so a zero bound is +0.
#include "hkv_common.h"

#include <mutex>
#include <type_traits>

namespace {

// --------------------------------------------------------------- a8: stats

// Ordered fp16 keys on both lanes: x ^ ((x >> 15) & 0x7fff) (an involution).
HKV_DEV uint32_t key2(uint32_t x) {
  const uint32_t s = as_u32(as_s2(x) >> (s2_t){15, 15});
  return x ^ (s & 0x7fff7fffu);
}
HKV_DEV uint32_t min2(uint32_t a, uint32_t b) {
  s2_t x = as_s2(a), y = as_s2(b);
  return as_u32((s2_t){x.x < y.x ? x.x : y.x, x.y < y.y ? x.y : y.y});
}
HKV_DEV uint32_t max2(uint32_t a, uint32_t b) {
  s2_t x = as_s2(a), y = as_s2(b);
  return as_u32((s2_t){x.x > y.x ? x.x : y.x, x.y > y.y ? x.y : y.y});
}
// 0xffff lanes where the fp16 value is NaN.
HKV_DEV uint32_t nan2(uint32_t x) {
  s2_t d = (s2_t){0x7c00, 0x7c00} - as_s2(x & 0x7fff7fffu);
  return as_u32(d >> (s2_t){15, 15});
}

// fp16 (P,S,H,D), D % 8 == 0: one thread per 8 channels of one (page, head).
__global__ void __launch_bounds__(256)
page_stats_f16(const uint16_t* __restrict__ K, int64_t P, int S, int H, int D,
               uint16_t* __restrict__ kmin, uint16_t* __restrict__ kmax) {
  const int64_t HD8 = (int64_t)H * D / 8;
  const int64_t n = P * HD8;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t p = i / HD8, j = i - p * HD8;
    const uint4* src = reinterpret_cast<const uint4*>(K + (p * S) * H * D) + j;
    uint32_t mn[4], mx[4], nn[4] = {0, 0, 0, 0};
    const uint4 v0 = src[0];
    const uint32_t w0[4] = {v0.x, v0.y, v0.z, v0.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) { mn[q] = mx[q] = key2(w0[q]); nn[q] = nan2(w0[q]); }
    for (int s = 1; s < S; ++s) {
      const uint4 v = src[(int64_t)s * HD8];
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t k = key2(w[q]);
        mn[q] = min2(mn[q], k);
        mx[q] = max2(mx[q], k);
        nn[q] |= nan2(w[q]);
      }
    }
    uint32_t a[4], b[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      a[q] = bsel(nn[q], 0x7e007e00u, key2(mn[q]));
      b[q] = bsel(nn[q], 0x7e007e00u, key2(mx[q]));
    }
    reinterpret_cast<uint4*>(kmin)[i] = make_uint4(a[0], a[1], a[2], a[3]);
    reinterpret_cast<uint4*>(kmax)[i] = make_uint4(b[0], b[1], b[2], b[3]);
  }
}

HKV_DEV int32_t fkey(float f) {
  const int32_t b = __builtin_bit_cast(int32_t, f);
  return b >= 0 ? b : (b ^ 0x7fffffff);
}

// Any dtype/D: one thread per (page, head, channel).
template <typename T>
__global__ void __launch_bounds__(256)
page_stats_generic(const T* __restrict__ K, int64_t P, int S, int H, int D, T* __restrict__ kmin,
                   T* __restrict__ kmax) {
  const int64_t HD = (int64_t)H * D;
  const int64_t n = P * HD;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int64_t p = i / HD, j = i - p * HD;
    const T* src = K + p * S * HD + j;
    float v = (float)src[0];
    float mn = v, mx = v;
    bool nan = __builtin_isnan(v);
    for (int s = 1; s < S; ++s) {
      v = (float)src[(int64_t)s * HD];
      nan |= __builtin_isnan(v);
      if (fkey(v) < fkey(mn)) mn = v;
      if (fkey(v) > fkey(mx)) mx = v;
    }
    if (nan) mn = mx = __builtin_nanf("");
    kmin[i] = (T)mn;
    kmax[i] = (T)mx;
  }
}

// --------------------------------------------------------------- a9: bound

// Ordered key: NaN above +inf, -0 == +0.
HKV_DEV uint32_t ukey(float f) {
  if (__builtin_isnan(f)) return 0xffffffffu;
  if (f == 0.0f) f = 0.0f;
  const uint32_t b = __builtin_bit_cast(uint32_t, f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

HKV_DEV float clamp_pos(float q) { return q < 0.0f ? 0.0f : q; }
HKV_DEV float clamp_neg(float q) { return q > 0.0f ? 0.0f : q; }

// The fp32 product of q and the fp16 half HI of w, rounded once: one
// v_fma_mix_f32 with addend -0 (x + -0 == x for every x, +0 included), instead
// of a conversion and a multiply.
template <int HI>
HKV_DEV float mul_f16(uint32_t w, float q) {
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(q), "v"(-0.0f));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(q), "v"(-0.0f));
  return r;
}

template <typename KT> HKV_DEV float kval(KT v);
template <> HKV_DEV float kval<uint16_t>(uint16_t v) { return h2f(v); }
template <> HKV_DEV float kval<float>(float v) { return v; }

// Chunk c (8 channels) of one row: positive and negative partial sums.
template <typename KT>
HKV_DEV void chunk_sums(const KT* __restrict__ mn_row, const KT* __restrict__ mx_row, int D, int c,
                        const float* qp, const float* qn, float& ps, float& ns) {
  ps = 0.0f;
  ns = 0.0f;
  const int d0 = 8 * c;
  if (d0 >= D) return;
  KT a[8], b[8];
  if (D % 8 == 0) {
    if constexpr (sizeof(KT) == 2) {
      *reinterpret_cast<uint4*>(a) = *reinterpret_cast<const uint4*>(mn_row + d0);
      *reinterpret_cast<uint4*>(b) = *reinterpret_cast<const uint4*>(mx_row + d0);
    } else {
      reinterpret_cast<uint4*>(a)[0] = reinterpret_cast<const uint4*>(mn_row + d0)[0];
      reinterpret_cast<uint4*>(a)[1] = reinterpret_cast<const uint4*>(mn_row + d0)[1];
      reinterpret_cast<uint4*>(b)[0] = reinterpret_cast<const uint4*>(mx_row + d0)[0];
      reinterpret_cast<uint4*>(b)[1] = reinterpret_cast<const uint4*>(mx_row + d0)[1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = d0 + i < D ? mn_row[d0 + i] : (KT)0;
      b[i] = d0 + i < D ? mx_row[d0 + i] : (KT)0;
    }
  }
  const int nd = D - d0 < 8 ? D - d0 : 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i < nd) {
      ps = __fadd_rn(ps, __fmul_rn(qp[i], kval<KT>(b[i])));
      ns = __fadd_rn(ns, __fmul_rn(qn[i], kval<KT>(a[i])));
    }
  }
}

// Butterfly over n lanes (n | 64, lanes of a row contiguous and aligned).
HKV_DEV float row_reduce(float v, int n) {
  for (int off = n >> 1; off >= 1; off >>= 1) v = __fadd_rn(v, __shfl_xor(v, off, 64));
  return v;
}

// The same butterfly as row_reduce(v, 16) on DPP moves instead of LDS
// permutes: row_ror:8 is xor 8; after it the values are symmetric under xor 8,
// so row_ror:4 reads the xor-4 partner's value; quad_perm gives xor 2 and
// xor 1.  Each step adds the same two operands as the xor butterfly (IEEE
// addition is commutative), so the sum is bit-identical.
template <int CTRL>
HKV_DEV float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xf, 0xf, false));
}
HKV_DEV float row16_reduce(float v) {
  v = __fadd_rn(v, dpp_f<0x128>(v));  // row_ror:8
  v = __fadd_rn(v, dpp_f<0x124>(v));  // row_ror:4
  v = __fadd_rn(v, dpp_f<0x4e>(v));   // quad_perm [2,3,0,1]
  v = __fadd_rn(v, dpp_f<0xb1>(v));   // quad_perm [1,0,3,2]
  return v;
}

// Integer wave reductions and scans on DPP moves (no LDS permutes): rows of
// 16 lanes by row_ror / quad_perm (every lane ends with its row's value) or
// by row_shr (a lane reads the lane n below it, 0 past the row start), then
// the four rows combined through readlane.
template <int CTRL>
HKV_DEV uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
HKV_DEV uint32_t rl_u(uint32_t v, int lane) { return (uint32_t)__builtin_amdgcn_readlane((int)v, lane); }
HKV_DEV uint32_t wave_sum_u(uint32_t v) {  // same value in every lane
  v += dpp_u<0x128>(v);
  v += dpp_u<0x124>(v);
  v += dpp_u<0x4e>(v);
  v += dpp_u<0xb1>(v);
  return rl_u(v, 0) + rl_u(v, 16) + rl_u(v, 32) + rl_u(v, 48);
}
HKV_DEV uint32_t min_u(uint32_t a, uint32_t b) { return a < b ? a : b; }
HKV_DEV uint32_t max_u(uint32_t a, uint32_t b) { return a > b ? a : b; }
HKV_DEV uint32_t wave_min_u(uint32_t v) {
  v = min_u(v, dpp_u<0x128>(v));
  v = min_u(v, dpp_u<0x124>(v));
  v = min_u(v, dpp_u<0x4e>(v));
  v = min_u(v, dpp_u<0xb1>(v));
  return min_u(min_u(rl_u(v, 0), rl_u(v, 16)), min_u(rl_u(v, 32), rl_u(v, 48)));
}
HKV_DEV uint32_t wave_max_u(uint32_t v) {
  v = max_u(v, dpp_u<0x128>(v));
  v = max_u(v, dpp_u<0x124>(v));
  v = max_u(v, dpp_u<0x4e>(v));
  v = max_u(v, dpp_u<0xb1>(v));
  return max_u(max_u(rl_u(v, 0), rl_u(v, 16)), max_u(rl_u(v, 32), rl_u(v, 48)));
}
HKV_DEV uint32_t wave_incl_scan_u(uint32_t x) {  // lane order
  x += dpp_u<0x111>(x);  // row_shr:1
  x += dpp_u<0x112>(x);  // row_shr:2
  x += dpp_u<0x114>(x);  // row_shr:4
  x += dpp_u<0x118>(x);  // row_shr:8: x = sum of the row's lanes up to this one
  const uint32_t t0 = rl_u(x, 15), t1 = rl_u(x, 31), t2 = rl_u(x, 47);
  const int row = (threadIdx.x & 63) >> 4;
  return x + (row >= 1 ? t0 : 0u) + (row >= 2 ? t1 : 0u) + (row >= 3 ? t2 : 0u);
}

HKV_DEV int lanes_for(int D) {
  int nch = (D + 7) / 8, n = 1;
  while (n < nch) n <<= 1;
  return n;
}

// q (Hq,D) -> per KV head clamp(q,0) / clamp(q,max=0) summed over its group in
// ascending head order (group == 1: the clamps themselves).
HKV_DEV void group_q(const void* q, int qdt, int g, int group, int D, int d, float& qp, float& qn) {
  float a = 0.0f, b = 0.0f;
  for (int j = 0; j < group; ++j) {
    const float v = load_scale(q, qdt, (int64_t)(g * group + j) * D + d);
    a = __fadd_rn(a, clamp_pos(v));
    b = __fadd_rn(b, clamp_neg(v));
  }
  qp = a;
  qn = b;
}

// Standalone bound: rows r = p*H + h; n lanes per row; q staged in LDS; each
// thread has the loads of kBoundUnroll rows in flight.
constexpr int kBoundUnroll = 4;

template <typename KT>
__global__ void __launch_bounds__(256)
bound_kernel(const void* q, int qdt, int group, const KT* __restrict__ kmin,
             const KT* __restrict__ kmax, int64_t P, int H, int D, void* out, int odt,
             int head_major, const int64_t* __restrict__ page_ids, int64_t nstat) {
  extern __shared__ float qs[];  // [2][H][D]
  for (int i = threadIdx.x; i < H * D; i += 256) {
    float a, b;
    group_q(q, qdt, i / D, group, D, i % D, a, b);
    qs[i] = a;
    qs[H * D + i] = b;
  }
  __syncthreads();
  const int n = lanes_for(D);
  const int rows_per_block = 256 / n;
  const int c = threadIdx.x % n;
  const int64_t nrows = P * H;
  const int64_t span = (int64_t)rows_per_block * kBoundUnroll;
  for (int64_t r0 = (int64_t)blockIdx.x * span; r0 < nrows; r0 += (int64_t)gridDim.x * span) {
    float ps[kBoundUnroll], ns[kBoundUnroll];
#pragma unroll
    for (int u = 0; u < kBoundUnroll; ++u) {
      const int64_t r = r0 + (int64_t)u * rows_per_block + threadIdx.x / n;
      ps[u] = 0.0f;
      ns[u] = 0.0f;
      if (r < nrows) {
        const int h = (int)(r % H);
        float qp[8], qn[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int d = 8 * c + i;
          qp[i] = d < D ? qs[h * D + d] : 0.0f;
          qn[i] = d < D ? qs[H * D + h * D + d] : 0.0f;
        }
        int64_t src = r;
        if (page_ids) {
          const int64_t id = page_ids[r / H];
          // a page id outside the statistics gets bound -inf (never preferred)
          src = (id >= 0 && id < nstat) ? id * H + h : -1;
        }
        if (src >= 0) chunk_sums<KT>(kmin + src * D, kmax + src * D, D, c, qp, qn, ps[u], ns[u]);
        else { ps[u] = -__builtin_inff(); ns[u] = 0.0f; }
      }
    }
#pragma unroll
    for (int u = 0; u < kBoundUnroll; ++u) {
      const int64_t r = r0 + (int64_t)u * rows_per_block + threadIdx.x / n;
      const float a = row_reduce(ps[u], n);
      const float b2 = row_reduce(ns[u], n);
      if (r < nrows && c == 0) {
        const float b = __fadd_rn(__fadd_rn(a, b2), 0.0f);
        const int64_t o = head_major ? (r % H) * P + r / H : r;
        if (odt == HKV_DT_F16) ((uint16_t*)out)[o] = f2h(b);
        else ((float*)out)[o] = b;
      }
    }
  }
}

constexpr int kMaxMMHeads = 64;  // heads with per-block key ranges (multi-block top-K)
constexpr int kPidStage = 2048;  // block-table ids a bound block stages in LDS
constexpr int kBoundUnrollF16 = 2;  // row groups per step (two steps of loads in flight)

// A lane's statistics are read once: load_stream keeps the 128 MiB stream
// from displacing the cached query, scores and key ranges (44.9 against
// 48.0 us per 1M-token selection, which also measured 2 row groups per step
// against 4 at 4 blocks per CU).

// fp16 stats with D = 8*G (G a power of two, G <= 64): lane c of a row owns
// channels [8c, 8c+8) and loads them with one 128-bit load per array.  HFIX:
// the rows of one wave (64/G) are a multiple of H, so a lane's head is fixed
// and its clamped query sums live in registers.  Same summation order as
// bound_kernel.
// out_p / out_off: head-major output goes to out[h * out_p + out_off + p]
// (out_p = P, out_off = 0 for one sequence; the ragged kernel writes each
// sequence's pages at its offset within the concatenated page axis).
// q_lds: the raw query (H*group*D elements, at most kQRawChunks*256 16-byte
// chunks, 16-byte aligned) is staged through LDS after qs; its loads are
// issued before the first two steps of statistics loads, so the group sums
// wait only for them.
constexpr int kQRawChunks = 4;

// U8: the statistics are u8 codes of the compact page metadata, read as
// fl(lo + fl(code * step)) with lo / step per (head, channel) (dq_lo,
// dq_step); a lane's head is fixed (HFIX), so its 8 channels' lo / step are
// loaded once.  The products and the order are the fp16 path's.
template <int G, bool HFIX, bool U8 = false>
HKV_DEV void bound_f16_rows(const void* q, int qdt, int group, const void* kmin_v,
                            const void* kmax_v, int64_t P, int H, void* out, int odt,
                            int head_major, int64_t out_p, int64_t out_off, int bx, int gx,
                            uint2* __restrict__ mm = nullptr, int q_lds = 0,
                            const float* __restrict__ dq_lo = nullptr,
                            const float* __restrict__ dq_step = nullptr,
                            const int64_t* __restrict__ pids = nullptr, int64_t nstat = 0) {
  static_assert(!U8 || HFIX, "u8 statistics need a fixed head per lane");
  using ET = typename std::conditional<U8, uint8_t, uint16_t>::type;  // one statistic
  using LT = typename std::conditional<U8, uint2, uint4>::type;       // a lane's 8 channels
  const ET* __restrict__ kmin = static_cast<const ET*>(kmin_v);
  const ET* __restrict__ kmax = static_cast<const ET*>(kmax_v);
  constexpr int D = 8 * G;
  constexpr int RB = 256 / G;  // rows per block per row group
  constexpr int U = kBoundUnrollF16;
  constexpr int span = RB * U;  // rows per block per step
  extern __shared__ float qs[];  // [2][H][D]
  const int c = threadIdx.x % G, rl = threadIdx.x / G;
  // 32-bit row arithmetic (P * H < 2^31 is checked by the host); with HFIX
  // the page of a row advances by a constant per step (H divides RB), so no
  // division is needed in the loop.
  const int nr = (int)(P * H);
  // No rows (an empty sequence of a ragged batch): nothing to load.  The loads
  // below clamp to row nr - 1, which must exist.  Uniform over the block.
  if (nr <= 0) return;
  const int step = gx * span;  // block bx of gx over these rows
  LT a0[U], b0[U], a1[U], b1[U];
  // Loads are unconditional, rows past the end clamped to the last row (their
  // results are not written): a fixed number of loads per step lets the
  // compiler wait for exactly one step's loads while the next step's are in
  // flight.
  // pids (HFIX only): page p's statistics are row pids[p] of (nstat, H, D)
  // -- a block table mapping the logical pages scored here to the pool's
  // blocks; an id outside [0, nstat) reads block 0.  The block's ids (span / H
  // consecutive pages per step) are staged in LDS first, -1 for an id outside
  // the statistics, so a step's statistics loads never wait on its id loads
  // (up to kPidStage ids a block; beyond, each load reads its id itself).
  __shared__ int s_pid[kPidStage];
  const int pps = span / H;  // pages per step (H divides RB)
  const int nsteps = nr > bx * span ? (nr - bx * span + step - 1) / step : 0;
  const bool pid_lds = HFIX && pids && nsteps * pps <= kPidStage;
  if (pid_lds) {
    for (int i = threadIdx.x; i < nsteps * pps; i += 256) {
      const int st = i / pps;
      int p = (bx * span + st * step) / H + (i - st * pps);
      p = p < (int)P ? p : (int)P - 1;
      const int64_t bk = pids[p];
      s_pid[i] = (bk < 0 || bk >= nstat) ? -1 : (int)bk;
    }
    __syncthreads();
  }
  auto load = [&](int r0, int sl, LT (&a)[U], LT (&b)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int r = r0 + u * RB + rl;
      r = r < nr ? r : nr - 1;
      if constexpr (HFIX) {
        if (pid_lds) {  // a step past the block's last (clamped rows) reads its last id
          const int bk = s_pid[sl < nsteps ? sl * pps + u * (RB / H) + rl / H : nsteps * pps - 1];
          r = (bk < 0 ? 0 : bk) * H + rl % H;
        } else if (pids) {  // r0 is a multiple of H, and so is RB
          int p = r0 / H + u * (RB / H) + rl / H;
          p = p < (int)P ? p : (int)P - 1;
          int64_t bk = pids[p];
          bk = (bk < 0 || bk >= nstat) ? 0 : bk;
          r = (int)bk * H + rl % H;
        }
      }
      a[u] = load_stream(reinterpret_cast<const LT*>(kmin + (uint32_t)r * D) + c);
      b[u] = load_stream(reinterpret_cast<const LT*>(kmax + (uint32_t)r * D) + c);
    }
  };
  int r0 = bx * span, sl = 0;
  // the block's clamped, group-summed query, [2][H][D] in LDS
  if (q_lds) {
    // raw query chunks first, then two steps of statistics: waiting for the
    // chunks (loads complete in order) does not wait for the statistics
    const int nch = H * group * D * (qdt == HKV_DT_F32 ? 4 : 2) / 16;
    const uint4* gq = reinterpret_cast<const uint4*>(q);
    uint4* qraw = reinterpret_cast<uint4*>(qs + 2 * H * D);
    uint4 qc[kQRawChunks];
#pragma unroll
    for (int k = 0; k < kQRawChunks; ++k) {
      const int i = threadIdx.x + 256 * k;
      qc[k] = gq[i < nch ? i : nch - 1];
    }
    load(r0, 0, a0, b0);
    load(r0 + step, 1, a1, b1);
    // unconditional stores (a clamped chunk rewrites the last one with its
    // own value), so the chunk loads stay ahead of the statistics loads
#pragma unroll
    for (int k = 0; k < kQRawChunks; ++k) {
      const int i = threadIdx.x + 256 * k;
      qraw[i < nch ? i : nch - 1] = qc[k];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < H * D; i += 256) {
      float qa, qb;
      group_q(qraw, qdt, i / D, group, D, i % D, qa, qb);
      qs[i] = qa;
      qs[H * D + i] = qb;
    }
  } else {
    load(r0, 0, a0, b0);
    load(r0 + step, 1, a1, b1);
    for (int i = threadIdx.x; i < H * D; i += 256) {
      float qa, qb;
      group_q(q, qdt, i / D, group, D, i % D, qa, qb);
      qs[i] = qa;
      qs[H * D + i] = qb;
    }
  }
  __syncthreads();
  float qp[8], qn[8];
  if constexpr (HFIX) {
    const int h = rl % H;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qp[i] = qs[h * D + 8 * c + i];
      qn[i] = qs[H * D + h * D + 8 * c + i];
    }
  }
  float dlo[8], dst[8];  // U8: the lane's channels' lo / step
  if constexpr (U8) {
    const int h = rl % H;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      dlo[i] = dq_lo[h * D + 8 * c + i];
      dst[i] = dq_step[h * D + 8 * c + i];
    }
  }
  uint32_t kmn_t = 0xffffffffu, kmx_t = 0u;  // key range of this thread's rows (HFIX: one head)
  auto compute = [&](int rs, int pb, int sl, const LT (&a)[U], const LT (&b)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = rs + u * RB + rl;
      int h, p;
      if constexpr (HFIX) {
        h = rl % H;
        p = pb + u * (RB / H) + rl / H;
      } else {
        p = r / H;
        h = r - p * H;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          qp[i] = qs[h * D + 8 * c + i];
          qn[i] = qs[H * D + h * D + 8 * c + i];
        }
      }
      float ps = 0.0f, ns = 0.0f;
      if constexpr (U8) {
        const uint32_t wa[2] = {a[u].x, a[u].y};
        const uint32_t wb[2] = {b[u].x, b[u].y};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float kx = __fadd_rn(dlo[i], __fmul_rn((float)((wb[i >> 2] >> (8 * (i & 3))) & 255u), dst[i]));
          const float kn = __fadd_rn(dlo[i], __fmul_rn((float)((wa[i >> 2] >> (8 * (i & 3))) & 255u), dst[i]));
          ps = __fadd_rn(ps, __fmul_rn(kx, qp[i]));
          ns = __fadd_rn(ns, __fmul_rn(kn, qn[i]));
        }
      } else {
        const uint32_t wa[4] = {a[u].x, a[u].y, a[u].z, a[u].w};
        const uint32_t wb[4] = {b[u].x, b[u].y, b[u].z, b[u].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float px = (i & 1) ? mul_f16<1>(wb[i >> 1], qp[i]) : mul_f16<0>(wb[i >> 1], qp[i]);
          const float pn = (i & 1) ? mul_f16<1>(wa[i >> 1], qn[i]) : mul_f16<0>(wa[i >> 1], qn[i]);
          ps = __fadd_rn(ps, px);
          ns = __fadd_rn(ns, pn);
        }
      }
      if constexpr (G == 16) {
        ps = row16_reduce(ps);
        ns = row16_reduce(ns);
      } else {
        ps = row_reduce(ps, G);
        ns = row_reduce(ns, G);
      }
      if (r < nr && c == 0) {
        float v = __fadd_rn(__fadd_rn(ps, ns), 0.0f);
        if constexpr (HFIX) {
          if (pid_lds) {  // a page id outside the statistics gets bound -inf (never preferred)
            if (s_pid[sl * pps + u * (RB / H) + rl / H] < 0) v = -__builtin_inff();
          } else if (pids) {
            const int64_t bk = pids[p];
            if (bk < 0 || bk >= nstat) v = -__builtin_inff();
          }
        }
        const int64_t o = head_major ? (int64_t)h * out_p + out_off + p : out_off * H + r;
        if (odt == HKV_DT_F16) ((uint16_t*)out)[o] = f2h(v);
        else ((float*)out)[o] = v;
        if constexpr (HFIX) {
          const uint32_t kk = ukey(v);
          kmn_t = kk < kmn_t ? kk : kmn_t;
          kmx_t = kk > kmx_t ? kk : kmx_t;
        }
      }
    }
  };
  // two register buffers: while a step is computed the next one is in
  // flight; a buffer is refilled (two steps ahead) once computed (unrolled
  // by 2 so no pending load is copied; loads past the end are clamped)
  int pb = HFIX ? r0 / H : 0;
  const int pstep = HFIX ? step / H : 0;
  while (r0 < nr) {
    compute(r0, pb, sl, a0, b0);
    load(r0 + 2 * step, sl + 2, a0, b0);
    r0 += step;
    pb += pstep;
    ++sl;
    if (r0 >= nr) break;
    compute(r0, pb, sl, a1, b1);
    load(r0 + 2 * step, sl + 2, a1, b1);
    r0 += step;
    pb += pstep;
    ++sl;
  }
  if constexpr (HFIX) {
    // per-block key range of each head for the multi-block top-K
    if (mm) {
      __shared__ uint32_t s_mn[kMaxMMHeads], s_mx[kMaxMMHeads];
      for (int i = threadIdx.x; i < H; i += 256) { s_mn[i] = 0xffffffffu; s_mx[i] = 0u; }
      __syncthreads();
      if (c == 0) {
        atomicMin(&s_mn[rl % H], kmn_t);
        atomicMax(&s_mx[rl % H], kmx_t);
      }
      __syncthreads();
      for (int i = threadIdx.x; i < H; i += 256) mm[(int64_t)i * gridDim.x + blockIdx.x] = make_uint2(s_mn[i], s_mx[i]);
    }
  }
}

template <int G, bool HFIX>
__global__ void __launch_bounds__(256)
bound_f16_kernel(const void* q, int qdt, int group, const uint16_t* __restrict__ kmin,
                 const uint16_t* __restrict__ kmax, int64_t P, int H, void* out, int odt,
                 int head_major, uint2* mm, int q_lds, const int64_t* pids, int64_t nstat) {
  bound_f16_rows<G, HFIX>(q, qdt, group, kmin, kmax, P, H, out, odt, head_major, P, 0, blockIdx.x,
                          gridDim.x, mm, q_lds, nullptr, nullptr, pids, nstat);
}

// Ragged batch: sequence s owns pages [off[s], off[s+1]) of the concatenated
// statistics and query q + s * q_bytes (the bound kernel's blocks
// [blk[s], blk[s+1]), the top-K kernel's blockIdx.y = s); scores head-major
// over the concatenated page axis, (H, off[nseg]).
constexpr int kMaxSeqs = 64;
// Paged (bt non-null, HFIX only): sequence s's logical page p has its
// statistics at row bt[bt0[s] + p] of the pool's (nstat, H, D) statistics.
struct Segs {
  int64_t off[kMaxSeqs + 1];
  int64_t k[kMaxSeqs];
  int64_t out_off[kMaxSeqs + 1];
  int64_t bt0[kMaxSeqs];
  int blk[kMaxSeqs + 1];  // the bound kernel's blocks of sequence b: [blk[b], blk[b+1])
  int nseg;
};

template <int G, bool HFIX>
__global__ void __launch_bounds__(256)
bound_f16_ragged_kernel(const char* q, int64_t q_bytes, int qdt, int group,
                        const uint16_t* __restrict__ kmin, const uint16_t* __restrict__ kmax, int H,
                        float* out, const Segs segs, int q_lds, const int64_t* bt, int64_t nstat) {
  // blocks are given to the sequences in proportion to their pages
  int sq = 0;
  while (sq + 1 < segs.nseg && segs.blk[sq + 1] <= (int)blockIdx.x) ++sq;
  const int bx = (int)blockIdx.x - segs.blk[sq], gx = segs.blk[sq + 1] - segs.blk[sq];
  const int64_t o0 = segs.off[sq], P = segs.off[sq + 1] - o0;
  if (HFIX && bt) {
    bound_f16_rows<G, HFIX>(q + sq * q_bytes, qdt, group, kmin, kmax, P, H, out, HKV_DT_F32, 1,
                            segs.off[segs.nseg], o0, bx, gx, nullptr, q_lds, nullptr, nullptr,
                            bt + segs.bt0[sq], nstat);
  } else {
    bound_f16_rows<G, HFIX>(q + sq * q_bytes, qdt, group, kmin + o0 * H * (8 * G),
                            kmax + o0 * H * (8 * G), P, H, out, HKV_DT_F32, 1, segs.off[segs.nseg],
                            o0, bx, gx, nullptr, q_lds);
  }
}

// --------------------------------------------------------- a10: top-K

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kBins = 2048;


constexpr int kCand = 4096;  // keys of the first digit's bin kept in LDS

struct SelShared {
  uint32_t hist[kBins];
  uint32_t wred[kSelWaves][4];
  uint32_t bcast[8];
  uint32_t cand[kCand];
  uint32_t ncand;
};

// Block-wide (1024 threads) reductions through LDS.
HKV_DEV uint32_t block_min_u32(uint32_t v, SelShared& sh) {
  for (int o = 32; o >= 1; o >>= 1) { uint32_t y = __shfl_xor(v, o, 64); v = y < v ? y : v; }
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wred[w][0] = v;
  __syncthreads();
  uint32_t r = sh.wred[0][0];
  for (int i = 1; i < kSelWaves; ++i) r = sh.wred[i][0] < r ? sh.wred[i][0] : r;
  return r;
}
HKV_DEV uint32_t block_max_u32(uint32_t v, SelShared& sh) {
  for (int o = 32; o >= 1; o >>= 1) { uint32_t y = __shfl_xor(v, o, 64); v = y > v ? y : v; }
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh.wred[w][1] = v;
  __syncthreads();
  uint32_t r = sh.wred[0][1];
  for (int i = 1; i < kSelWaves; ++i) r = sh.wred[i][1] > r ? sh.wred[i][1] : r;
  return r;
}

// Key of candidate i (i in [0, n)) of the column; column element p = s + i.
// Column h of a score matrix: page p at base[h * hstride + p * stride].
struct ColumnF32 {
  const float* base;
  int64_t stride, hstride;
  HKV_DEV uint32_t key(int64_t p) const { return ukey(base[p * stride]); }
};
struct ColumnF16 {
  const uint16_t* base;
  int64_t stride, hstride;
  HKV_DEV uint32_t key(int64_t p) const { return ukey(h2f(base[p * stride])); }
};

// Select, for one column of P scores, the sinks plus the k_eff highest non-sink
// pages (ties to the lower page), ascending, into out[i*ostride].  Candidate
// pages [s, P) are split into 16 contiguous wave chunks walked in rounds of 64
// consecutive pages (coalesced); ordering within a chunk comes from ballots.
template <typename Col>
HKV_DEV void select_column(const Col& col, int64_t P, int64_t s, int64_t keff, int64_t* out,
                           int64_t ostride, SelShared& sh) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int64_t i = tid; i < s; i += kSelThreads) out[i * ostride] = i;
  if (keff <= 0) return;
  const int64_t n = P - s;
  const int64_t chunk = ((n + kSelWaves - 1) / kSelWaves + 63) / 64 * 64;
  const int64_t c0 = s + (int64_t)w * chunk;
  const int64_t c1 = (c0 + chunk < P) ? c0 + chunk : P;

  // 1. key range
  uint32_t kmn = 0xffffffffu, kmx = 0;
  for (int64_t p = c0 + lane; p < c1; p += 64) {
    const uint32_t k = col.key(p);
    kmn = k < kmn ? k : kmn;
    kmx = k > kmx ? k : kmx;
  }
  kmn = block_min_u32(kmn, sh);
  kmx = block_max_u32(kmx, sh);

  // 2. radix select of the keff-th largest key T, digits of <= 11 bits
  //    starting at the highest bit where the keys differ.
  uint32_t prefix = kmx, pmask = 0xffffffffu;  // keys matching prefix under pmask
  uint32_t krem = (uint32_t)keff, gt = 0;
  if (kmn != kmx) {
    int hb = 31 - __builtin_clz(kmn ^ kmx);
    pmask = hb == 31 ? 0u : ~((2u << hb) - 1u);
    prefix = kmx & pmask;
    while (true) {
      const int lo = hb >= 10 ? hb - 10 : 0;
      const uint32_t nb = 1u << (hb - lo + 1);
      for (int i = tid; i < (int)nb; i += kSelThreads) sh.hist[i] = 0;
      if (tid == 0) { sh.bcast[0] = 0; sh.bcast[1] = 0; }
      __syncthreads();
      for (int64_t p = c0 + lane; p < c1; p += 64) {
        const uint32_t k = col.key(p);
        if ((k & pmask) == prefix) atomicAdd(&sh.hist[(k >> lo) & (nb - 1)], 1u);
      }
      __syncthreads();
      // find bin b (from the top) where the running count reaches krem:
      // thread t owns bins 2t, 2t+1; suffix sums by a reversed block scan.
      {
        const uint32_t h0 = 2 * tid < (int)nb ? sh.hist[2 * tid] : 0u;
        const uint32_t h1 = 2 * tid + 1 < (int)nb ? sh.hist[2 * tid + 1] : 0u;
        const uint32_t loc = h0 + h1;
        uint32_t inc = loc;  // inclusive suffix within the wave
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t y = __shfl_down(inc, o, 64);
          if (lane + o < 64) inc += y;
        }
        if (lane == 0) sh.wred[w][0] = inc;
        __syncthreads();
        uint32_t later = 0;
        for (int i = w + 1; i < kSelWaves; ++i) later += sh.wred[i][0];
        const uint32_t sfx = later + inc - loc;  // count in bins above 2t+1
        if (sfx < krem && krem <= sfx + loc) {
          if (sfx + h1 >= krem) { sh.bcast[0] = 2 * tid + 1; sh.bcast[1] = sfx; }
          else { sh.bcast[0] = 2 * tid; sh.bcast[1] = sfx + h1; }
        }
        __syncthreads();
      }
      const uint32_t b = sh.bcast[0], above = sh.bcast[1];
      gt += above;
      krem -= above;
      prefix |= b << lo;
      pmask |= (nb - 1) << lo;
      if (lo == 0) break;
      hb = lo - 1;
      __syncthreads();
    }
  }
  const uint32_t T = prefix;
  const uint32_t need_eq = krem;  // keys == T to take, lowest pages first

  // 3. per-wave counts of > T and == T, then wave offsets
  uint32_t cgt = 0, ceq = 0;
  for (int64_t p = c0 + lane; p < c1; p += 64) {
    const uint32_t k = col.key(p);
    cgt += k > T;
    ceq += k == T;
  }
  for (int o = 32; o >= 1; o >>= 1) {
    cgt += __shfl_xor(cgt, o, 64);
    ceq += __shfl_xor(ceq, o, 64);
  }
  __syncthreads();
  if (lane == 0) { sh.wred[w][2] = cgt; sh.wred[w][3] = ceq; }
  __syncthreads();
  uint32_t eq_before = 0, out_before = 0;
  for (int i = 0; i < w; ++i) {
    const uint32_t e = sh.wred[i][3];
    const uint32_t take = eq_before >= need_eq ? 0u : (need_eq - eq_before < e ? need_eq - eq_before : e);
    out_before += sh.wred[i][2] + take;
    eq_before += e;
  }
  (void)gt;

  // 4. ordered write within the chunk
  uint32_t run_out = 0, run_eq = 0;
  const uint64_t lanemask_lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t p0 = c0; p0 < c1; p0 += 64) {
    const int64_t p = p0 + lane;
    const uint32_t k = p < c1 ? col.key(p) : 0u;
    const bool is_eq = p < c1 && k == T;
    const uint64_t eqm = __ballot(is_eq);
    const uint32_t eq_rank = eq_before + run_eq + __builtin_popcountll(eqm & lanemask_lt);
    const bool sel = p < c1 && (k > T || (is_eq && eq_rank < need_eq));
    const uint64_t selm = __ballot(sel);
    if (sel) {
      const uint32_t pos = out_before + run_out + __builtin_popcountll(selm & lanemask_lt);
      if (pos < (uint64_t)keff) out[(s + (int64_t)pos) * ostride] = p;
    }
    run_out += __builtin_popcountll(selm);
    run_eq += __builtin_popcountll(eqm);
  }
}

// One radix digit over bits [lo, hb] (lo = max(hb - 10, 0)) of the keys that
// match `prefix` under `pmask`: finds the bin holding the krem-th largest such
// key, narrows prefix / pmask to it and subtracts the keys in higher bins from
// krem.  `count(pmask, prefix, lo, nb)` adds, into sh.hist, the digit
// (k >> lo) & (nb - 1) of every candidate key k with (k & pmask) == prefix.
// Returns lo; *inbin = the number of keys in the chosen bin.
template <typename CountFn>
HKV_DEV int radix_digit(int hb, uint32_t& prefix, uint32_t& pmask, uint32_t& krem, SelShared& sh,
                        CountFn count, uint32_t* inbin) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lo = hb >= 10 ? hb - 10 : 0;
  const uint32_t nb = 1u << (hb - lo + 1);
  for (int i = tid; i < (int)nb; i += kSelThreads) sh.hist[i] = 0;
  __syncthreads();
  count(pmask, prefix, lo, nb);
  __syncthreads();
  {
    const uint32_t h0 = 2 * tid < (int)nb ? sh.hist[2 * tid] : 0u;
    const uint32_t h1 = 2 * tid + 1 < (int)nb ? sh.hist[2 * tid + 1] : 0u;
    const uint32_t loc = h0 + h1;
    uint32_t inc = loc;  // inclusive suffix within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_down(inc, o, 64);
      if (lane + o < 64) inc += y;
    }
    if (lane == 0) sh.wred[w][0] = inc;
    __syncthreads();
    uint32_t later = 0;
    for (int i = w + 1; i < kSelWaves; ++i) later += sh.wred[i][0];
    const uint32_t sfx = later + inc - loc;  // count in bins above 2t+1
    if (sfx < krem && krem <= sfx + loc) {
      if (sfx + h1 >= krem) { sh.bcast[0] = 2 * tid + 1; sh.bcast[1] = sfx; sh.bcast[2] = h1; }
      else { sh.bcast[0] = 2 * tid; sh.bcast[1] = sfx + h1; sh.bcast[2] = h0; }
    }
    __syncthreads();
  }
  const uint32_t b = sh.bcast[0], above = sh.bcast[1];
  *inbin = sh.bcast[2];
  krem -= above;
  prefix |= b << lo;
  pmask |= (nb - 1) << lo;
  __syncthreads();
  return lo;
}

// Register-resident selector for n = P - s <= 1024 * KPT candidates: wave w
// holds pages s + w*64*KPT + i*64 + lane (i < KPT) as keys; the radix passes
// and the ordered write read only registers.  Slots past the last page hold
// key 0, which is below every real key (ukey >= 0x007fffff), so it is never
// selected, never equal to the threshold and never in the threshold's radix
// bin: no pass needs a validity test.  Same contract as select_column.
template <int KPT, typename Col>
HKV_DEV void select_column_regs(const Col& col, int64_t P, int64_t s, int64_t keff, int64_t* out,
                                int64_t ostride, SelShared& sh) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int64_t i = tid; i < s; i += kSelThreads) out[i * ostride] = i;
  if (keff <= 0) return;
  const int64_t c0 = s + (int64_t)w * (64 * KPT) + lane;  // page of key[0]
  const int64_t lim = P - c0;                              // key[i] is a page iff i*64 < lim
  uint32_t key[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) key[i] = (int64_t)i * 64 < lim ? col.key(c0 + (int64_t)i * 64) : 0u;
  // min over real keys: the sentinel 0 wraps to the largest value under "- 1"
  uint32_t kmn = 0xffffffffu, kmx = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const uint32_t m1 = key[i] - 1u;
    kmn = m1 < kmn ? m1 : kmn;
    kmx = key[i] > kmx ? key[i] : kmx;
  }
  kmn = block_min_u32(kmn, sh) + 1u;
  kmx = block_max_u32(kmx, sh);
  auto count_regs = [&](uint32_t pmask, uint32_t prefix, int lo, uint32_t nb) {
#pragma unroll
    for (int i = 0; i < KPT; ++i)
      atomicAdd(&sh.hist[(key[i] >> lo) & (nb - 1)], (key[i] & pmask) == prefix ? 1u : 0u);
  };
  // First digit over the registers; then, when the chosen bin is small, its
  // keys are compacted into LDS and the remaining digits run over them only.
  uint32_t T = kmx, need_eq = (uint32_t)keff;
  if (kmn != kmx) {
    int hb = 31 - __builtin_clz(kmn ^ kmx);
    uint32_t pmask = hb == 31 ? 0u : ~((2u << hb) - 1u);
    uint32_t prefix = kmx & pmask, krem = (uint32_t)keff, inbin;
    int lo = radix_digit(hb, prefix, pmask, krem, sh, count_regs, &inbin);
    if (lo > 0 && inbin <= (uint32_t)kCand) {
      if (tid == 0) sh.ncand = 0;
      __syncthreads();
      const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        const bool in = (key[i] & pmask) == prefix;
        const uint64_t m = __ballot(in);
        if (m) {
          const int leader = __builtin_ctzll(m);
          uint32_t base = 0;
          if (lane == leader) base = atomicAdd(&sh.ncand, (uint32_t)__builtin_popcountll(m));
          base = __shfl(base, leader, 64);
          if (in) sh.cand[base + __builtin_popcountll(m & lt)] = key[i];
        }
      }
      __syncthreads();
      const uint32_t nc = sh.ncand;
      auto count_cand = [&](uint32_t pm, uint32_t pf, int l, uint32_t nbins) {
        for (uint32_t j = tid; j < nc; j += kSelThreads) {
          const uint32_t k = sh.cand[j];
          atomicAdd(&sh.hist[(k >> l) & (nbins - 1)], (k & pm) == pf ? 1u : 0u);
        }
      };
      while (lo > 0) lo = radix_digit(lo - 1, prefix, pmask, krem, sh, count_cand, &inbin);
    } else {
      while (lo > 0) lo = radix_digit(lo - 1, prefix, pmask, krem, sh, count_regs, &inbin);
    }
    T = prefix;
    need_eq = krem;
  }

  uint32_t cgt = 0, ceq = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    cgt += key[i] > T ? 1u : 0u;
    ceq += key[i] == T ? 1u : 0u;
  }
  // A fresh copy of T for the ordered write: otherwise the compiler keeps the
  // 64 compare masks of the count pass alive (in SGPRs, then spilled) to reuse.
  uint32_t Tw;
  asm volatile("v_mov_b32 %0, %1" : "=v"(Tw) : "v"(T));
  for (int o = 32; o >= 1; o >>= 1) {
    cgt += __shfl_xor(cgt, o, 64);
    ceq += __shfl_xor(ceq, o, 64);
  }
  __syncthreads();
  if (lane == 0) { sh.wred[w][2] = cgt; sh.wred[w][3] = ceq; }
  __syncthreads();
  uint32_t eq_before = 0, out_before = 0;
  for (int i = 0; i < w; ++i) {
    const uint32_t e = sh.wred[i][3];
    const uint32_t take = eq_before >= need_eq ? 0u : (need_eq - eq_before < e ? need_eq - eq_before : e);
    out_before += sh.wred[i][2] + take;
    eq_before += e;
  }
  uint32_t run_out = 0, run_eq = 0;
  const uint64_t lanemask_lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const bool is_eq = key[i] == Tw;
    const uint64_t eqm = __ballot(is_eq);
    const uint32_t eq_rank = eq_before + run_eq + __builtin_popcountll(eqm & lanemask_lt);
    const bool sel = key[i] > Tw || (is_eq && eq_rank < need_eq);
    const uint64_t selm = __ballot(sel);
    if (sel) {
      const uint32_t pos = out_before + run_out + __builtin_popcountll(selm & lanemask_lt);
      if (pos < (uint64_t)keff) out[(s + (int64_t)pos) * ostride] = c0 + (int64_t)i * 64;
    }
    run_out += __builtin_popcountll(selm);
    run_eq += __builtin_popcountll(eqm);
  }
}

// KPT == 0: streaming selector (any P); else register-resident.
template <int KPT, typename Col>
HKV_DEV void select_any(const Col& col, int64_t P, int64_t s, int64_t keff, int64_t* out,
                        int64_t ostride, SelShared& sh) {
  if constexpr (KPT == 0) select_column(col, P, s, keff, out, ostride, sh);
  else select_column_regs<KPT>(col, P, s, keff, out, ostride, sh);
}

// Smallest register tile that holds n candidates (0: too many, stream).
int kpt_for(int64_t n) {
  if (n <= (int64_t)kSelThreads * 4) return 4;
  if (n <= (int64_t)kSelThreads * 16) return 16;
  if (n <= (int64_t)kSelThreads * 64) return 64;
  return 0;
}

template <int KPT, typename Col>
__global__ void __launch_bounds__(kSelThreads)
topk_kernel(Col col0, int64_t P, int H, int64_t s, int64_t keff, int64_t* out) {
  __shared__ SelShared sh;
  const int h = blockIdx.x;
  Col col = col0;
  col.base += h * col.hstride;
  select_any<KPT>(col, P, s, keff, out + h, H, sh);
}

// Ragged batch: block (h, s) selects over pages [off[s], off[s+1]) of column h
// of the head-major scores (H, off[nseg]) with sinks and k[s]; the indices
// (local to the sequence) go to rows out_off[s] .. of out (rows, H).
template <int KPT>
__global__ void __launch_bounds__(kSelThreads)
topk_ragged_kernel(const float* scores, int H, int64_t sinks, int64_t* out, const Segs segs) {
  __shared__ SelShared sh;
  const int h = blockIdx.x, sq = blockIdx.y;
  const int64_t o0 = segs.off[sq], P = segs.off[sq + 1] - o0;
  const int64_t s = sinks < 0 ? 0 : (sinks > P ? P : sinks);
  const int64_t k = segs.k[sq];
  const int64_t keff = k < 0 ? 0 : (k > P - s ? P - s : k);
  ColumnF32 col{scores + (int64_t)h * segs.off[segs.nseg] + o0, 1, 0};
  select_any<KPT>(col, P, s, keff, out + segs.out_off[sq] * H + h, H, sh);
}

// ------------------------------------------ multi-block top-K (large columns)
//
// One head's candidates [s, P) are split into NB slices of kMBThreads*KPT
// consecutive pages, one block each, in two kernels (no block ever waits):
//  topk_mb_hist: every block histograms its slice into 4096 bins of
//    (key - kmn) >> sh, where kmn / kmx come from the bound kernel's per-block
//    key ranges and sh makes the range fit; it stores the histogram and the
//    keys of the bins around its own estimate of the threshold bin (the bin
//    of its proportional share of keff), then arrives at the head's counter.
//    The last block to arrive sums the histograms, finds the bin b1 of the
//    keff-th largest key, gathers that bin's keys (from the slices' windows
//    when b1 lies in every window that can hold keys of b1, else by re-reading
//    the column), ranks them (key descending, page ascending) and writes the
//    threshold key T, how many keys equal to T are taken, and for every slice
//    the output row of its first selected page and the number of T-equal keys
//    before it.  It leaves the counter at zero for the next call.  A bin of
//    more than kMBCand keys falls back to the single-block selector.
//  topk_mb_write: each block writes its slice's selected pages in page order.
// Same result as select_column_regs: sinks, then the keff highest keys with
// ties to the lower page, ascending.
constexpr int kMBThreads = 1024;
constexpr int kMBWaves = kMBThreads / 64;
constexpr int kMBBins = 4096;
constexpr int kMBCand = 4096;
constexpr int kMBMaxSlices = 64;
constexpr int kMBWinBins = 24;   // window half-width around a slice's own threshold-bin estimate
constexpr int kMBWin = 1024;     // window keys stored per slice

struct MBWork {
  uint32_t* ctr;     // [H] arrival counters (zero between calls)
  uint32_t* leave;   // [H] departure counters of the fused form (zero between calls)
  const uint2* mm;   // [H][nmm] (min key, max key) of the bound kernel's blocks
  int nmm;
  uint32_t* hist;    // [H][NB][kMBBins / 2] u16 counts, bin 2i in the low half of word i
  int* meta;         // [H][NB][2] (out row of the slice's first selected page, T-equal keys before it)
  uint32_t* thr;     // [H][4] (T, T-equal keys taken, 1 = selection already written, s + keff)
  uint32_t* wcand;   // [H][NB][kMBWin] keys of the slice's window bins
  int* wmeta;        // [H][NB][4] (first window bin, last window bin, keys stored, overflowed)
};

struct MBShared {
  uint32_t hist[kMBBins];
  unsigned long long cand[kMBCand];
  uint32_t ncand;
  uint32_t red[2][kMBWaves];
  uint32_t bc[8];
  int wm[kMBMaxSlices][4];
  uint32_t sl_b1[kMBMaxSlices];
  uint4 red4[kMBWaves];
  int sl_gt[kMBMaxSlices], sl_eq[kMBMaxSlices];
  int win_half;  // the slice's window half-width in bins
};

// Block-wide minimum of a and maximum of b (one pair of barriers).
HKV_DEV void mb_minmax(uint32_t& a, uint32_t& b, uint32_t (*red)[kMBWaves]) {
  a = wave_min_u(a);
  b = wave_max_u(b);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    red[0][w] = a;
    red[1][w] = b;
  }
  __syncthreads();
  a = red[0][0];
  b = red[1][0];
  for (int i = 1; i < kMBWaves; ++i) {
    a = red[0][i] < a ? red[0][i] : a;
    b = red[1][i] > b ? red[1][i] : b;
  }
}

// Exclusive prefix sum over the block in thread order; total in `total`.
HKV_DEV uint32_t mb_excl_scan(uint32_t v, uint32_t* red, uint32_t& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t x = wave_incl_scan_u(v);
  __syncthreads();
  if (lane == 63) red[w] = x;
  __syncthreads();
  uint32_t before = 0, tot = 0;
  for (int i = 0; i < kMBWaves; ++i) {
    const uint32_t r = red[i];
    before += i < w ? r : 0u;
    tot += r;
  }
  total = tot;
  return before + x - v;
}

// Exclusive prefix sums of four values over the block in thread order.
HKV_DEV uint4 mb_excl_scan4(uint4 v, uint4* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint4 x = make_uint4(wave_incl_scan_u(v.x), wave_incl_scan_u(v.y), wave_incl_scan_u(v.z),
                             wave_incl_scan_u(v.w));
  __syncthreads();
  if (lane == 63) red[w] = x;
  __syncthreads();
  uint4 b = make_uint4(0u, 0u, 0u, 0u);
  for (int i = 0; i < w; ++i) {
    const uint4 r = red[i];
    b.x += r.x;
    b.y += r.y;
    b.z += r.z;
    b.w += r.w;
  }
  return make_uint4(b.x + x.x - v.x, b.y + x.y - v.y, b.z + x.z - v.z, b.w + x.w - v.w);
}

// Waits until this wave's global stores are complete (s_waitcnt vmcnt(0);
// the export and LDS counters are left alone).  __syncthreads() does not wait
// for them, so without this another wave's agent-scope release could write L2
// back to memory before this wave's stores have reached L2.
HKV_DEV void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }

constexpr uint32_t kMBStage = 8192;     // pages staged in LDS per round of the ordered write
constexpr uint32_t kMBSpan = (1u << 27) - 1u;  // ordered keys the histogram bins span at most
constexpr int kMBSpinLimit = 1 << 22;   // polls of the fused form's wait for a head's slices

// Block j's part of the output: the selected pages of slice j -- every key
// > T and, of the keys == T, those whose rank among the head's T-equal keys
// is below need_eq -- in page order from output row `first` (eqb0 T-equal
// keys of the head lie in slices before j).  Positions come from one block
// scan of the per-thread counts, (== T) << 16 | (> T) (at most kMBThreads *
// KPT each).  The pages are staged in LDS in output order and written by
// consecutive threads: the column of head h is strided by H, so each
// 128-byte line is written with one request instead of one per page.
// kv: the thread's keys, candidates j * slice + i * kMBThreads + tid when
// the stage holds the slice (they are transposed through it so that the
// thread holds candidates c0 .. c0 + KPT - 1), else c0 + i directly.
template <int KPT>
HKV_DEV void mb_write_slice(float (&kv)[KPT], int n, int64_t s, int64_t* out, int H, int h, int j,
                            uint32_t T, uint32_t need_eq, uint32_t row_end, uint32_t first,
                            uint32_t eqb0, uint32_t* stage, uint32_t* red) {
  const int tid = threadIdx.x;
  const int c0 = j * (kMBThreads * KPT) + tid * KPT;
  if constexpr (kMBThreads * KPT <= (int)kMBStage) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) stage[i * kMBThreads + tid] = __float_as_uint(kv[i]);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KPT; ++i) kv[i] = __uint_as_float(stage[tid * KPT + i]);
  }
  auto taken = [&](uint32_t eqs) { return eqs < need_eq ? eqs : need_eq; };
  uint32_t key[KPT];
  uint32_t gt = 0, eq = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    key[i] = c0 + i < n ? ukey(kv[i]) : 0u;  // 0: below every real key
    gt += key[i] > T ? 1u : 0u;
    eq += (c0 + i < n && key[i] == T) ? 1u : 0u;
  }
  uint32_t tot;
  const uint32_t pre = mb_excl_scan(gt | (eq << 16), red, tot);  // its barriers order the stage
  const uint32_t nsel = (tot & 0xffffu) + taken(eqb0 + (tot >> 16)) - taken(eqb0);
  const uint32_t rel0 = (pre & 0xffffu) + taken(eqb0 + (pre >> 16)) - taken(eqb0);
  for (uint32_t sub = 0; sub < nsel; sub += kMBStage) {
    uint32_t rel = rel0, eqr = eqb0 + (pre >> 16);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const bool is_eq = c0 + i < n && key[i] == T;
      const bool sel = key[i] > T || (is_eq && eqr < need_eq);
      eqr += is_eq ? 1u : 0u;
      if (sel && rel - sub < kMBStage) stage[rel - sub] = (uint32_t)(s + c0 + i);
      rel += sel ? 1u : 0u;
    }
    __syncthreads();
    const uint32_t cnt = nsel - sub < kMBStage ? nsel - sub : kMBStage;
    for (uint32_t i = tid; i < cnt; i += kMBThreads) {
      const uint32_t r = first + sub + i;
      if (r < row_end) out[(int64_t)r * H + h] = (int64_t)stage[i];
    }
    __syncthreads();
  }
}

// Fused form: a block leaves once it is done with the head's shared state;
// the last of the head's NB blocks to leave zeroes both counters for the next
// call (every block has passed its wait by then).
HKV_DEV void mb_leave(const MBWork& w, int h, int NB) {
  if (threadIdx.x == 0 && atomicAdd(&w.leave[h], 1u) == (uint32_t)(NB - 1)) {
    atomicExch(&w.ctr[h], 0u);
    atomicExch(&w.leave[h], 0u);
  }
}

// FUSED: every block of the head computes the threshold itself once all NB
// slices have arrived, then writes its own slice (no second kernel, the keys
// stay in registers).  Blocks wait for one another, so the host uses this
// form only when the whole grid is resident at once (at most one block per
// CU); else the last block to arrive computes the threshold for
// topk_mb_write.
template <int KPT, bool FUSED>
__global__ void __launch_bounds__(kMBThreads)
topk_mb_hist(const float* scores, int64_t P, int64_t s, int64_t keff, int64_t* out, int H,
               MBWork w) {
  __shared__ MBShared sh;
  __shared__ int s_last;
  const int j = blockIdx.x, h = blockIdx.y, NB = gridDim.x, tid = threadIdx.x;
  const int n = (int)(P - s);
  const float* col = scores + (int64_t)h * P + s;  // candidate i is page s + i
  constexpr int slice = kMBThreads * KPT;
  // key i of the thread is candidate c0 + i * kMBThreads: each load
  // instruction reads consecutive words across the block.  Loads are
  // unconditional (clamped index) so that all KPT are in flight at once.
  const int c0 = j * slice + tid;
  float kv[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int c = c0 + i * kMBThreads;
    kv[i] = col[c < n ? c : n - 1];
  }
  // key range of the head (all pages, sinks included: a superset of the
  // candidates'); the first range is requested with the keys
  const uint2* hmm = w.mm + (int64_t)h * w.nmm;
  uint2 v0 = hmm[tid < w.nmm ? tid : w.nmm - 1];
  uint32_t mn = v0.x, mx = v0.y;
  for (int b = tid + kMBThreads; b < w.nmm; b += kMBThreads) {
    const uint2 v = hmm[b];
    mn = v.x < mn ? v.x : mn;
    mx = v.y > mx ? v.y : mx;
  }
  for (int b = tid; b < kMBBins; b += kMBThreads) sh.hist[b] = 0u;  // ordered by mb_minmax's barriers
  mb_minmax(mn, mx, sh.red);
  // Bins over at most the top kMBSpan ordered keys below the largest (16
  // binades of one sign): a few keys far below the rest (a bound of the
  // other sign lies about 2^31 keys away) would otherwise put most keys in
  // the threshold's bin and send the selection to the single-block
  // fallback.  Keys below the range share bin 0, whose key range is then
  // open below.
  if (mx - mn > kMBSpan) mn = mx - kMBSpan;
  const uint32_t range = mx - mn;
  const int wbits = range ? 32 - __builtin_clz(range) : 0;
  const int sh1 = wbits > 12 ? wbits - 12 : 0;
  auto bin_of = [&](uint32_t k) {
    const uint32_t b0 = k < mn ? 0u : (k - mn) >> sh1;
    return b0 < (uint32_t)kMBBins ? (int)b0 : kMBBins - 1;
  };
#pragma unroll
  for (int i = 0; i < KPT; ++i)
    if (c0 + i * kMBThreads < n) atomicAdd(&sh.hist[bin_of(ukey(kv[i]))], 1u);
  __syncthreads();
  // the slice's histogram as u16 (a slice holds at most 2^15 keys): thread t
  // stores bins 4t .. 4t + 3
  static_assert(kMBBins == 4 * kMBThreads, "four bins per thread");
  static_assert(kMBThreads * KPT <= 65535, "u16 bin counts");
  {
    const uint4 hb = reinterpret_cast<const uint4*>(sh.hist)[tid];
    reinterpret_cast<uint2*>(w.hist + ((int64_t)h * NB + j) * (kMBBins / 2))[tid] =
        make_uint2(hb.x | (hb.y << 16), hb.z | (hb.w << 16));
  }
  {
    // This slice's own estimate of the threshold bin (the bin of its
    // proportional share of keff), and the keys of the bins around it: if the
    // true threshold bin lies in every slice's window, the last block finds
    // its candidates here instead of re-reading the column.
    const int nj = n - j * slice < slice ? n - j * slice : slice;
    uint64_t kj = ((uint64_t)keff * (uint64_t)nj + (uint64_t)n - 1) / (uint64_t)n;
    kj = kj < 1 ? 1 : (kj > (uint64_t)nj ? (uint64_t)nj : kj);
    uint32_t mine_l = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) mine_l += sh.hist[kMBBins - 1 - 4 * tid - k];
    if (tid == 0) sh.bc[2] = 0u;  // ordered before the writes below by the scan's barriers
    uint32_t tot_l;
    uint32_t above_l = mb_excl_scan(mine_l, sh.red[0], tot_l);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int b = kMBBins - 1 - 4 * tid - k;
      const uint32_t c = sh.hist[b];
      if (above_l < (uint32_t)kj && above_l + c >= (uint32_t)kj) sh.bc[2] = (uint32_t)b;
      above_l += c;
    }
    if (tid == 0) sh.ncand = 0u;
    __syncthreads();
    const int bj = (int)sh.bc[2];
    // The window: the widest (half-width up to kMBWinBins) whose keys fit in
    // kMBWin.  Where the bins are dense the estimate is also sharp in bins,
    // so a narrow window still holds the threshold bin.  Lane i of wave 0
    // takes bin bj - kMBWinBins + i; a wave scan gives every window's count.
    static_assert(2 * kMBWinBins + 1 <= 64, "one bin per lane");
    if (tid < 64) {
      const int b = bj - kMBWinBins + tid;
      const uint32_t c = (tid <= 2 * kMBWinBins && b >= 0 && b < kMBBins) ? sh.hist[b] : 0u;
      const uint32_t incl = wave_incl_scan_u(c);  // bins bj - kMBWinBins .. b
      // window of half-width a = tid: lanes kMBWinBins - a .. kMBWinBins + a
      const int a = tid;
      const int hi_l = kMBWinBins + a < 63 ? kMBWinBins + a : 63;
      const int lo_l = kMBWinBins - a - 1;
      const uint32_t at_hi = (uint32_t)__shfl((int)incl, hi_l, 64);
      const uint32_t at_lo = (uint32_t)__shfl((int)incl, lo_l < 0 ? 0 : lo_l, 64);
      const uint32_t cnt = at_hi - (lo_l < 0 ? 0u : at_lo);
      // windows nest, so the ones that fit are a prefix of the half-widths
      const uint64_t fit = __ballot(a <= kMBWinBins && cnt <= (uint32_t)kMBWin);
      if (tid == 0) sh.win_half = fit ? 63 - __builtin_clzll(fit) : 0;
    }
    __syncthreads();
    const int wh = sh.win_half;
    const int wlo = bj - wh > 0 ? bj - wh : 0;
    const int whi = bj + wh < kMBBins - 1 ? bj + wh : kMBBins - 1;
    uint32_t* wc = w.wcand + ((int64_t)h * NB + j) * kMBWin;
    // the thread's window keys (a mask), their offset among the wave's by a
    // wave scan, and one LDS atomic per wave for the wave's base
    static_assert(KPT <= 32, "window mask");
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int b = bin_of(ukey(kv[i]));
      m |= (c0 + i * kMBThreads < n && b >= wlo && b <= whi) ? 1u << i : 0u;
    }
    const uint32_t cm = (uint32_t)__builtin_popcount(m);
    const uint32_t incl = wave_incl_scan_u(cm);
    const uint32_t wtot = rl_u(incl, 63);
    if (wtot) {
      uint32_t b0 = 0;
      if ((tid & 63) == 0) b0 = atomicAdd(&sh.ncand, wtot);
      uint32_t slot = rl_u(b0, 0) + incl - cm;
#pragma unroll
      for (int i = 0; i < KPT; ++i) {
        if ((m >> i) & 1u) {
          if (slot < (uint32_t)kMBWin) wc[slot] = ukey(kv[i]);
          ++slot;
        }
      }
    }
    __syncthreads();
    if (tid == 0) {
      int* wm = w.wmeta + ((int64_t)h * NB + j) * 4;
      wm[0] = wlo;
      wm[1] = whi;
      wm[2] = sh.ncand < (uint32_t)kMBWin ? (int)sh.ncand : kMBWin;
      wm[3] = sh.ncand > (uint32_t)kMBWin ? 1 : 0;
    }
  }
  wait_stores();
  __syncthreads();
  if constexpr (FUSED) {
    if (tid == 0) {
      __threadfence();  // release this slice's histogram and window
      uint32_t a = atomicAdd(&w.ctr[h], 1u) + 1u;
      int it = 0;
      while (a < (uint32_t)NB && it < kMBSpinLimit) {
        __builtin_amdgcn_s_sleep(2);
        a = __hip_atomic_load(&w.ctr[h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        ++it;
      }
      s_last = a >= (uint32_t)NB;
      __threadfence();  // acquire every slice's histogram (one cache invalidation for the block)
      if (!s_last) w.thr[h * 4 + 2] = 2u;  // gave up waiting: this slice's pages are not written
    }
    __syncthreads();
    if (!s_last) return;
  } else {
    if (tid == 0) {
      __threadfence();  // release this slice's histogram and window
      s_last = atomicAdd(&w.ctr[h], 1u) == (uint32_t)(NB - 1);
    }
    __syncthreads();
    if (!s_last) return;
    if (tid == 0) {
      __threadfence();  // acquire every slice's histogram (one cache invalidation for the block)
      atomicExch(&w.ctr[h], 0u);  // every slice has arrived: ready for the next call
    }
    __syncthreads();
  }

  // ---- every block (FUSED) or the last block of head h: the threshold
  // Thread t owns bins 4 * ch .. 4 * ch + 3, ch = 1023 - t (bins high to low
  // over the threads; its k-th bin from the top is field 3 - k), one 8-byte
  // chunk of every slice's u16 histogram.  Per group of 8 slices a packed
  // scan (two slices per word) of the thread's per-slice sums gives every
  // slice's count in the bins above the thread's.  The slices' windows and
  // window descriptors are requested in the same round trip (up to 8 slices).
  static_assert(kMBWin == kMBThreads, "window word u of thread t is entry t of slice u");
  const int NBc = NB < kMBMaxSlices ? NB : kMBMaxSlices;
  const bool win_regs = NBc <= 8;
  uint32_t wcr[8];
  if (win_regs) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int jj = u < NBc ? u : NBc - 1;
      wcr[u] = w.wcand[((int64_t)h * NB + jj) * kMBWin + tid];
    }
  }
  // the slices' window descriptors, one int per thread (NBc * 4 <= 256),
  // requested before the histograms and stored to LDS after them: a load
  // whose result is needed first would be waited for before the histograms
  // are requested
  const int nwm = NBc * 4;
  const int wmv = w.wmeta[((int64_t)h * NB) * 4 + (tid < nwm ? tid : nwm - 1)];
  const uint2* hist2 = reinterpret_cast<const uint2*>(w.hist + (int64_t)h * NB * (kMBBins / 2));
  const int ch = kMBThreads - 1 - tid;
  auto field = [](uint2 x, int e) {  // bin 4 * ch + e of a chunk
    const uint32_t v = e < 2 ? x.x : x.y;
    return (e & 1) ? v >> 16 : v & 0xffffu;
  };
  uint2 hv[8];                          // chunks of slices g * 8 .. g * 8 + 7
  uint32_t binc[4] = {0u, 0u, 0u, 0u};  // the thread's bins summed over the slices
  auto load_group = [&](int g) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int jj = g * 8 + u < NBc ? g * 8 + u : NBc - 1;
      hv[u] = hist2[(int64_t)jj * (kMBBins / 4) + ch];
    }
  };
  // the group's per-slice sums of the thread's bins, packed two per word (a
  // slice holds at most 2^15 keys), and its exclusive scan over the threads
  auto group_scan = [&](int g) {
    uint32_t ss[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      uint32_t t = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) t += field(hv[u], e);
      ss[u] = g * 8 + u < NBc ? t : 0u;
    }
    return mb_excl_scan4(make_uint4(ss[0] | ss[1] << 16, ss[2] | ss[3] << 16, ss[4] | ss[5] << 16,
                                    ss[6] | ss[7] << 16),
                         sh.red4);
  };
  auto half = [](uint4 p, int u) {
    const uint32_t v = u < 2 ? p.x : u < 4 ? p.y : u < 6 ? p.z : p.w;
    return (u & 1) ? v >> 16 : v & 0xffffu;
  };
  auto add_bins = [&](int g) {
#pragma unroll
    for (int u = 0; u < 8; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) binc[e] += g * 8 + u < NBc ? field(hv[u], e) : 0u;
  };
  if (tid == 0) {  // found below (defaults keep every index in range)
    sh.bc[0] = 0u;
    sh.bc[1] = 0u;
    sh.bc[5] = 0u;
    sh.bc[6] = 0u;
    sh.bc[7] = 0u;
  }
  if (tid < kMBMaxSlices) sh.sl_eq[tid] = 0;
  load_group(0);
  add_bins(0);
  for (int g = 1; g * 8 < NBc; ++g) {  // more than 8 slices: totals first
    load_group(g);
    add_bins(g);
  }
  {
    // unconditional (threads past nwm rewrite the last entry with its own
    // value) so that the load above is not moved after the histogram loads
    const int i = tid < nwm ? tid : nwm - 1;
    sh.wm[i >> 2][i & 3] = wmv;
  }
  const uint32_t need = (uint32_t)keff;
  uint4 p0 = make_uint4(0u, 0u, 0u, 0u);
  uint32_t above;
  if (NBc <= 8) {
    // one packed scan gives the counts above the thread's bins, in all and per slice
    p0 = group_scan(0);
    above = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) above += half(p0, u);
  } else {
    uint32_t tot;
    above = mb_excl_scan(binc[0] + binc[1] + binc[2] + binc[3], sh.red[0], tot);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t c = binc[3 - k];
    if (above < need && above + c >= need) {
      // the threshold bin (up to 8 slices, with every slice's count above and in it)
      sh.bc[0] = (uint32_t)(4 * ch + 3 - k);
      sh.bc[1] = above;
      sh.bc[5] = c;
      sh.bc[6] = (uint32_t)k;
      sh.bc[7] = (uint32_t)ch;
      if (NBc <= 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          uint32_t gt = half(p0, u), in = 0;
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            gt += kk < k ? field(hv[u], 3 - kk) : 0u;
            in = kk == k ? field(hv[u], 3 - kk) : in;
          }
          if (u < NBc) {
            sh.sl_gt[u] = (int)gt;
            sh.sl_b1[u] = in;
          }
        }
      }
    }
    above += c;
  }
  __syncthreads();
  const uint32_t b1 = sh.bc[0], above1 = sh.bc[1], cnt1 = sh.bc[5];
  if (NBc > 8) {
    // per group: the packed scan again (chunks reloaded); the owner of the
    // threshold bin keeps every slice's count above its bins, then thread jj
    // adds slice jj's bins of the owner's chunk above the threshold bin
    const int own = kMBThreads - 1 - (int)sh.bc[7];
    for (int g = 0; g * 8 < NBc; ++g) {
      load_group(g);
      const uint4 pg = group_scan(g);
      if (tid == own) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (g * 8 + u < NBc) sh.sl_gt[g * 8 + u] = (int)half(pg, u);
      }
    }
    __syncthreads();
    if (tid < NBc) {
      const int k = (int)sh.bc[6];
      const uint2 x = hist2[(int64_t)tid * (kMBBins / 4) + (int)sh.bc[7]];
      uint32_t gt = 0, in = 0;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        gt += kk < k ? field(x, 3 - kk) : 0u;
        in = kk == k ? field(x, 3 - kk) : in;
      }
      sh.sl_gt[tid] += (int)gt;
      sh.sl_b1[tid] = in;
    }
    __syncthreads();
  }
  const uint32_t r = need - above1;  // 1 <= r <= cnt1
  const uint32_t lo1b = mn + (b1 << sh1);  // first key of bin b1's range
  // last key of bin b1, saturated (the top bin can end past 2^32 - 1)
  const uint64_t hi1w = (uint64_t)lo1b + ((1ull << sh1) - 1ull);
  const uint32_t hi1 = hi1w > 0xffffffffull ? 0xffffffffu : (uint32_t)hi1w;
  const uint32_t lo1 = b1 == 0 ? 0u : lo1b;  // bin 0 also holds the keys below the range
  if (cnt1 > (uint32_t)kMBCand) {
    // a huge bin: the single-block selector over the whole column (block 0
    // of the head in the fused form)
    __shared__ SelShared ssh;
    ColumnF32 cc{scores + (int64_t)h * P, 1, 0};
    if (!FUSED || j == 0) select_column(cc, P, s, keff, out + h, H, ssh);
    if constexpr (FUSED) mb_leave(w, h, NB);
    else if (tid == 0) w.thr[h * 4 + 2] = 1u;
    return;
  }
  if (tid == 0) {
    sh.ncand = 0u;
    sh.bc[3] = 0u;
    sh.bc[4] = 0xffffffffu;
  }
  // the windows hold every key of bin b1 if b1 lies in every window of a slice
  // with keys there (and no window overflowed); one slice per thread
  bool bad = false;
  if (tid < NBc) {
    const bool covers = (int)b1 >= sh.wm[tid][0] && (int)b1 <= sh.wm[tid][1];
    bad = sh.wm[tid][3] != 0 || !(covers || sh.sl_b1[tid] == 0u);
  }
  const bool use_win = win_regs && !__syncthreads_or(bad);
  if (use_win) {
    // the thread's keys of bin b1 (a mask over the slices' windows), their
    // offset among the wave's by a wave scan, one LDS atomic per wave
    uint32_t m = 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int cntu = u < NBc ? sh.wm[u][2] : 0;
      m |= (tid < cntu && wcr[u] >= lo1 && wcr[u] <= hi1) ? 1u << u : 0u;
    }
    const uint32_t cm = (uint32_t)__builtin_popcount(m);
    const uint32_t incl = wave_incl_scan_u(cm);
    const uint32_t wtot = rl_u(incl, 63);
    if (wtot) {
      uint32_t b0 = 0;
      if ((tid & 63) == 0) b0 = atomicAdd(&sh.ncand, wtot);
      uint32_t slot = rl_u(b0, 0) + incl - cm;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if ((m >> u) & 1u) {
          if (slot < (uint32_t)kMBCand) sh.cand[slot] = ((unsigned long long)wcr[u] << 32) | (uint32_t)u;
          ++slot;
        }
      }
    }
  } else {
    // candidates: the keys of bin b1 (re-read, the next 16 in flight while 16 are checked)
    const int per = (n + kMBThreads - 1) / kMBThreads;
    constexpr int RU = 16;
    uint32_t ka[RU], kb[RU];
    auto load_keys = [&](int i0, uint32_t (&kk)[RU]) {
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const int idx = (i0 + u) * kMBThreads + tid;
        kk[u] = ukey(col[idx < n ? idx : n - 1]);  // validity is checked where kk is used
      }
    };
    auto scan_keys = [&](int i0, const uint32_t (&kk)[RU]) {
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const int idx = (i0 + u) * kMBThreads + tid;
        const uint32_t k = kk[u];
        if (idx < n && k >= lo1 && k <= hi1) {
          const uint32_t slot = atomicAdd(&sh.ncand, 1u);
          if (slot < (uint32_t)kMBCand)
            sh.cand[slot] = ((unsigned long long)k << 32) | (uint32_t)(idx / slice);
        }
      }
    };
    load_keys(0, ka);
    for (int i0 = 0; i0 < per; i0 += 2 * RU) {
      load_keys(i0 + RU, kb);
      scan_keys(i0, ka);
      if (i0 + RU >= per) break;
      load_keys(i0 + 2 * RU, ka);
      scan_keys(i0 + RU, kb);
    }
  }
  __syncthreads();
  const uint32_t nc = sh.ncand < (uint32_t)kMBCand ? sh.ncand : (uint32_t)kMBCand;  // == cnt1
  const uint32_t rr = r < 1u ? 1u : (r > nc ? nc : r);  // r is in [1, nc]; clamped for safety
  // T = the rr-th largest candidate key; ngt = candidates above T
  uint32_t T, ngt;
  if (nc <= (uint32_t)kMBThreads) {
    // few candidates: a candidate's key is T iff fewer than rr keys exceed it
    // and at least rr keys are >= it
    const uint32_t* ck = reinterpret_cast<const uint32_t*>(sh.cand);  // key of candidate u: ck[2u + 1]
    const uint32_t mk = tid < (int)nc ? ck[2 * tid + 1] : 0u;
    uint32_t gtc = 0, gec = 0, u = 0;
    if ((uint32_t)(tid & ~63) < nc) {  // waves holding candidates
      for (; u + 8 <= nc; u += 8) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const uint32_t k = ck[2 * (u + q) + 1];
          gtc += k > mk ? 1u : 0u;
          gec += k >= mk ? 1u : 0u;
        }
      }
      for (; u < nc; ++u) {
        const uint32_t k = ck[2 * u + 1];
        gtc += k > mk ? 1u : 0u;
        gec += k >= mk ? 1u : 0u;
      }
    }
    if (tid < (int)nc && gtc < rr && rr <= gec) {  // every such candidate has key T
      sh.bc[4] = mk;
      sh.bc[3] = gtc;
    }
    __syncthreads();
    T = sh.bc[4];
    ngt = sh.bc[3];
  } else {
    // bitonic sort, key descending, page ascending
    uint32_t np2 = 1;
    while (np2 < nc) np2 <<= 1;
    for (uint32_t i = nc + tid; i < np2; i += kMBThreads) sh.cand[i] = 0ull;
    __syncthreads();
    for (uint32_t k = 2; k <= np2; k <<= 1) {
      for (uint32_t jj = k >> 1; jj > 0; jj >>= 1) {
        for (uint32_t i = tid; i < np2; i += kMBThreads) {
          const uint32_t ixj = i ^ jj;
          if (ixj > i) {
            const unsigned long long a = sh.cand[i], b = sh.cand[ixj];
            const bool desc = (i & k) == 0;
            if (desc ? (a < b) : (a > b)) {
              sh.cand[i] = b;
              sh.cand[ixj] = a;
            }
          }
        }
        __syncthreads();
      }
    }
    T = (uint32_t)(sh.cand[rr - 1] >> 32);
    for (uint32_t i = tid; i < nc; i += kMBThreads) {  // the first T-equal candidate in rank order
      const uint32_t k = (uint32_t)(sh.cand[i] >> 32);
      if (k == T && (i == 0 || (uint32_t)(sh.cand[i - 1] >> 32) > T)) sh.bc[3] = i;
    }
    __syncthreads();
    ngt = sh.bc[3];
  }
  const uint32_t need_eq = rr - ngt;  // T-equal keys taken, lowest pages first
  // the slices' candidates above and equal to T (a candidate's low word is
  // its slice)
  for (uint32_t i = tid; i < nc; i += kMBThreads) {
    const unsigned long long v = sh.cand[i];
    const uint32_t k = (uint32_t)(v >> 32);
    const int jj = (int)(uint32_t)v;
    if (k > T) atomicAdd(&sh.sl_gt[jj], 1);
    else if (k == T) atomicAdd(&sh.sl_eq[jj], 1);
  }
  __syncthreads();
  if constexpr (FUSED) {
    // this slice's first output row and the T-equal keys before it, then its pages
    if (tid == 0) {
      int outp = (int)s, eqb = 0;
      for (int jj = 0; jj < j; ++jj) {
        const int e = sh.sl_eq[jj];
        const int take = eqb >= (int)need_eq ? 0 : ((int)need_eq - eqb < e ? (int)need_eq - eqb : e);
        outp += sh.sl_gt[jj] + take;
        eqb += e;
      }
      sh.bc[0] = (uint32_t)outp;
      sh.bc[1] = (uint32_t)eqb;
    }
    if (j == 0)
      for (int64_t i = tid; i < s; i += kMBThreads) out[i * H + h] = i;
    __syncthreads();
    const uint32_t first = sh.bc[0], eqb0 = sh.bc[1];
    if constexpr (kMBThreads * KPT > (int)kMBStage) {
      // the stage cannot transpose the slice: the thread's consecutive keys, read again
      const int cd = j * slice + tid * KPT;
#pragma unroll
      for (int i = 0; i < KPT; ++i) kv[i] = col[cd + i < n ? cd + i : n - 1];
    }
    mb_write_slice<KPT>(kv, n, s, out, H, h, j, T, need_eq, (uint32_t)(s + keff), first, eqb0,
                        reinterpret_cast<uint32_t*>(sh.cand), sh.red[0]);
    mb_leave(w, h, NB);
  } else {
    if (tid == 0) {
      int outp = (int)s, eqb = 0;
      for (int jj = 0; jj < NB; ++jj) {
        w.meta[((int64_t)h * NB + jj) * 2] = outp;
        w.meta[((int64_t)h * NB + jj) * 2 + 1] = eqb;
        const int e = sh.sl_eq[jj];
        const int take = eqb >= (int)need_eq ? 0 : ((int)need_eq - eqb < e ? (int)need_eq - eqb : e);
        outp += sh.sl_gt[jj] + take;
        eqb += e;
      }
      w.thr[h * 4] = T;
      w.thr[h * 4 + 1] = need_eq;
      w.thr[h * 4 + 2] = 0u;
      w.thr[h * 4 + 3] = (uint32_t)(s + keff);
    }
  }
}

// Two-kernel form: block j writes the selected pages of slice j from the
// threshold and offsets the last block of topk_mb_hist left.
template <int KPT>
__global__ void __launch_bounds__(kMBThreads)
topk_mb_write(const float* scores, int64_t P, int64_t s, int64_t* out, int H, MBWork w) {
  __shared__ uint32_t red[kMBWaves];
  __shared__ uint32_t stage[kMBStage];
  const int j = blockIdx.x, h = blockIdx.y, NB = gridDim.x, tid = threadIdx.x;
  const int n = (int)(P - s);
  const float* col = scores + (int64_t)h * P + s;
  // the keys, the threshold and the slice's offsets are requested together,
  // in the layout mb_write_slice takes
  constexpr bool kTranspose = kMBThreads * KPT <= (int)kMBStage;
  float kv[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int c = kTranspose ? j * (kMBThreads * KPT) + i * kMBThreads + tid : j * (kMBThreads * KPT) + tid * KPT + i;
    kv[i] = col[c < n ? c : n - 1];
  }
  const uint4 th = *reinterpret_cast<const uint4*>(w.thr + h * 4);
  const int2 me = *reinterpret_cast<const int2*>(w.meta + ((int64_t)h * NB + j) * 2);
  if (j == 0)
    for (int64_t i = tid; i < s; i += kMBThreads) out[i * H + h] = i;
  if (th.z) return;  // written by the fallback
  mb_write_slice<KPT>(kv, n, s, out, H, h, j, th.x, th.y, th.w, (uint32_t)me.x, (uint32_t)me.y, stage,
                      red);
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

bool fdt(int dt) { return dt == HKV_DT_F16 || dt == HKV_DT_F32; }

}  // namespace

extern "C" int hkv_quest_page_stats(const void* k_pages, int dtype, int64_t P, int S, int H, int D,
                                    void* kmin, void* kmax, void* stream) {
  if (!fdt(dtype)) return HKV_ERR_DTYPE;
  if (P < 0 || S < 1 || H < 1 || D < 1) return HKV_ERR_SHAPE;
  if (P == 0) return HKV_OK;
  if (!k_pages || !kmin || !kmax) return HKV_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const bool vec = dtype == HKV_DT_F16 && D % 8 == 0 && !((uintptr_t)k_pages & 15u) &&
                   !((uintptr_t)kmin & 15u) && !((uintptr_t)kmax & 15u);
  const int64_t n = vec ? P * H * D / 8 : P * H * D;
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, (int64_t)num_cus() * 16);
  if (vec)
    hipLaunchKernelGGL(page_stats_f16, dim3(grid), dim3(256), 0, s, (const uint16_t*)k_pages, P, S,
                       H, D, (uint16_t*)kmin, (uint16_t*)kmax);
  else if (dtype == HKV_DT_F16)
    hipLaunchKernelGGL(page_stats_generic<_Float16>, dim3(grid), dim3(256), 0, s,
                       (const _Float16*)k_pages, P, S, H, D, (_Float16*)kmin, (_Float16*)kmax);
  else
    hipLaunchKernelGGL(page_stats_generic<float>, dim3(grid), dim3(256), 0, s,
                       (const float*)k_pages, P, S, H, D, (float*)kmin, (float*)kmax);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

namespace {

template <int G>
__global__ void __launch_bounds__(256)
bound_u8_kernel(const void* q, int qdt, int group, const uint8_t* __restrict__ kmin,
                const uint8_t* __restrict__ kmax, const float* __restrict__ lo,
                const float* __restrict__ step, int64_t P, int H, float* out, uint2* mm, int q_lds) {
  bound_f16_rows<G, true, true>(q, qdt, group, kmin, kmax, P, H, out, HKV_DT_F32, 1, P, 0, blockIdx.x,
                                gridDim.x, mm, q_lds, lo, step);
}

template <int G>
void launch_bound_f16(bool hfix, unsigned grid, size_t lds, hipStream_t s, const void* q, int qdt,
                      int group, const uint16_t* kmin, const uint16_t* kmax, int64_t P, int H,
                      void* out, int odt, int head_major, uint2* mm, int q_lds,
                      const int64_t* pids = nullptr, int64_t nstat = 0) {
  if (hfix)
    hipLaunchKernelGGL((bound_f16_kernel<G, true>), dim3(grid), dim3(256), lds, s, q, qdt, group,
                       kmin, kmax, P, H, out, odt, head_major, mm, q_lds, pids, nstat);
  else
    hipLaunchKernelGGL((bound_f16_kernel<G, false>), dim3(grid), dim3(256), lds, s, q, qdt, group,
                       kmin, kmax, P, H, out, odt, head_major, nullptr, q_lds, nullptr, (int64_t)0);
}

// Bytes of LDS for the raw query of the fp16 bound kernels (0: read it from
// global memory): whole 16-byte chunks, at most kQRawChunks per thread.
size_t q_raw_lds(const void* q, int qdt, int Hq, int D) {
  const size_t nb = (size_t)Hq * D * (qdt == HKV_DT_F32 ? 4 : 2);
  if (((uintptr_t)q & 15u) || nb % 16 || nb / 16 > (size_t)kQRawChunks * 256) return 0;
  return nb;
}

// Bound into out, (P,H) or head-major (H,P).
int page_bound(const void* q, int q_dtype, int Hq, const void* kmin, const void* kmax, int k_dtype,
               int64_t P, int H, int D, void* out, int out_dtype, int head_major,
               hipStream_t s, const int64_t* page_ids = nullptr, int64_t nstat = 0,
               uint2* mm = nullptr, int* nmm = nullptr) {
  if (nmm) *nmm = 0;
  if (!fdt(q_dtype) && q_dtype != HKV_DT_BF16) return HKV_ERR_DTYPE;
  if (!fdt(k_dtype) || !fdt(out_dtype)) return HKV_ERR_DTYPE;
  if (P < 0 || H < 1 || D < 1 || D > 512 || Hq < H || Hq % H) return HKV_ERR_SHAPE;
  if (P * H >= ((int64_t)1 << 31)) return HKV_ERR_SHAPE;
  if (P == 0) return HKV_OK;
  if (!q || !kmin || !kmax || !out) return HKV_ERR_ARG;
  if (D % 8 == 0 && (((uintptr_t)kmin | (uintptr_t)kmax) & 15u)) return HKV_ERR_ARG;
  const int64_t rows = P * H;
  size_t lds = sizeof(float) * 2 * H * D;
  if (lds > 64 * 1024) return HKV_ERR_SHAPE;
  const int G = D / 8;
  // (the fp16 kernel indexes elements r * D in 32 bits; with page ids, a lane's
  // head must be fixed and the statistics' rows too must fit).  A lane's head
  // is fixed when the heads divide the rows of a block's row group (256 / G):
  // the lane keeps its row of every group.
  const bool hfix = G <= 64 && G > 0 && (256 / G) % H == 0;
  if ((!page_ids || (hfix && page_ids && nstat * H * D < ((int64_t)1 << 31))) &&
      k_dtype == HKV_DT_F16 && D % 8 == 0 && (G & (G - 1)) == 0 && G <= 64 &&
      rows * D < ((int64_t)1 << 32)) {
    const int64_t span = (int64_t)(256 / G) * kBoundUnrollF16;
    const unsigned grid =
        (unsigned)std::min<int64_t>((rows + span - 1) / span, (int64_t)num_cus() * 4);
    auto mn = (const uint16_t*)kmin;
    auto mx = (const uint16_t*)kmax;
    const int group = Hq / H;
    // key ranges per block only where a head is fixed per lane and scores are fp32
    uint2* mmp = (mm && hfix && H <= kMaxMMHeads && out_dtype == HKV_DT_F32) ? mm : nullptr;
    size_t qraw = q_raw_lds(q, q_dtype, Hq, D);
    if (lds + qraw > 64 * 1024) qraw = 0;
    const int qlds = qraw != 0;
    lds += qraw;
    switch (G) {
      case 1: launch_bound_f16<1>(hfix, grid, lds, s, q, q_dtype, group, mn, mx, P, H, out, out_dtype, head_major, mmp, qlds, page_ids, nstat); break;
      case 2: launch_bound_f16<2>(hfix, grid, lds, s, q, q_dtype, group, mn, mx, P, H, out, out_dtype, head_major, mmp, qlds, page_ids, nstat); break;
      case 4: launch_bound_f16<4>(hfix, grid, lds, s, q, q_dtype, group, mn, mx, P, H, out, out_dtype, head_major, mmp, qlds, page_ids, nstat); break;
      case 8: launch_bound_f16<8>(hfix, grid, lds, s, q, q_dtype, group, mn, mx, P, H, out, out_dtype, head_major, mmp, qlds, page_ids, nstat); break;
      case 16: launch_bound_f16<16>(hfix, grid, lds, s, q, q_dtype, group, mn, mx, P, H, out, out_dtype, head_major, mmp, qlds, page_ids, nstat); break;
      case 32: launch_bound_f16<32>(hfix, grid, lds, s, q, q_dtype, group, mn, mx, P, H, out, out_dtype, head_major, mmp, qlds, page_ids, nstat); break;
      default: launch_bound_f16<64>(hfix, grid, lds, s, q, q_dtype, group, mn, mx, P, H, out, out_dtype, head_major, mmp, qlds, page_ids, nstat); break;
    }
    HKV_CHECK_LAUNCH();
    if (nmm && mmp) *nmm = (int)grid;
    return HKV_OK;
  }
  int n = 1;
  while (n < (D + 7) / 8) n <<= 1;
  const int rpb = 256 / n;
  const int64_t span = (int64_t)rpb * kBoundUnroll;
  const unsigned grid = (unsigned)std::min<int64_t>((rows + span - 1) / span, (int64_t)num_cus() * 8);
  if (k_dtype == HKV_DT_F16)
    hipLaunchKernelGGL(bound_kernel<uint16_t>, dim3(grid), dim3(256), lds, s, q, q_dtype, Hq / H,
                       (const uint16_t*)kmin, (const uint16_t*)kmax, P, H, D, out, out_dtype,
                       head_major, page_ids, nstat);
  else
    hipLaunchKernelGGL(bound_kernel<float>, dim3(grid), dim3(256), lds, s, q, q_dtype, Hq / H,
                       (const float*)kmin, (const float*)kmax, P, H, D, out, out_dtype,
                       head_major, page_ids, nstat);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

// Top-K over columns of a score matrix with page stride `ps` and head stride
// `hs` (elements).
int topk(const void* bound, int b_dtype, int64_t P, int H, int64_t ps, int64_t hs, int64_t k,
         int64_t sink_pages, int64_t* out, int64_t* n_out, hipStream_t st) {
  if (!fdt(b_dtype)) return HKV_ERR_DTYPE;
  if (P < 0 || H < 1) return HKV_ERR_SHAPE;
  const int64_t s = sink_pages < 0 ? 0 : (sink_pages > P ? P : sink_pages);
  const int64_t keff = k < 0 ? 0 : (k > P - s ? P - s : k);
  if (n_out) *n_out = s + keff;
  if (s + keff == 0) return HKV_OK;
  if (!bound || !out) return HKV_ERR_ARG;
  const int kpt = kpt_for(P - s);
#define HKV_TOPK(K)                                                                        \
  if (b_dtype == HKV_DT_F32)                                                               \
    hipLaunchKernelGGL((topk_kernel<K, ColumnF32>), dim3(H), dim3(kSelThreads), 0, st,     \
                       ColumnF32{(const float*)bound, ps, hs}, P, H, s, keff, out);       \
  else                                                                                     \
    hipLaunchKernelGGL((topk_kernel<K, ColumnF16>), dim3(H), dim3(kSelThreads), 0, st,     \
                       ColumnF16{(const uint16_t*)bound, ps, hs}, P, H, s, keff, out);
  switch (kpt) {
    case 4: HKV_TOPK(4) break;
    case 16: HKV_TOPK(16) break;
    case 64: HKV_TOPK(64) break;
    default: HKV_TOPK(0) break;
  }
#undef HKV_TOPK
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

// Union of the per-head selections as flags over pool block ids.
__global__ void __launch_bounds__(256)
mark_blocks_kernel(const int64_t* __restrict__ sel, int64_t nsel,
                   const int64_t* __restrict__ used, int64_t NU, uint8_t* __restrict__ flags,
                   int64_t nblocks) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nsel) return;
  const int64_t j = sel[i];
  if (j < 0 || j >= NU) return;
  const int64_t id = used[j];
  if (id >= 0 && id < nblocks) flags[id] = 1;
}

// One block: flagged ids in ascending order, their first positions, the
// count; the flags are cleared on the way (left all zero for the next call).
// Windows of 16 flags per thread (one 128-bit load; flags 16-byte aligned).
__global__ void __launch_bounds__(kSelThreads)
compact_blocks_kernel(uint8_t* __restrict__ flags, int64_t nblocks, int64_t block_size,
                      int64_t* __restrict__ out_ids, int64_t* __restrict__ out_first,
                      int64_t* __restrict__ n_out) {
  __shared__ uint32_t s_w[kSelWaves];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint32_t carry = 0;
  for (int64_t w0 = 0; w0 < nblocks; w0 += 16 * kSelThreads) {
    const int64_t i0 = w0 + (int64_t)tid * 16;
    uint32_t f[4] = {0u, 0u, 0u, 0u};
    const bool full = i0 + 16 <= nblocks;
    if (full) {
      const uint4 v = *reinterpret_cast<const uint4*>(flags + i0);
      f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
    } else {
      for (int k = 0; k < 16; ++k)
        if (i0 + k < nblocks && flags[i0 + k]) f[k >> 2] |= 1u << (8 * (k & 3));
    }
    uint32_t bits = 0;  // bit k: flag k set
#pragma unroll
    for (int k = 0; k < 16; ++k) bits |= ((f[k >> 2] >> (8 * (k & 3))) & 0xffu) ? (1u << k) : 0u;
    const uint32_t cnt = __builtin_popcount(bits);
    uint32_t inc = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(inc, o, 64);
      if (lane >= o) inc += y;
    }
    if (lane == 63) s_w[w] = inc;
    __syncthreads();
    uint32_t pos = carry + inc - cnt, total = 0;
    for (int i = 0; i < kSelWaves; ++i) {
      if (i < w) pos += s_w[i];
      total += s_w[i];
    }
    while (bits) {
      const int k = __builtin_ctz(bits);
      bits &= bits - 1u;
      out_ids[pos] = i0 + k;
      out_first[pos] = (i0 + k) * block_size;
      ++pos;
    }
    if (full) {
      if (f[0] | f[1] | f[2] | f[3])
        *reinterpret_cast<uint4*>(flags + i0) = make_uint4(0u, 0u, 0u, 0u);
    } else {
      for (int k = 0; k < 16; ++k)
        if (i0 + k < nblocks) flags[i0 + k] = 0;
    }
    carry += total;
    __syncthreads();  // s_w is reused by the next window
  }
  if (tid == 0) *n_out = carry;
}

// ------------------------------------------- compact (u8) page metadata
//
// Per (head, channel) over the finite statistics of all pages: lo = the
// smallest, hi = the largest; step = fl((hi - lo) / 255), raised one ulp at a
// time (at most 16) until deq(255) >= hi, with deq(q) = fl(lo + fl(q * step))
// (step = 1 when hi <= lo or nothing is finite, lo = 0 then).  A minimum
// codes as the floor of fl(fl(x - lo) / step), clamped to [0, 255] and lowered
// (at most 4 times, then 0) while deq(q) > x; a maximum as the ceiling,
// raised (at most 4 times, then 255) while deq(q) < x.  So deq(qmin) <= min
// and deq(qmax) >= max for every finite statistic, and the bound from the
// dequantised statistics is never below the fp16 one.  A non-finite
// statistic codes as 0 (minimum) / 255 (maximum).

HKV_DEV float u8_deq(uint32_t q, float lo, float step) { return __fadd_rn(lo, __fmul_rn((float)q, step)); }

HKV_DEV float u8_step(float lo, float hi) {
  if (!(hi > lo)) return 1.0f;
  float st = __fdiv_rn(__fsub_rn(hi, lo), 255.0f);
  for (int i = 0; i < 16 && u8_deq(255u, lo, st) < hi; ++i)
    st = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, st) + 1u);  // next float up
  return st;
}

HKV_DEV uint32_t u8_code(float x, float lo, float st, bool up) {
  if (!__builtin_isfinite(x)) return up ? 255u : 0u;
  float t = __fdiv_rn(__fsub_rn(x, lo), st);
  t = up ? ceilf(t) : floorf(t);
  int q = t < 0.0f ? 0 : (t > 255.0f ? 255 : (int)t);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float d = u8_deq((uint32_t)q, lo, st);
    if (up) q = (q < 255 && d < x) ? q + 1 : q;
    else q = (q > 0 && d > x) ? q - 1 : q;
  }
  const float d = u8_deq((uint32_t)q, lo, st);
  if (up) q = d < x ? 255 : q;
  else q = d > x ? 0 : q;
  return (uint32_t)q;
}

HKV_DEV float key_to_f(uint32_t k) {  // inverse of ukey for finite values
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

template <typename KT>
HKV_DEV float stat_f(KT v) {
  if constexpr (sizeof(KT) == 2) return h2f(v);
  else return v;
}

__global__ void __launch_bounds__(256) stats_u8_init_kernel(uint32_t* __restrict__ rk, int HD) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < HD; i += gridDim.x * 256) {
    rk[i] = 0xffffffffu;  // smallest key seen
    rk[HD + i] = 0u;      // largest key seen
  }
}

// Each thread keeps channels tid, tid + 256, ... over the block's pages
// (consecutive threads read consecutive channels) and folds them into the
// channel's range with device-scope atomics on the ordered keys.
template <typename KT>
__global__ void __launch_bounds__(256)
stats_u8_range_kernel(const KT* __restrict__ kmin, const KT* __restrict__ kmax, int64_t P, int HD,
                      uint32_t* __restrict__ rk) {
  for (int ch = threadIdx.x; ch < HD; ch += 256) {
    uint32_t lo = 0xffffffffu, hi = 0u;
    bool any = false;
    for (int64_t p = blockIdx.x; p < P; p += gridDim.x) {
      const float a = stat_f(kmin[p * HD + ch]), b = stat_f(kmax[p * HD + ch]);
      if (__builtin_isfinite(a)) {
        const uint32_t k = ukey(a);
        lo = k < lo ? k : lo;
        hi = k > hi ? k : hi;
        any = true;
      }
      if (__builtin_isfinite(b)) {
        const uint32_t k = ukey(b);
        lo = k < lo ? k : lo;
        hi = k > hi ? k : hi;
        any = true;
      }
    }
    if (any) {
      atomicMin(&rk[ch], lo);
      atomicMax(&rk[HD + ch], hi);
    }
  }
}

__global__ void __launch_bounds__(256)
stats_u8_params_kernel(const uint32_t* __restrict__ rk, int HD, float* __restrict__ lo,
                       float* __restrict__ step) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= HD) return;
  float l = 0.0f, h = 0.0f;
  if (rk[i] != 0xffffffffu) {
    l = key_to_f(rk[i]);
    h = key_to_f(rk[HD + i]);
  }
  lo[i] = l;
  step[i] = u8_step(l, h);
}

// Four statistics per thread (HD is a multiple of 4), one 32-bit store each.
template <typename KT>
__global__ void __launch_bounds__(256)
stats_u8_quant_kernel(const KT* __restrict__ kmin, const KT* __restrict__ kmax, int64_t n4, int HD,
                      const float* __restrict__ lo, const float* __restrict__ step,
                      uint8_t* __restrict__ qmin, uint8_t* __restrict__ qmax) {
  for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < n4; j += (int64_t)gridDim.x * 256) {
    const int64_t i0 = 4 * j;
    const int ch0 = (int)(i0 % HD);
    uint32_t wn = 0, wx = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float l = lo[ch0 + e], st = step[ch0 + e];
      wn |= u8_code(stat_f(kmin[i0 + e]), l, st, false) << (8 * e);
      wx |= u8_code(stat_f(kmax[i0 + e]), l, st, true) << (8 * e);
    }
    reinterpret_cast<uint32_t*>(qmin)[j] = wn;
    reinterpret_cast<uint32_t*>(qmax)[j] = wx;
  }
}

// Group-summed bound from the u8 metadata, (H, P) fp32 scores, plus each
// block's key range (mm) when given.  Shapes: D a multiple of 8 with
// G = D / 8 a power of two <= 64 and H dividing 64 / G (a lane's head is
// fixed), P * H * D < 2^32.
int page_bound_u8(const void* q, int q_dtype, int Hq, const uint8_t* kmin, const uint8_t* kmax,
                  const float* lo, const float* step, int64_t P, int H, int D, float* out,
                  hipStream_t s, uint2* mm, int* nmm) {
  if (nmm) *nmm = 0;
  if (!fdt(q_dtype) && q_dtype != HKV_DT_BF16) return HKV_ERR_DTYPE;
  if (P < 0 || H < 1 || D < 8 || D % 8 || Hq < H || Hq % H) return HKV_ERR_SHAPE;
  const int G = D / 8;
  if ((G & (G - 1)) || G > 64 || (256 / G) % H) return HKV_ERR_SHAPE;  // a lane's head fixed
  if (P * H * D >= ((int64_t)1 << 32) || P * H >= ((int64_t)1 << 31)) return HKV_ERR_SHAPE;
  if (P == 0) return HKV_OK;
  if (!q || !kmin || !kmax || !lo || !step || !out) return HKV_ERR_ARG;
  if ((((uintptr_t)kmin | (uintptr_t)kmax) & 7u) || (((uintptr_t)lo | (uintptr_t)step) & 3u))
    return HKV_ERR_ARG;
  size_t lds = sizeof(float) * 2 * H * D;
  if (lds > 64 * 1024) return HKV_ERR_SHAPE;
  size_t qraw = q_raw_lds(q, q_dtype, Hq, D);
  if (lds + qraw > 64 * 1024) qraw = 0;
  const int qlds = qraw != 0;
  lds += qraw;
  const int64_t rows = P * H;
  const int64_t span = (int64_t)(256 / G) * kBoundUnrollF16;
  const unsigned grid = (unsigned)std::min<int64_t>((rows + span - 1) / span, (int64_t)num_cus() * 4);
  uint2* mmp = (mm && H <= kMaxMMHeads) ? mm : nullptr;
  const int group = Hq / H;
#define HKV_BU8(GG)                                                                                 \
  hipLaunchKernelGGL((bound_u8_kernel<GG>), dim3(grid), dim3(256), lds, s, q, q_dtype, group, kmin, \
                     kmax, lo, step, P, H, out, mmp, qlds)
  switch (G) {
    case 1: HKV_BU8(1); break;
    case 2: HKV_BU8(2); break;
    case 4: HKV_BU8(4); break;
    case 8: HKV_BU8(8); break;
    case 16: HKV_BU8(16); break;
    case 32: HKV_BU8(32); break;
    default: HKV_BU8(64); break;
  }
#undef HKV_BU8
  HKV_CHECK_LAUNCH();
  if (nmm && mmp) *nmm = (int)grid;
  return HKV_OK;
}

}  // namespace

namespace {

// Workspace of hkv_quest_select's multi-block top-K (NB = 0: not used).
struct SelectWs {
  int NB, kpt;
  size_t ctr_off, thr_off, mm_off, hist_off, meta_off, wcand_off, wmeta_off, bytes;
};

int select_after_bound(const float* scores, int64_t P, int H, int64_t k, int64_t sink_pages, int64_t s,
                       int64_t keff, int64_t* out, const struct SelectWs& lay, bool mb, char* ws,
                       int nmm, hipStream_t st);

SelectWs select_ws_layout(int64_t P, int H) {
  SelectWs l{};
  const int64_t n = P;  // candidates are at most P
  if (H < 1 || H > kMaxMMHeads || n < 4 * (int64_t)kMBThreads * 8) return l;  // small: one block per head
  int kpt = 8;
  int64_t nb = (n + kMBThreads * 8 - 1) / (kMBThreads * 8);
  if (nb > kMBMaxSlices) {
    kpt = 32;
    nb = (n + kMBThreads * 32 - 1) / (kMBThreads * 32);
    if (nb > kMBMaxSlices) return l;
  }
  auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
  l.NB = (int)nb;
  l.kpt = kpt;
  l.ctr_off = 0;
  l.thr_off = al(sizeof(uint32_t) * 2 * H);  // arrival, then departure counters
  l.mm_off = l.thr_off + al(sizeof(uint32_t) * 4 * H);
  l.hist_off = l.mm_off + al(sizeof(uint2) * (size_t)num_cus() * 4 * H);
  l.meta_off = l.hist_off + al(sizeof(uint32_t) * (size_t)H * nb * (kMBBins / 2));
  l.wcand_off = l.meta_off + al(sizeof(int) * 2 * (size_t)H * nb);
  l.wmeta_off = l.wcand_off + al(sizeof(uint32_t) * (size_t)H * nb * kMBWin);
  l.bytes = l.wmeta_off + al(sizeof(int) * 4 * (size_t)H * nb);
  return l;
}

}  // namespace

extern "C" size_t hkv_quest_select_workspace_bytes(int64_t P, int H) {
  const SelectWs l = select_ws_layout(P, H);
  return l.NB ? l.bytes : 256;
}

extern "C" int hkv_quest_page_bound(const void* q, int q_dtype, int Hq, const void* kmin,
                                    const void* kmax, int k_dtype, int64_t P, int H, int D,
                                    void* out, int out_dtype, void* stream) {
  return page_bound(q, q_dtype, Hq, kmin, kmax, k_dtype, P, H, D, out, out_dtype, 0,
                    (hipStream_t)stream);
}

// The selectors keep all state in LDS and registers; a nominal size is
// returned so callers that always pass a workspace keep working.
extern "C" size_t hkv_quest_topk_workspace_bytes(int64_t P, int H) {
  (void)P;
  (void)H;
  return 256;
}

extern "C" int hkv_quest_topk(const void* bound, int b_dtype, int64_t P, int H, int64_t k,
                              int64_t sink_pages, int64_t* out, int64_t* n_out, void* workspace,
                              size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  return topk(bound, b_dtype, P, H, H, 1, k, sink_pages, out, n_out, (hipStream_t)stream);
}

extern "C" int hkv_quest_select(const void* q, int q_dtype, int Hq, const void* kmin,
                                const void* kmax, int k_dtype, int64_t P, int H, int D, int64_t k,
                                int64_t sink_pages, float* scores, int64_t* out, int64_t* n_out,
                                void* workspace, size_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
  if (!fdt(q_dtype) && q_dtype != HKV_DT_BF16) return HKV_ERR_DTYPE;
  if (!fdt(k_dtype)) return HKV_ERR_DTYPE;
  if (P < 0 || H < 1 || D < 1 || D > 512 || Hq < H || Hq % H) return HKV_ERR_SHAPE;
  const int64_t s = sink_pages < 0 ? 0 : (sink_pages > P ? P : sink_pages);
  const int64_t keff = k < 0 ? 0 : (k > P - s ? P - s : k);
  if (n_out) *n_out = s + keff;
  if (P == 0) return HKV_OK;
  if (!q || !kmin || !kmax || !scores || !out) return HKV_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const SelectWs lay = select_ws_layout(P, H);
  const bool mb = workspace && workspace_bytes >= lay.bytes && lay.NB > 0 && keff > 0 &&
                  ((uintptr_t)workspace & 255u) == 0;
  char* ws = (char*)workspace;
  int nmm = 0;
  const int rc = page_bound(q, q_dtype, Hq, kmin, kmax, k_dtype, P, H, D, scores, HKV_DT_F32, 1, st,
                            nullptr, 0, mb ? (uint2*)(ws + lay.mm_off) : nullptr, &nmm);
  if (rc != HKV_OK) return rc;
  return select_after_bound(scores, P, H, k, sink_pages, s, keff, out, lay, mb, ws, nmm, st);
}

extern "C" int hkv_quest_select_paged(const void* q, int q_dtype, int Hq, const hkv_paged_side* kside,
                                      const int64_t* block_table, int64_t P, int64_t k,
                                      int64_t sink_pages, float* scores, int64_t* out,
                                      int64_t* n_out, void* workspace, size_t workspace_bytes,
                                      void* stream) {
  if (!kside) return HKV_ERR_ARG;
  const int H = kside->heads, D = 128, k_dtype = HKV_DT_F16;
  const int64_t num_blocks = kside->num_blocks;
  const void* kmin = kside->kmin;
  const void* kmax = kside->kmax;
  if (!fdt(q_dtype) && q_dtype != HKV_DT_BF16) return HKV_ERR_DTYPE;
  if (P < 0 || num_blocks < 0 || H < 1 || H > 16 || Hq < H || Hq % H) return HKV_ERR_SHAPE;
  const int64_t s = sink_pages < 0 ? 0 : (sink_pages > P ? P : sink_pages);
  const int64_t keff = k < 0 ? 0 : (k > P - s ? P - s : k);
  if (n_out) *n_out = s + keff;
  if (P == 0) return HKV_OK;
  if (!q || !kmin || !kmax || !scores || !out || !block_table) return HKV_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const SelectWs lay = select_ws_layout(P, H);
  const bool mb = workspace && workspace_bytes >= lay.bytes && lay.NB > 0 && keff > 0 &&
                  ((uintptr_t)workspace & 255u) == 0;
  char* ws = (char*)workspace;
  int nmm = 0;
  const int rc = page_bound(q, q_dtype, Hq, kmin, kmax, k_dtype, P, H, D, scores, HKV_DT_F32, 1, st,
                            block_table, num_blocks, mb ? (uint2*)(ws + lay.mm_off) : nullptr, &nmm);
  if (rc != HKV_OK) return rc;
  return select_after_bound(scores, P, H, k, sink_pages, s, keff, out, lay, mb, ws, nmm, st);
}

extern "C" int hkv_quest_select_u8(const void* q, int q_dtype, int Hq, const uint8_t* kmin,
                                   const uint8_t* kmax, const float* lo, const float* step, int64_t P,
                                   int H, int D, int64_t k, int64_t sink_pages, float* scores,
                                   int64_t* out, int64_t* n_out, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  if (P < 0 || H < 1 || D < 1 || D > 512 || Hq < H || Hq % H) return HKV_ERR_SHAPE;
  const int64_t s = sink_pages < 0 ? 0 : (sink_pages > P ? P : sink_pages);
  const int64_t keff = k < 0 ? 0 : (k > P - s ? P - s : k);
  if (n_out) *n_out = s + keff;
  if (P == 0) return HKV_OK;
  if (!scores || !out) return HKV_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  const SelectWs lay = select_ws_layout(P, H);
  const bool mb = workspace && workspace_bytes >= lay.bytes && lay.NB > 0 && keff > 0 &&
                  ((uintptr_t)workspace & 255u) == 0;
  char* ws = (char*)workspace;
  int nmm = 0;
  const int rc = page_bound_u8(q, q_dtype, Hq, kmin, kmax, lo, step, P, H, D, scores, st,
                               mb ? (uint2*)(ws + lay.mm_off) : nullptr, &nmm);
  if (rc != HKV_OK) return rc;
  return select_after_bound(scores, P, H, k, sink_pages, s, keff, out, lay, mb, ws, nmm, st);
}

namespace {

// The top-K half of a select: the multi-block top-K when the workspace and
// the bound kernel's key ranges allow it, else the single-block selector.
int select_after_bound(const float* scores, int64_t P, int H, int64_t k, int64_t sink_pages, int64_t s,
                       int64_t keff, int64_t* out, const SelectWs& lay, bool mb, char* ws, int nmm,
                       hipStream_t st) {
  if (!mb || nmm == 0) return topk(scores, HKV_DT_F32, P, H, 1, P, k, sink_pages, out, nullptr, st);
  MBWork w;
  w.ctr = (uint32_t*)(ws + lay.ctr_off);
  w.leave = w.ctr + H;
  w.mm = (const uint2*)(ws + lay.mm_off);
  w.nmm = nmm;
  w.hist = (uint32_t*)(ws + lay.hist_off);
  w.meta = (int*)(ws + lay.meta_off);
  w.thr = (uint32_t*)(ws + lay.thr_off);
  w.wcand = (uint32_t*)(ws + lay.wcand_off);
  w.wmeta = (int*)(ws + lay.wmeta_off);
  const dim3 grid((unsigned)lay.NB, (unsigned)H);
  // the fused form's blocks wait for one another: only where every block of
  // the grid has a CU of its own
  const bool fused = (int64_t)lay.NB * H <= (int64_t)num_cus();
  if (lay.kpt == 8) {
    if (fused) {
      hipLaunchKernelGGL((topk_mb_hist<8, true>), grid, dim3(kMBThreads), 0, st, scores, P, s, keff, out, H, w);
    } else {
      hipLaunchKernelGGL((topk_mb_hist<8, false>), grid, dim3(kMBThreads), 0, st, scores, P, s, keff, out, H, w);
      HKV_CHECK_LAUNCH();
      hipLaunchKernelGGL((topk_mb_write<8>), grid, dim3(kMBThreads), 0, st, scores, P, s, out, H, w);
    }
  } else {
    if (fused) {
      hipLaunchKernelGGL((topk_mb_hist<32, true>), grid, dim3(kMBThreads), 0, st, scores, P, s, keff, out, H, w);
    } else {
      hipLaunchKernelGGL((topk_mb_hist<32, false>), grid, dim3(kMBThreads), 0, st, scores, P, s, keff, out, H, w);
      HKV_CHECK_LAUNCH();
      hipLaunchKernelGGL((topk_mb_write<32>), grid, dim3(kMBThreads), 0, st, scores, P, s, out, H, w);
    }
  }
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

}  // namespace

extern "C" size_t hkv_quest_page_stats_u8_workspace_bytes(int H, int D) {
  return H < 1 || D < 1 ? 0 : sizeof(uint32_t) * 2 * (size_t)H * D;
}

extern "C" int hkv_quest_page_stats_u8(const void* kmin, const void* kmax, int dtype, int64_t P, int H,
                                       int D, uint8_t* qmin, uint8_t* qmax, float* lo, float* step,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  if (!fdt(dtype)) return HKV_ERR_DTYPE;
  if (P < 0 || H < 1 || D < 1 || D % 4) return HKV_ERR_SHAPE;
  const int HD = H * D;
  if (!lo || !step || !workspace) return HKV_ERR_ARG;
  if (workspace_bytes < hkv_quest_page_stats_u8_workspace_bytes(H, D) || ((uintptr_t)workspace & 3u))
    return HKV_ERR_WORKSPACE;
  if (P > 0 && (!kmin || !kmax || !qmin || !qmax)) return HKV_ERR_ARG;
  if (((uintptr_t)qmin | (uintptr_t)qmax) & 3u) return HKV_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  uint32_t* rk = (uint32_t*)workspace;
  const unsigned gch = (unsigned)((HD + 255) / 256);
  hipLaunchKernelGGL(stats_u8_init_kernel, dim3(gch), dim3(256), 0, st, rk, HD);
  HKV_CHECK_LAUNCH();
  if (P > 0) {
    const unsigned gr = (unsigned)std::min<int64_t>(P, (int64_t)num_cus() * 4);
    if (dtype == HKV_DT_F16)
      hipLaunchKernelGGL(stats_u8_range_kernel<uint16_t>, dim3(gr), dim3(256), 0, st,
                         (const uint16_t*)kmin, (const uint16_t*)kmax, P, HD, rk);
    else
      hipLaunchKernelGGL(stats_u8_range_kernel<float>, dim3(gr), dim3(256), 0, st, (const float*)kmin,
                         (const float*)kmax, P, HD, rk);
    HKV_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(stats_u8_params_kernel, dim3(gch), dim3(256), 0, st, rk, HD, lo, step);
  HKV_CHECK_LAUNCH();
  if (P > 0) {
    const int64_t n4 = P * HD / 4;
    const unsigned gq = (unsigned)std::min<int64_t>((n4 + 255) / 256, (int64_t)num_cus() * 16);
    if (dtype == HKV_DT_F16)
      hipLaunchKernelGGL(stats_u8_quant_kernel<uint16_t>, dim3(gq), dim3(256), 0, st,
                         (const uint16_t*)kmin, (const uint16_t*)kmax, n4, HD, lo, step, qmin, qmax);
    else
      hipLaunchKernelGGL(stats_u8_quant_kernel<float>, dim3(gq), dim3(256), 0, st, (const float*)kmin,
                         (const float*)kmax, n4, HD, lo, step, qmin, qmax);
    HKV_CHECK_LAUNCH();
  }
  return HKV_OK;
}

extern "C" int hkv_quest_select_blocks(const void* q, int q_dtype, int H, const void* kmin,
                                       const void* kmax, int k_dtype, int64_t num_blocks, int D,
                                       const int64_t* used_block_ids, int64_t NU, int64_t top_k,
                                       int64_t sink_blocks, int64_t block_size, float* scores,
                                       int64_t* sel, uint8_t* flags, int64_t* out_ids,
                                       int64_t* out_first_pos, int64_t* n_selected,
                                       void* stream) {
  if (NU < 0 || num_blocks < 0 || H < 1 || H > 64 || block_size < 1) return HKV_ERR_SHAPE;
  if (!n_selected) return HKV_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (NU == 0 || num_blocks == 0) {
    hipLaunchKernelGGL(compact_blocks_kernel, dim3(1), dim3(kSelThreads), 0, st, flags,
                       (int64_t)0, block_size, out_ids, out_first_pos, n_selected);
    HKV_CHECK_LAUNCH();
    return HKV_OK;
  }
  if (!q || !kmin || !kmax || !used_block_ids || !scores || !sel || !flags || !out_ids ||
      !out_first_pos)
    return HKV_ERR_ARG;
  if ((uintptr_t)flags & 15u) return HKV_ERR_ARG;
  int rc = page_bound(q, q_dtype, H, kmin, kmax, k_dtype, NU, H, D, scores, HKV_DT_F32, 1, st,
                      used_block_ids, num_blocks);
  if (rc != HKV_OK) return rc;
  int64_t n = 0;
  rc = topk(scores, HKV_DT_F32, NU, H, 1, NU, top_k, sink_blocks, sel, &n, st);
  if (rc != HKV_OK) return rc;
  const int64_t nsel = n * H;
  if (nsel > 0)
    hipLaunchKernelGGL(mark_blocks_kernel, dim3((unsigned)((nsel + 255) / 256)), dim3(256), 0, st,
                       sel, nsel, used_block_ids, NU, flags, num_blocks);
  hipLaunchKernelGGL(compact_blocks_kernel, dim3(1), dim3(kSelThreads), 0, st, flags, num_blocks,
                     block_size, out_ids, out_first_pos, n_selected);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

namespace {

// The ragged selection of both layouts: compact (bt NULL: sequence b's
// statistics are rows page_offsets[b].. of kmin / kmax) or paged (logical
// page p of sequence b at row bt[bt_offsets[b] + p] of the pool's nstat
// blocks; a lane's head must be fixed).
int select_ragged(const void* q, int q_dtype, int B, int Hq, const void* kmin, const void* kmax,
                  int k_dtype, int H, int D, const int64_t* page_offsets, const int64_t* top_k,
                  int64_t sink_pages, float* scores, int64_t* out, int64_t* out_offsets,
                  const int64_t* bt, const int64_t* bt_offsets, int64_t nstat, hipStream_t st) {
  if (B < 1 || B > kMaxSeqs) return HKV_ERR_SHAPE;
  if (!page_offsets || !top_k || !out_offsets || (bt && !bt_offsets)) return HKV_ERR_ARG;
  if (q_dtype != HKV_DT_F16 && q_dtype != HKV_DT_F32 && q_dtype != HKV_DT_BF16) return HKV_ERR_DTYPE;
  if (k_dtype != HKV_DT_F16) return HKV_ERR_DTYPE;
  if (H < 1 || Hq < H || Hq % H || D < 8 || D % 8 || D > 512) return HKV_ERR_SHAPE;
  const int G = D / 8;
  if (G & (G - 1)) return HKV_ERR_SHAPE;
  Segs sg;
  sg.nseg = B;
  int64_t maxn = 0;
  if (page_offsets[0] != 0) return HKV_ERR_ARG;
  out_offsets[0] = 0;
  for (int b = 0; b < B; ++b) {
    const int64_t P = page_offsets[b + 1] - page_offsets[b];
    if (P < 0) return HKV_ERR_ARG;
    sg.off[b] = page_offsets[b];
    sg.k[b] = top_k[b];
    sg.bt0[b] = bt ? bt_offsets[b] : 0;
    if (sg.bt0[b] < 0) return HKV_ERR_ARG;
    const int64_t s = sink_pages < 0 ? 0 : (sink_pages > P ? P : sink_pages);
    const int64_t keff = top_k[b] < 0 ? 0 : (top_k[b] > P - s ? P - s : top_k[b]);
    out_offsets[b + 1] = out_offsets[b] + s + keff;
    maxn = std::max<int64_t>(maxn, P - s);
  }
  sg.off[B] = page_offsets[B];
  for (int b = 0; b <= B; ++b) sg.out_off[b] = out_offsets[b];
  const int64_t Ptot = page_offsets[B];
  if (Ptot * H >= ((int64_t)1 << 31) || Ptot * H * D >= ((int64_t)1 << 32)) return HKV_ERR_SHAPE;
  // paged: the pool's statistics rows are addressed in 32 bits, a lane's head
  // fixed (the heads divide a block's rows per row group, 256 / G)
  if (bt && (nstat < 1 || nstat * H * D >= ((int64_t)1 << 31) || G > 64 || (256 / G) % H))
    return HKV_ERR_SHAPE;
  if (Ptot == 0) return HKV_OK;
  if (!q || !kmin || !kmax || !scores || (out_offsets[B] > 0 && !out)) return HKV_ERR_ARG;
  if (((uintptr_t)kmin | (uintptr_t)kmax) & 15u) return HKV_ERR_ARG;
  const size_t lds = sizeof(float) * 2 * H * D;
  if (lds > 64 * 1024) return HKV_ERR_SHAPE;
  // blocks per sequence: num_cus * 4 in all, shared in proportion to the
  // sequences' pages (at least one for a non-empty sequence, at most one per
  // row group); an empty sequence gets none
  const int64_t span = (int64_t)(256 / G) * kBoundUnrollF16;
  const int64_t nbt = (int64_t)num_cus() * 4;
  sg.blk[0] = 0;
  for (int b = 0; b < B; ++b) {
    const int64_t rows_b = (page_offsets[b + 1] - page_offsets[b]) * H;
    int64_t nb = 0;
    if (rows_b > 0) {
      nb = (nbt * rows_b + Ptot * H / 2) / (Ptot * H);
      nb = std::max<int64_t>(1, std::min<int64_t>(nb, (rows_b + span - 1) / span));
    }
    sg.blk[b + 1] = sg.blk[b] + (int)nb;
  }
  const unsigned gx = (unsigned)sg.blk[B];
  const int64_t q_bytes = (int64_t)Hq * D * (q_dtype == HKV_DT_F32 ? 4 : 2);
  // a lane's head is fixed when the heads divide the rows of a block's row
  // group (256 / G): a lane keeps its row of every group
  const bool hfix = (256 / G) % H == 0;
  auto mn = (const uint16_t*)kmin;
  auto mx = (const uint16_t*)kmax;
  const int group = Hq / H;
  size_t qraw = q_raw_lds(q, q_dtype, Hq, D);
  if (lds + qraw > 64 * 1024) qraw = 0;
  const int qlds = qraw != 0;
  const size_t ldsq = lds + qraw;
#define HKV_RB(GG)                                                                                \
  if (hfix)                                                                                       \
    hipLaunchKernelGGL((bound_f16_ragged_kernel<GG, true>), dim3(gx), dim3(256), ldsq, st,        \
                       (const char*)q, q_bytes, q_dtype, group, mn, mx, H, scores, sg, qlds, bt,  \
                       nstat);                                                                    \
  else                                                                                            \
    hipLaunchKernelGGL((bound_f16_ragged_kernel<GG, false>), dim3(gx), dim3(256), ldsq, st,       \
                       (const char*)q, q_bytes, q_dtype, group, mn, mx, H, scores, sg, qlds,     \
                       nullptr, 0);
  switch (G) {
    case 1: HKV_RB(1) break;
    case 2: HKV_RB(2) break;
    case 4: HKV_RB(4) break;
    case 8: HKV_RB(8) break;
    case 16: HKV_RB(16) break;
    case 32: HKV_RB(32) break;
    default: HKV_RB(64) break;
  }
#undef HKV_RB
  HKV_CHECK_LAUNCH();
  if (out_offsets[B] == 0) return HKV_OK;
  const int kpt = kpt_for(maxn);
  switch (kpt) {
    case 4: hipLaunchKernelGGL((topk_ragged_kernel<4>), dim3(H, B), dim3(kSelThreads), 0, st, scores, H, sink_pages, out, sg); break;
    case 16: hipLaunchKernelGGL((topk_ragged_kernel<16>), dim3(H, B), dim3(kSelThreads), 0, st, scores, H, sink_pages, out, sg); break;
    case 64: hipLaunchKernelGGL((topk_ragged_kernel<64>), dim3(H, B), dim3(kSelThreads), 0, st, scores, H, sink_pages, out, sg); break;
    default: hipLaunchKernelGGL((topk_ragged_kernel<0>), dim3(H, B), dim3(kSelThreads), 0, st, scores, H, sink_pages, out, sg); break;
  }
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

}  // namespace

extern "C" int hkv_quest_select_ragged(const void* q, int q_dtype, int B, int Hq, const void* kmin,
                                       const void* kmax, int k_dtype, int H, int D,
                                       const int64_t* page_offsets, const int64_t* top_k,
                                       int64_t sink_pages, float* scores, int64_t* out,
                                       int64_t* out_offsets, void* stream) {
  return select_ragged(q, q_dtype, B, Hq, kmin, kmax, k_dtype, H, D, page_offsets, top_k, sink_pages,
                       scores, out, out_offsets, nullptr, nullptr, 0, (hipStream_t)stream);
}

extern "C" int hkv_quest_select_paged_ragged(const void* q, int q_dtype, int B, int Hq,
                                             const hkv_paged_side* kside, const int64_t* block_table,
                                             const int64_t* bt_offsets, const int64_t* page_offsets,
                                             const int64_t* top_k, int64_t sink_pages, float* scores,
                                             int64_t* out, int64_t* out_offsets, void* stream) {
  if (!kside || !block_table) return HKV_ERR_ARG;
  if (kside->heads < 1 || kside->heads > 16) return HKV_ERR_SHAPE;
  return select_ragged(q, q_dtype, B, Hq, kside->kmin, kside->kmax, HKV_DT_F16, kside->heads, 128,
                       page_offsets, top_k, sink_pages, scores, out, out_offsets, block_table,
                       bt_offsets, kside->num_blocks, (hipStream_t)stream);
}

// ------------------------------------------------ allocation-free selection
//
// hkv_quest_select_noalloc: hkv_quest_select with its workspace in a fixed
// file-scope device array instead of a caller buffer, for callers that cannot
// allocate device memory (code under graph capture, serving loops).  Each GPU
// holds its own copy of the array for the life of the process; its address on
// a device is looked up once, with that device current, and used for every
// later call there.  The array's name is never passed to a kernel or copy
// from host code: on the host it only names the symbol.

namespace {

constexpr size_t kSelectScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kSelectScratchBytes];

constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchDevices];

__global__ void __launch_bounds__(256) zero_words_kernel(uint4* __restrict__ p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// The device address of the current device's scratch.  The first call on a
// device looks it up and clears it with a fill kernel on `st` (ordered before
// the caller's kernels on that stream; a fill kernel, not a memset, so the
// call may also be captured into a graph).
static int scratch_for_current_device(hipStream_t st, char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) return HKV_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return HKV_ERR_LAUNCH;
    hipLaunchKernelGGL(zero_words_kernel, dim3(256), dim3(256), 0, st, (uint4*)p,
                       kSelectScratchBytes / 16);
    HKV_CHECK_LAUNCH();
    g_scratch_ptr[dev] = p;
  }
  *out = (char*)g_scratch_ptr[dev];
  return HKV_OK;
}

}  // namespace

extern "C" size_t hkv_quest_select_noalloc_max_workspace(void) { return kSelectScratchBytes; }

extern "C" int hkv_quest_select_noalloc(const void* q, int q_dtype, int Hq, const void* kmin,
                                        const void* kmax, int k_dtype, int64_t P, int H, int D,
                                        int64_t k, int64_t sink_pages, float* scores, int64_t* out,
                                        int64_t* n_out, void* stream) {
  if (!fdt(q_dtype) && q_dtype != HKV_DT_BF16) return HKV_ERR_DTYPE;
  if (!fdt(k_dtype)) return HKV_ERR_DTYPE;
  if (P < 0 || H < 1 || D < 1 || D > 512 || Hq < H || Hq % H) return HKV_ERR_SHAPE;
  const SelectWs lay = select_ws_layout(P, H);
  if (lay.NB > 0 && lay.bytes > kSelectScratchBytes) return HKV_ERR_SCRATCH;
  const int64_t s = sink_pages < 0 ? 0 : (sink_pages > P ? P : sink_pages);
  const int64_t keff = k < 0 ? 0 : (k > P - s ? P - s : k);
  if (n_out) *n_out = s + keff;
  if (P == 0) return HKV_OK;
  if (!q || !kmin || !kmax || !scores || !out) return HKV_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  char* ws = nullptr;
  if (lay.NB > 0) {
    const int rc = scratch_for_current_device(st, &ws);
    if (rc != HKV_OK) return rc;
  }
  const bool mb = ws != nullptr && keff > 0;
  int nmm = 0;
  const int rc = page_bound(q, q_dtype, Hq, kmin, kmax, k_dtype, P, H, D, scores, HKV_DT_F32, 1, st,
                            nullptr, 0, mb ? (uint2*)(ws + lay.mm_off) : nullptr, &nmm);
  if (rc != HKV_OK) return rc;
  return select_after_bound(scores, P, H, k, sink_pages, s, keff, out, lay, mb, ws, nmm, st);
}

