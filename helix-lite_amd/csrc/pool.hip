// pool.hip -- the compact KV pool's write and selective read.
//
// Pool layout (the reference's, so the pool's tensors are a drop-in:
// src/kvquant/compact_pool.py:418-444): per layer codes u8, outlier values
// fp16 (0 where not an outlier) and outlier mask u8, each (NB, BS, H, D);
// per-block statistics of the reconstructed K, k_min / k_max (NB, H, D)
// fp32.  A slot s = block * BS + position addresses one token row.
//
// Write (src/kvquant/compact_pool.py:447-489, kernels :160-287): token t of a
// (T, H, D) batch goes to slot slot_mapping[t]; slots < 0 are padding and
// skipped (:184-186, :245-247).  V's per-token scale row is
// min(abs_positions[t], T_cal - 1) (:467).  K's block statistics take the
// min / max of the reconstructed value (the input for outliers, the pole
// otherwise, in fp32) with -0 ordered below +0.
//
// Read (unpack_to_staging, :492-537, kernels :292-395): kept block k with pool
// id block_ids[k] is dequantised into staging[k] (BS, H, D) fp16; V's scale
// row of position p is min(first_pos[k] + p, T_cal - 1).
//
// Both directions also bounds-check what the reference does not: slots at or
// beyond NB * BS are skipped and block ids outside [0, NB) produce zero rows,
// so a bad index can never address memory outside the pool.
#include "nuq_core.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTokPerThread = 4;  // consecutive tokens per thread (stat merging)

// Order-preserving fp32 min / max through integer atomics (no float atomics
// needed).  The sign bit picks the integer view in which the order is
// monotone: non-negative floats order as signed ints, negative ones reversed
// as unsigned ints; -0 sorts just below +0.
HKV_DEV void atomic_min_f32(float* a, float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  if (!(b >> 31)) atomicMin(reinterpret_cast<int*>(a), (int)b);
  else atomicMax(reinterpret_cast<unsigned int*>(a), b);
}
HKV_DEV void atomic_max_f32(float* a, float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  if (!(b >> 31)) atomicMax(reinterpret_cast<int*>(a), (int)b);
  else atomicMin(reinterpret_cast<unsigned int*>(a), b);
}
// Ordered key of an fp32 value for local comparisons, with the same order.
HKV_DEV int32_t okey(float v) {
  const int32_t b = __builtin_bit_cast(int32_t, v);
  return b >= 0 ? b : -(b & 0x7fffffff) - 1;
}

// Block (token tile, head h): each thread owns 8 consecutive channels of
// kTokPerThread consecutive tokens.  STATS (K only): the thread merges the
// reconstructed values of its tokens while they stay in one pool block and
// issues one atomic pair per channel per pool block it touched.
template <int NB, bool PT, int G, bool STATS>
__global__ void __launch_bounds__(kThreads)
pool_write_kernel(const uint16_t* __restrict__ x, int64_t T, int H, hkv_nuq_scales sc,
                  const int64_t* __restrict__ slots, int64_t nslots, int bs,
                  uint8_t* __restrict__ codes, uint16_t* __restrict__ outv,
                  uint8_t* __restrict__ outm, float* __restrict__ kmin, float* __restrict__ kmax) {
  constexpr int R = kThreads / G;
  constexpr int D = 8 * G;
  const int tid = threadIdx.x, cg = tid % G, rl = tid / G;
  const int h = blockIdx.y;
  const int64_t tbase = ((int64_t)blockIdx.x * R + rl) * kTokPerThread;
  const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;
  const SlowInfo si = slow_info(sc);
  Search2<NB> S[PT ? 1 : 4];
  const int64_t ktab0 = (int64_t)h * D + 8 * cg;
  if constexpr (!PT) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      load_search_pair<NB>(tabs + ktab0 + 2 * j, tabs + ktab0 + 2 * j + 1, S[j]);
  }
  float mn[8], mx[8];
  int64_t cur_blk = -1;
  auto flush = [&]() {
    if constexpr (STATS) {
      if (cur_blk >= 0) {
        float* a = kmin + (cur_blk * H + h) * D + 8 * cg;
        float* b = kmax + (cur_blk * H + h) * D + 8 * cg;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          atomic_min_f32(a + e, mn[e]);
          atomic_max_f32(b + e, mx[e]);
        }
      }
    }
  };
  for (int k = 0; k < kTokPerThread; ++k) {
    const int64_t t = tbase + k;
    if (t >= T) break;
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= nslots) continue;
    int64_t tab0 = ktab0;
    if constexpr (PT) {
      tab0 = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
      load_search_bcast<NB>(tabs + tab0, S[0]);
    }
    const uint4 xv = *reinterpret_cast<const uint4*>(x + (t * H + h) * D + 8 * cg);
    uint32_t c[4], om[4];
    if constexpr (PT) quant8<NB, PT>(xv, S, si, RowTab{tab0}, c, om);
    else quant8<NB, PT>(xv, S, si, ChanTab{tab0}, c, om);
    const int64_t off = (slot * H + h) * D + 8 * cg;
    uint2 cb, mb;
    cb.x = lanes_to_bytes(c[0]) | (lanes_to_bytes(c[1]) << 16);
    cb.y = lanes_to_bytes(c[2]) | (lanes_to_bytes(c[3]) << 16);
    mb.x = lanes_to_bytes(om[0] & 0x00010001u) | (lanes_to_bytes(om[1] & 0x00010001u) << 16);
    mb.y = lanes_to_bytes(om[2] & 0x00010001u) | (lanes_to_bytes(om[3] & 0x00010001u) << 16);
    *reinterpret_cast<uint2*>(codes + off) = cb;
    *reinterpret_cast<uint4*>(outv + off) =
        make_uint4(xv.x & om[0], xv.y & om[1], xv.z & om[2], xv.w & om[3]);
    *reinterpret_cast<uint2*>(outm + off) = mb;
    if constexpr (STATS) {
      const int64_t blk = slot / bs;
      if (blk != cur_blk) {
        flush();
        cur_blk = blk;
#pragma unroll
        for (int e = 0; e < 8; ++e) { mn[e] = __builtin_inff(); mx[e] = -__builtin_inff(); }
      }
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t code = (c[e >> 1] >> (16 * (e & 1))) & 0xffu;
        const bool o = (om[e >> 1] >> (16 * (e & 1))) & 1u;
        const float r = o ? h2f((uint16_t)(xw[e >> 1] >> (16 * (e & 1))))
                          : load_scale(sc.poles, sc.poles_dtype, (ktab0 + e) * sc.levels + code);
        if (okey(r) < okey(mn[e])) mn[e] = r;
        if (okey(r) > okey(mx[e])) mx[e] = r;
      }
    }
  }
  flush();
}

// Gather-dequant of kept blocks: grid (NK, H); block_size rows per kept block;
// thread = 8 channels of one row.
template <bool PT>
__global__ void __launch_bounds__(kThreads)
pool_gather_kernel(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ outv,
                   const uint8_t* __restrict__ outm, int64_t nblocks, int bs, int H, int D,
                   hkv_nuq_scales sc, const int64_t* __restrict__ block_ids,
                   const int64_t* __restrict__ first_pos, uint16_t* __restrict__ staging) {
  const int G = D / 8;
  const int kk = blockIdx.x, h = blockIdx.y;
  const int L = sc.levels;
  const int64_t bid = block_ids[kk];
  const bool ok = bid >= 0 && bid < nblocks;
  const int64_t p0 = PT ? first_pos[kk] : 0;
  for (int i = threadIdx.x; i < bs * G; i += kThreads) {
    const int pos = i / G, cg = i - pos * G;
    const int64_t dst = (((int64_t)kk * bs + pos) * H + h) * D + 8 * cg;
    if (!ok) {
      *reinterpret_cast<uint4*>(staging + dst) = make_uint4(0u, 0u, 0u, 0u);
      continue;
    }
    const int64_t src = ((bid * bs + pos) * H + h) * D + 8 * cg;
    const uint2 cb = *reinterpret_cast<const uint2*>(codes + src);
    const uint2 mb = *reinterpret_cast<const uint2*>(outm + src);
    const uint4 ov = *reinterpret_cast<const uint4*>(outv + src);
    const uint32_t cw[2] = {cb.x, cb.y}, mw[2] = {mb.x, mb.y};
    const uint32_t vw[4] = {ov.x, ov.y, ov.z, ov.w};
    const int64_t tab = PT ? (int64_t)h * sc.rows + clamp_row(p0 + pos, sc.rows) : 0;
    uint32_t res[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t pr = 0;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int e = 2 * j + k;
        const uint32_t c = (cw[e >> 2] >> (8 * (e & 3))) & 0xffu;
        const uint32_t m = (mw[e >> 2] >> (8 * (e & 3))) & 0xffu;
        uint16_t v;
        if (m) {
          v = (uint16_t)(vw[j] >> (16 * k));
        } else if (c >= (uint32_t)L) {
          v = 0;  // a code without a level decodes to +0, like the where-chain
        } else {
          const int64_t pidx = PT ? tab * L + c : (((int64_t)h * D + 8 * cg + e) * L + c);
          v = f2h(load_scale(sc.poles, sc.poles_dtype, pidx));
        }
        pr |= (uint32_t)v << (16 * k);
      }
      res[j] = pr;
    }
    store_stream(staging + dst, make_uint4(res[0], res[1], res[2], res[3]));
  }
}

bool pow2_G(int D) { return D % 8 == 0 && D >= 8 && D <= 256 && ((D / 8) & (D / 8 - 1)) == 0; }

template <int NB, bool PT, bool STATS>
void launch_write(int G, dim3 grid, hipStream_t s, const uint16_t* x, int64_t T, int H,
                  const hkv_nuq_scales& sc, const int64_t* slots, int64_t nslots, int bs,
                  uint8_t* c, uint16_t* v, uint8_t* m, float* mn, float* mx) {
  switch (G) {
#define HKV_CASE(g)                                                                            \
  case g:                                                                                      \
    hipLaunchKernelGGL((pool_write_kernel<NB, PT, g, STATS>), grid, dim3(kThreads), 0, s, x, T, \
                       H, sc, slots, nslots, bs, c, v, m, mn, mx);                             \
    break;
    HKV_CASE(1) HKV_CASE(2) HKV_CASE(4) HKV_CASE(8) HKV_CASE(16) HKV_CASE(32)
#undef HKV_CASE
  }
}

template <bool PT, bool STATS>
void launch_write_nb(int nb, int G, dim3 grid, hipStream_t s, const uint16_t* x, int64_t T, int H,
                     const hkv_nuq_scales& sc, const int64_t* slots, int64_t nslots, int bs,
                     uint8_t* c, uint16_t* v, uint8_t* m, float* mn, float* mx) {
  switch (nb) {
    case 0: launch_write<0, PT, STATS>(G, grid, s, x, T, H, sc, slots, nslots, bs, c, v, m, mn, mx); break;
    case 1: launch_write<1, PT, STATS>(G, grid, s, x, T, H, sc, slots, nslots, bs, c, v, m, mn, mx); break;
    case 2: launch_write<2, PT, STATS>(G, grid, s, x, T, H, sc, slots, nslots, bs, c, v, m, mn, mx); break;
    case 3: launch_write<3, PT, STATS>(G, grid, s, x, T, H, sc, slots, nslots, bs, c, v, m, mn, mx); break;
    default: launch_write<4, PT, STATS>(G, grid, s, x, T, H, sc, slots, nslots, bs, c, v, m, mn, mx); break;
  }
}

}  // namespace

extern "C" int hkv_pool_write(const void* values, int64_t T, int H, int D,
                              const hkv_nuq_scales* scales, const int64_t* slot_mapping,
                              int64_t num_blocks, int block_size, void* codes, void* outlier_v,
                              void* outlier_m, float* k_min, float* k_max, void* stream) {
  if (!scales || !scales->tables || !scales->poles || !scales->upper || !scales->lower)
    return HKV_ERR_ARG;
  if (scales->levels < 1 || scales->levels > 16) return HKV_ERR_ARG;
  if (scales->per_token && scales->rows < 1) return HKV_ERR_SHAPE;
  if (T < 0 || H < 1 || !pow2_G(D) || num_blocks < 0 || block_size < 1) return HKV_ERR_SHAPE;
  if ((k_min == nullptr) != (k_max == nullptr)) return HKV_ERR_ARG;
  if (scales->per_token && k_min) return HKV_ERR_ARG;  // statistics are kept for K only
  if (T == 0 || num_blocks == 0) return HKV_OK;
  if (!values || !slot_mapping || !codes || !outlier_v || !outlier_m) return HKV_ERR_ARG;
  if (((uintptr_t)values & 15u) || ((uintptr_t)outlier_v & 15u) || ((uintptr_t)codes & 7u) ||
      ((uintptr_t)outlier_m & 7u))
    return HKV_ERR_ARG;
  const int G = D / 8;
  const int64_t per_block = (int64_t)(kThreads / G) * kTokPerThread;
  dim3 grid((unsigned)((T + per_block - 1) / per_block), (unsigned)H);
  hipStream_t s = (hipStream_t)stream;
  const hkv_nuq_scales sc = *scales;
  const int nb = nb_for_levels_host(sc.levels);
  const int64_t nslots = num_blocks * block_size;
  auto x = (const uint16_t*)values;
  auto c = (uint8_t*)codes;
  auto v = (uint16_t*)outlier_v;
  auto m = (uint8_t*)outlier_m;
  if (sc.per_token)
    launch_write_nb<true, false>(nb, G, grid, s, x, T, H, sc, slot_mapping, nslots, block_size, c, v, m, nullptr, nullptr);
  else if (k_min)
    launch_write_nb<false, true>(nb, G, grid, s, x, T, H, sc, slot_mapping, nslots, block_size, c, v, m, k_min, k_max);
  else
    launch_write_nb<false, false>(nb, G, grid, s, x, T, H, sc, slot_mapping, nslots, block_size, c, v, m, nullptr, nullptr);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" int hkv_pool_gather(const void* codes, const void* outlier_v, const void* outlier_m,
                               int64_t num_blocks, int block_size, int H, int D,
                               const hkv_nuq_scales* scales, const int64_t* block_ids,
                               const int64_t* first_pos, int64_t NK, void* staging, void* stream) {
  if (!scales || !scales->poles) return HKV_ERR_ARG;
  if (scales->levels < 1 || scales->levels > 16) return HKV_ERR_ARG;
  if (scales->per_token && scales->rows < 1) return HKV_ERR_SHAPE;
  if (NK < 0 || num_blocks < 0 || block_size < 1 || H < 1 || !pow2_G(D)) return HKV_ERR_SHAPE;
  if (NK == 0) return HKV_OK;
  if (NK > 0x7fffffff || H > 65535) return HKV_ERR_SHAPE;
  if (!codes || !outlier_v || !outlier_m || !block_ids || !staging) return HKV_ERR_ARG;
  if (scales->per_token && !first_pos) return HKV_ERR_ARG;
  if (((uintptr_t)outlier_v & 15u) || ((uintptr_t)staging & 15u) || ((uintptr_t)codes & 7u) ||
      ((uintptr_t)outlier_m & 7u))
    return HKV_ERR_ARG;
  dim3 grid((unsigned)NK, (unsigned)H);
  hipStream_t s = (hipStream_t)stream;
  if (scales->per_token)
    hipLaunchKernelGGL(pool_gather_kernel<true>, grid, dim3(kThreads), 0, s, (const uint8_t*)codes,
                       (const uint16_t*)outlier_v, (const uint8_t*)outlier_m, num_blocks,
                       block_size, H, D, *scales, block_ids, first_pos, (uint16_t*)staging);
  else
    hipLaunchKernelGGL(pool_gather_kernel<false>, grid, dim3(kThreads), 0, s, (const uint8_t*)codes,
                       (const uint16_t*)outlier_v, (const uint8_t*)outlier_m, num_blocks,
                       block_size, H, D, *scales, block_ids, first_pos, (uint16_t*)staging);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
