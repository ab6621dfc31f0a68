// nuq_dense.hip -- nuq pack/unpack in the reference's byte-per-code format:
// codes u8, dense fp16 outlier values (0 elsewhere), outlier mask u8, all
// (T,H,D).  Drop-in for src/kvquant/triton_batched.py (K5-K8) and, with H = 1,
// src/kvquant/triton_kernels.py (K1-K4).
//
// Layout of work: block (t-tile, head h), 256 threads, G = D/8 threads per row
// each owning 8 consecutive channels (one 128-bit load).  Per-channel (K)
// tables are loaded once per thread; per-token (V) tables once per row.
#include "nuq_core.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTokTile = 64;  // tokens per block (per head)

template <int NB, bool PT, int G>
__global__ void __launch_bounds__(kThreads)
pack_dense_kernel(const uint16_t* __restrict__ x, int64_t T, int H, hkv_nuq_scales sc,
                  uint8_t* __restrict__ codes, uint16_t* __restrict__ outv,
                  uint8_t* __restrict__ outm) {
  constexpr int R = kThreads / G;
  constexpr int D = 8 * G;
  const int tid = threadIdx.x, cg = tid % G, rl = tid / G;
  const int h = blockIdx.y;
  const int64_t t0 = (int64_t)blockIdx.x * kTokTile;
  const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;
  const SlowInfo si = slow_info(sc);
  Search2<NB> S[PT ? 1 : 4];
  int64_t tab0 = (int64_t)h * D + 8 * cg;
  if constexpr (!PT) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      load_search_pair<NB>(tabs + tab0 + 2 * j, tabs + tab0 + 2 * j + 1, S[j]);
  }
  for (int tt = rl; tt < kTokTile; tt += R) {
    const int64_t t = t0 + tt;
    if (t >= T) break;
    if constexpr (PT) {
      tab0 = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
      load_search_bcast<NB>(tabs + tab0, S[0]);
    }
    const int64_t off = (t * H + h) * D + 8 * cg;
    const uint4 xv = *reinterpret_cast<const uint4*>(x + off);
    uint32_t c[4], om[4];
    if constexpr (PT) quant8<NB, PT>(xv, S, si, RowTab{tab0}, c, om);
    else quant8<NB, PT>(xv, S, si, ChanTab{tab0}, c, om);
    uint2 cb, mb;
    cb.x = lanes_to_bytes(c[0]) | (lanes_to_bytes(c[1]) << 16);
    cb.y = lanes_to_bytes(c[2]) | (lanes_to_bytes(c[3]) << 16);
    mb.x = lanes_to_bytes(om[0] & 0x00010001u) | (lanes_to_bytes(om[1] & 0x00010001u) << 16);
    mb.y = lanes_to_bytes(om[2] & 0x00010001u) | (lanes_to_bytes(om[3] & 0x00010001u) << 16);
    uint4 ov = make_uint4(xv.x & om[0], xv.y & om[1], xv.z & om[2], xv.w & om[3]);
    *reinterpret_cast<uint2*>(codes + off) = cb;
    *reinterpret_cast<uint4*>(outv + off) = ov;
    *reinterpret_cast<uint2*>(outm + off) = mb;
  }
}

// Any D / alignment: one thread per element, exact scan (no tables needed).
__global__ void __launch_bounds__(kThreads)
pack_dense_generic(const uint16_t* __restrict__ x, int64_t T, int H, int D, hkv_nuq_scales sc,
                   uint8_t* __restrict__ codes, uint16_t* __restrict__ outv,
                   uint8_t* __restrict__ outm) {
  const int64_t n = T * H * D;
  const SlowInfo si = slow_info(sc);
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t t = i / ((int64_t)H * D);
    const int h = (int)((i / D) % H), d = (int)(i % D);
    const int64_t tab = sc.per_token ? (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows)
                                     : (int64_t)h * D + d;
    int o;
    const int c = slow_one(x[i], si, tab, &o);
    codes[i] = (uint8_t)c;
    outv[i] = o ? x[i] : (uint16_t)0;
    outm[i] = (uint8_t)o;
  }
}

// Dense unpack.  Poles of the block's head (per-channel) or of each row
// (per-token) are staged in LDS as fp16, [level][channel] / [row][level].
template <bool PT, int G>
__global__ void __launch_bounds__(kThreads)
unpack_dense_kernel(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ outv,
                    const uint8_t* __restrict__ outm, int64_t T, int H, hkv_nuq_scales sc,
                    uint16_t* __restrict__ out) {
  constexpr int R = kThreads / G;
  constexpr int D = 8 * G;
  __shared__ uint16_t lds[16 * 256];
  const int tid = threadIdx.x, cg = tid % G, rl = tid / G;
  const int h = blockIdx.y;
  const int L = sc.levels;
  const int64_t t0 = (int64_t)blockIdx.x * kTokTile;
  if constexpr (!PT) {
    for (int i = tid; i < L * D; i += kThreads) {
      const int l = i / D, d = i % D;
      lds[i] = f2h(load_scale(sc.poles, sc.poles_dtype, ((int64_t)h * D + d) * L + l));
    }
    __syncthreads();
  }
  for (int base = 0; base < kTokTile; base += R) {
    const int64_t t = t0 + base + rl;
    const bool live = t < T;
    if constexpr (PT) {
      __syncthreads();
      if (live && cg < L) {
        for (int l = cg; l < L; l += G) {
          const int64_t tab = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
          lds[rl * 16 + l] = f2h(load_scale(sc.poles, sc.poles_dtype, tab * L + l));
        }
      }
      __syncthreads();
    }
    if (!live) continue;
    const int64_t off = (t * H + h) * D + 8 * cg;
    const uint2 cb = *reinterpret_cast<const uint2*>(codes + off);
    const uint2 mb = *reinterpret_cast<const uint2*>(outm + off);
    const uint4 ov = *reinterpret_cast<const uint4*>(outv + off);
    const uint32_t cw[2] = {cb.x, cb.y}, mw[2] = {mb.x, mb.y};
    const uint32_t vw[4] = {ov.x, ov.y, ov.z, ov.w};
    uint32_t res[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t half2 = 0;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int e = 2 * j + k;
        const uint32_t c = (cw[e >> 2] >> (8 * (e & 3))) & 0xffu;
        const uint32_t m = (mw[e >> 2] >> (8 * (e & 3))) & 0xffu;
        // a code without a level decodes to +0, as the reference's where-chain
        // over levels leaves it (src/kvquant/triton_batched.py:113-117)
        const uint16_t pole = c >= (uint32_t)L ? (uint16_t)0
                              : (PT ? lds[rl * 16 + c] : lds[c * D + 8 * cg + e]);
        const uint16_t v = m ? (uint16_t)(vw[j] >> (16 * k)) : pole;
        half2 |= (uint32_t)v << (16 * k);
      }
      res[j] = half2;
    }
    store_stream(out + off, make_uint4(res[0], res[1], res[2], res[3]));
  }
}

__global__ void __launch_bounds__(kThreads)
unpack_dense_generic(const uint8_t* __restrict__ codes, const uint16_t* __restrict__ outv,
                     const uint8_t* __restrict__ outm, int64_t T, int H, int D,
                     hkv_nuq_scales sc, uint16_t* __restrict__ out) {
  const int64_t n = T * H * D;
  const int L = sc.levels;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t t = i / ((int64_t)H * D);
    const int h = (int)((i / D) % H), d = (int)(i % D);
    const int64_t tab = sc.per_token ? (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows)
                                     : (int64_t)h * D + d;
    const int c = codes[i];
    out[i] = outm[i] ? outv[i]
                     : (c >= L ? (uint16_t)0 : f2h(load_scale(sc.poles, sc.poles_dtype, tab * L + c)));
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int NB, bool PT>
void launch_pack(int G, dim3 grid, hipStream_t st, const uint16_t* x, int64_t T, int H,
                 const hkv_nuq_scales& sc, uint8_t* c, uint16_t* v, uint8_t* m) {
  switch (G) {
#define HKV_CASE(g)                                                                          \
  case g:                                                                                    \
    hipLaunchKernelGGL((pack_dense_kernel<NB, PT, g>), grid, dim3(kThreads), 0, st, x, T, H, \
                       sc, c, v, m);                                                         \
    break;
    HKV_CASE(1) HKV_CASE(2) HKV_CASE(4) HKV_CASE(8) HKV_CASE(16) HKV_CASE(32)
#undef HKV_CASE
  }
}

template <bool PT>
void launch_unpack(int G, dim3 grid, hipStream_t st, const uint8_t* c, const uint16_t* v,
                   const uint8_t* m, int64_t T, int H, const hkv_nuq_scales& sc, uint16_t* o) {
  switch (G) {
#define HKV_CASE(g)                                                                            \
  case g:                                                                                      \
    hipLaunchKernelGGL((unpack_dense_kernel<PT, g>), grid, dim3(kThreads), 0, st, c, v, m, T, \
                       H, sc, o);                                                              \
    break;
    HKV_CASE(1) HKV_CASE(2) HKV_CASE(4) HKV_CASE(8) HKV_CASE(16) HKV_CASE(32)
#undef HKV_CASE
  }
}

bool pow2_G(int D) { return D % 8 == 0 && D >= 8 && D <= 256 && ((D / 8) & (D / 8 - 1)) == 0; }

int check_scales(const hkv_nuq_scales* sc, int64_t T, int H, int D, bool need_tables) {
  if (!sc || !sc->poles || !sc->upper || !sc->lower) return HKV_ERR_ARG;
  if (sc->levels < 1 || sc->levels > 16) return HKV_ERR_ARG;
  if (sc->poles_dtype < 0 || sc->poles_dtype > 2 || sc->thr_dtype < 0 || sc->thr_dtype > 2)
    return HKV_ERR_DTYPE;
  if (sc->per_token && sc->rows < 1) return HKV_ERR_SHAPE;
  if (need_tables && !sc->tables) return HKV_ERR_ARG;
  if (T < 0 || H < 1 || D < 1) return HKV_ERR_SHAPE;
  return HKV_OK;
}

}  // namespace

extern "C" int hkv_nuq_pack_dense(const void* values, int64_t T, int H, int D,
                                  const hkv_nuq_scales* scales, void* codes, void* outlier_v,
                                  void* outlier_m, void* stream) {
  int st = check_scales(scales, T, H, D, false);
  if (st) return st;
  if (T == 0) return HKV_OK;
  if (!values || !codes || !outlier_v || !outlier_m) return HKV_ERR_ARG;
  const hkv_nuq_scales sc = *scales;
  hipStream_t s = (hipStream_t)stream;
  const bool fast = sc.tables && pow2_G(D) && aligned16(values) && aligned16(outlier_v) &&
                    ((uintptr_t)codes & 7u) == 0 && ((uintptr_t)outlier_m & 7u) == 0;
  if (fast) {
    const int G = D / 8;
    dim3 grid((unsigned)((T + kTokTile - 1) / kTokTile), (unsigned)H);
    const int nb = nb_for_levels_host(sc.levels);
    auto x = (const uint16_t*)values;
    auto c = (uint8_t*)codes;
    auto v = (uint16_t*)outlier_v;
    auto m = (uint8_t*)outlier_m;
    if (sc.per_token) {
      switch (nb) {
        case 0: launch_pack<0, true>(G, grid, s, x, T, H, sc, c, v, m); break;
        case 1: launch_pack<1, true>(G, grid, s, x, T, H, sc, c, v, m); break;
        case 2: launch_pack<2, true>(G, grid, s, x, T, H, sc, c, v, m); break;
        case 3: launch_pack<3, true>(G, grid, s, x, T, H, sc, c, v, m); break;
        default: launch_pack<4, true>(G, grid, s, x, T, H, sc, c, v, m); break;
      }
    } else {
      switch (nb) {
        case 0: launch_pack<0, false>(G, grid, s, x, T, H, sc, c, v, m); break;
        case 1: launch_pack<1, false>(G, grid, s, x, T, H, sc, c, v, m); break;
        case 2: launch_pack<2, false>(G, grid, s, x, T, H, sc, c, v, m); break;
        case 3: launch_pack<3, false>(G, grid, s, x, T, H, sc, c, v, m); break;
        default: launch_pack<4, false>(G, grid, s, x, T, H, sc, c, v, m); break;
      }
    }
  } else {
    const int64_t n = T * H * D;
    const int64_t blocks = std::min<int64_t>((n + kThreads - 1) / kThreads, 1 << 16);
    hipLaunchKernelGGL(pack_dense_generic, dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       (const uint16_t*)values, T, H, D, sc, (uint8_t*)codes,
                       (uint16_t*)outlier_v, (uint8_t*)outlier_m);
  }
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" int hkv_nuq_unpack_dense(const void* codes, const void* outlier_v,
                                    const void* outlier_m, int64_t T, int H, int D,
                                    const hkv_nuq_scales* scales, void* out, void* stream) {
  int st = check_scales(scales, T, H, D, false);
  if (st) return st;
  if (T == 0) return HKV_OK;
  if (!codes || !outlier_v || !outlier_m || !out) return HKV_ERR_ARG;
  const hkv_nuq_scales sc = *scales;
  hipStream_t s = (hipStream_t)stream;
  const bool fast = pow2_G(D) && aligned16(outlier_v) && aligned16(out) &&
                    ((uintptr_t)codes & 7u) == 0 && ((uintptr_t)outlier_m & 7u) == 0;
  if (fast) {
    dim3 grid((unsigned)((T + kTokTile - 1) / kTokTile), (unsigned)H);
    if (sc.per_token)
      launch_unpack<true>(D / 8, grid, s, (const uint8_t*)codes, (const uint16_t*)outlier_v,
                          (const uint8_t*)outlier_m, T, H, sc, (uint16_t*)out);
    else
      launch_unpack<false>(D / 8, grid, s, (const uint8_t*)codes, (const uint16_t*)outlier_v,
                           (const uint8_t*)outlier_m, T, H, sc, (uint16_t*)out);
  } else {
    const int64_t n = T * H * D;
    const int64_t blocks = std::min<int64_t>((n + kThreads - 1) / kThreads, 1 << 16);
    hipLaunchKernelGGL(unpack_dense_generic, dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       (const uint8_t*)codes, (const uint16_t*)outlier_v,
                       (const uint8_t*)outlier_m, T, H, D, sc, (uint16_t*)out);
  }
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
