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
// Pack is one pass over the fp16 input.  The CSR offsets need a global
// exclusive scan of per-row outlier counts; tiles of rows obtain their offset
// by a decoupled look-back: each tile publishes its count, then its inclusive
// prefix once known, and a tile sums its predecessors' published values.
// Tiles take ids from an atomic ticket, so every tile waited on is already
// running.  Status words carry a launch epoch so the workspace never needs
// clearing between calls; the last tile to finish advances the epoch.
#include "nuq_core.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPasses = 4;               // passes of kThreads*8 elements per tile
constexpr uint32_t kSpinLimit = 1u << 22;

struct PackWs {
  uint32_t ticket;
  uint32_t done;
  uint32_t epoch;
  uint32_t err;
  uint32_t pad[12];
};
static_assert(sizeof(PackWs) == 64, "workspace header");

constexpr uint32_t kFlagAgg = 1, kFlagPrefix = 2;

HKV_DEV uint64_t status_word(uint32_t epoch, uint32_t flag, uint32_t value) {
  return ((uint64_t)(((epoch & 0x3fffffffu) << 2) | flag) << 32) | value;
}

HKV_DEV void publish(uint64_t* st, uint32_t tile, uint64_t w) {
  __hip_atomic_store(st + tile, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Sum of the counts of all tiles before `tile`.
HKV_DEV uint32_t look_back(uint64_t* st, uint32_t tile, uint32_t epoch, PackWs* ws) {
  uint32_t sum = 0, spins = 0;
  int64_t j = (int64_t)tile - 1;
  const uint32_t e30 = epoch & 0x3fffffffu;
  while (j >= 0) {
    const uint64_t s = __hip_atomic_load(st + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t hi = (uint32_t)(s >> 32);
    if ((hi >> 2) == e30 && (hi & 3u) != 0) {
      sum += (uint32_t)s;
      if ((hi & 3u) == kFlagPrefix) return sum;
      --j;
      continue;
    }
    if (++spins > kSpinLimit) {  // never expected; reported to the host
      atomicOr(&ws->err, 1u);
      return sum;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  return sum;
}

template <int NB, bool PT, int G, int BITS, bool KFIX>
__global__ void __launch_bounds__(kThreads)
pack_compact_kernel(const uint16_t* __restrict__ x, int64_t nrows, int H, hkv_nuq_scales sc,
                    uint8_t* __restrict__ packed, int32_t* __restrict__ row_ptr,
                    uint8_t* __restrict__ col, uint16_t* __restrict__ val, uint32_t cap,
                    PackWs* ws, uint64_t* st, uint32_t ntiles) {
  constexpr int R = kThreads / G;
  constexpr int TR = R * kPasses;
  constexpr int D = 8 * G;
  constexpr int RB = D * BITS / 8;  // packed bytes per row
  __shared__ uint32_t s_ticket, s_epoch, s_off;
  __shared__ uint32_t s_wave[kPasses][kThreads / 64];

  const int tid = threadIdx.x, cg = tid % G, rl = tid / G;
  const int lane = tid & 63, wv = tid >> 6;
  if (tid == 0) {
    const uint32_t tk = atomicAdd(&ws->ticket, 1u);
    s_ticket = tk;
    s_epoch = __hip_atomic_load(&ws->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tk == ntiles - 1) atomicExch(&ws->ticket, 0u);  // last ticket handed out
  }
  __syncthreads();
  const uint32_t tile = s_ticket, epoch = s_epoch;
  const int64_t r0 = (int64_t)tile * TR;
  const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;
  const SlowInfo si = slow_info(sc);

  Search2<NB> S[PT ? 1 : 4];
  int64_t tab0 = 0;
  if constexpr (!PT && KFIX) {
    tab0 = (int64_t)(rl % H) * D + 8 * cg;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      load_search_pair<NB>(tabs + tab0 + 2 * j, tabs + tab0 + 2 * j + 1, S[j]);
  }

  uint32_t xs[kPasses][4];
  uint32_t mk[kPasses];
  uint32_t excl[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int64_t r = r0 + p * R + rl;
    mk[p] = 0;
    xs[p][0] = xs[p][1] = xs[p][2] = xs[p][3] = 0;
    if (r < nrows) {
      const int64_t t = r / H;
      const int h = (int)(r - t * H);
      if constexpr (PT) {
        tab0 = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
        load_search_bcast<NB>(tabs + tab0, S[0]);
      } else if constexpr (!KFIX) {
        tab0 = (int64_t)h * D + 8 * cg;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          load_search_pair<NB>(tabs + tab0 + 2 * j, tabs + tab0 + 2 * j + 1, S[j]);
      }
      const uint4 xv = *reinterpret_cast<const uint4*>(x + r * D + 8 * cg);
      uint32_t c[4], om[4];
      quant8<NB, PT>(xv, S, si, tab0, c, om);
      if constexpr (BITS == 4) {
        *reinterpret_cast<uint32_t*>(packed + r * RB + 4 * cg) = pack_nibbles(c);
      } else {
        *reinterpret_cast<uint16_t*>(packed + r * RB + 2 * cg) = (uint16_t)pack_crumbs(c);
      }
      mk[p] = mask_bits(om);
      xs[p][0] = xv.x; xs[p][1] = xv.y; xs[p][2] = xv.z; xs[p][3] = xv.w;
    }
    // wave-inclusive scan of this pass's counts
    const uint32_t cnt = __builtin_popcount(mk[p]);
    uint32_t inc = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t y = __shfl_up(inc, o, 64);
      if (lane >= o) inc += y;
    }
    excl[p] = inc - cnt;
    if (lane == 63) s_wave[p][wv] = inc;
  }
  __syncthreads();

  // Tile-local offsets in (pass, wave) order, and the tile total.
  uint32_t base[kPasses];
  uint32_t total = 0;
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
      if (w == wv) base[p] = total;
      total += s_wave[p][w];
    }
  }

  if (tid == 0) {
    uint32_t off = 0;
    if (tile == 0) {
      publish(st, tile, status_word(epoch, kFlagPrefix, total));
    } else {
      publish(st, tile, status_word(epoch, kFlagAgg, total));
      off = look_back(st, tile, epoch, ws);
      publish(st, tile, status_word(epoch, kFlagPrefix, off + total));
    }
    s_off = off;
  }
  __syncthreads();
  const uint32_t off = s_off;

#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int64_t r = r0 + p * R + rl;
    if (r >= nrows) continue;
    uint32_t pos = off + base[p] + excl[p];
    if (cg == 0) row_ptr[r] = (int32_t)pos;
    const uint32_t m = mk[p];
    if (m) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if ((m >> e) & 1u) {
          if (pos < cap) {
            col[pos] = (uint8_t)(8 * cg + e);
            val[pos] = (uint16_t)(xs[p][e >> 1] >> (16 * (e & 1)));
          }
          ++pos;
        }
      }
    }
  }
  if (tile == ntiles - 1 && tid == 0) row_ptr[nrows] = (int32_t)(off + total);

  if (tid == 0) {
    __threadfence();
    const uint32_t prev = atomicAdd(&ws->done, 1u);
    if (prev == ntiles - 1) {
      atomicExch(&ws->done, 0u);
      __hip_atomic_store(&ws->epoch, epoch + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Compact unpack.  Blocks loop over tiles of rows; each tile is dequantised
// into LDS, the tile's CSR entries are scattered into it, and it is written
// out with 128-bit stores.  Per-channel fp16 poles for all heads sit in LDS
// for the block's lifetime when they fit (KLDS), else are read through L1.
template <bool PT, int G, int BITS, bool KLDS>
__global__ void __launch_bounds__(kThreads)
unpack_compact_kernel(const uint8_t* __restrict__ packed, const int32_t* __restrict__ row_ptr,
                      const uint8_t* __restrict__ col, const uint16_t* __restrict__ val,
                      int64_t nrows, int H, hkv_nuq_scales sc, uint16_t* __restrict__ out,
                      uint32_t ntiles) {
  constexpr int R = kThreads / G;
  constexpr int TR = R * kPasses;
  constexpr int D = 8 * G;
  constexpr int RB = D * BITS / 8;
  extern __shared__ uint16_t dyn[];
  uint16_t* tile_lds = dyn;                 // TR * D
  uint16_t* pole_lds = dyn + TR * D;        // PT: TR*16; K: H*16*D when KLDS
  const int tid = threadIdx.x, cg = tid % G, rl = tid / G;
  const hkv_table_t* tabs = (const hkv_table_t*)sc.tables;

  if constexpr (!PT && KLDS) {
    for (int i = tid; i < H * 16 * D; i += kThreads) {
      const int d = i % D, l = (i / D) % 16, h = i / (16 * D);
      pole_lds[i] = tabs[(int64_t)h * D + d].pf16[l];
    }
  }

  for (uint32_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t r0 = (int64_t)tile * TR;
    __syncthreads();  // previous tile fully written out; K poles staged
    if constexpr (PT) {
      for (int i = tid; i < TR * 16; i += kThreads) {
        const int rr = i / 16, l = i % 16;
        const int64_t r = r0 + rr;
        if (r < nrows) {
          const int64_t t = r / H;
          const int h = (int)(r - t * H);
          const int64_t tab = (int64_t)h * sc.rows + clamp_row(token_pos(sc, t), sc.rows);
          pole_lds[i] = tabs[tab].pf16[l];
        }
      }
      __syncthreads();
    }
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int rr = p * R + rl;
      const int64_t r = r0 + rr;
      if (r >= nrows) continue;
      const int h = (int)(r % H);
      uint32_t cw;
      if constexpr (BITS == 4) cw = *reinterpret_cast<const uint32_t*>(packed + r * RB + 4 * cg);
      else cw = *reinterpret_cast<const uint16_t*>(packed + r * RB + 2 * cg);
      uint32_t res[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t pr = 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const int e = 2 * j + k;
          const uint32_t c = (cw >> (BITS * e)) & ((1u << BITS) - 1u);
          uint16_t v;
          if constexpr (PT) v = pole_lds[rr * 16 + c];
          else if constexpr (KLDS) v = pole_lds[(h * 16 + c) * D + 8 * cg + e];
          else v = tabs[(int64_t)h * D + 8 * cg + e].pf16[c];
          pr |= (uint32_t)v << (16 * k);
        }
        res[j] = pr;
      }
      *reinterpret_cast<uint4*>(tile_lds + rr * D + 8 * cg) = make_uint4(res[0], res[1], res[2], res[3]);
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int rr = p * R + rl;
      const int64_t r = r0 + rr;
      if (r >= nrows) continue;
      const int32_t a = row_ptr[r], b = row_ptr[r + 1];
      for (int32_t i = a + cg; i < b; i += G) {
        const uint32_t d = col[i];
        if (d < (uint32_t)D) tile_lds[rr * D + d] = val[i];
      }
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int rr = p * R + rl;
      const int64_t r = r0 + rr;
      if (r >= nrows) continue;
      *reinterpret_cast<uint4*>(out + r * D + 8 * cg) =
          *reinterpret_cast<const uint4*>(tile_lds + rr * D + 8 * cg);
    }
  }
}

__global__ void write_zero_rowptr(int32_t* row_ptr) { row_ptr[0] = 0; }

bool pow2_G(int D) { return D % 8 == 0 && D >= 8 && D <= 256 && ((D / 8) & (D / 8 - 1)) == 0; }

int64_t tiles_for(int64_t nrows, int D) {
  const int64_t TR = (int64_t)(kThreads / (D / 8)) * kPasses;
  return (nrows + TR - 1) / TR;
}

template <int NB, bool PT, int BITS, bool KFIX>
void launch_pack_g(int G, unsigned ntiles, hipStream_t s, const uint16_t* x, int64_t nrows, int H,
                   const hkv_nuq_scales& sc, uint8_t* pk, int32_t* rp, uint8_t* col,
                   uint16_t* val, uint32_t cap, PackWs* ws, uint64_t* st) {
  switch (G) {
#define HKV_CASE(g)                                                                         \
  case g:                                                                                   \
    hipLaunchKernelGGL((pack_compact_kernel<NB, PT, g, BITS, KFIX>), dim3(ntiles),          \
                       dim3(kThreads), 0, s, x, nrows, H, sc, pk, rp, col, val, cap, ws, st, \
                       ntiles);                                                             \
    break;
    HKV_CASE(1) HKV_CASE(2) HKV_CASE(4) HKV_CASE(8) HKV_CASE(16) HKV_CASE(32)
#undef HKV_CASE
  }
}

template <int NB, bool PT, int BITS>
void launch_pack_k(bool kfix, int G, unsigned ntiles, hipStream_t s, const uint16_t* x,
                   int64_t nrows, int H, const hkv_nuq_scales& sc, uint8_t* pk, int32_t* rp,
                   uint8_t* col, uint16_t* val, uint32_t cap, PackWs* ws, uint64_t* st) {
  if (kfix) launch_pack_g<NB, PT, BITS, true>(G, ntiles, s, x, nrows, H, sc, pk, rp, col, val, cap, ws, st);
  else launch_pack_g<NB, PT, BITS, false>(G, ntiles, s, x, nrows, H, sc, pk, rp, col, val, cap, ws, st);
}

template <bool PT, int BITS, bool KLDS>
void launch_unpack_g(int G, unsigned grid, size_t lds, hipStream_t s, const uint8_t* pk,
                     const int32_t* rp, const uint8_t* col, const uint16_t* val, int64_t nrows,
                     int H, const hkv_nuq_scales& sc, uint16_t* out, uint32_t ntiles) {
  switch (G) {
#define HKV_CASE(g)                                                                            \
  case g:                                                                                      \
    hipLaunchKernelGGL((unpack_compact_kernel<PT, g, BITS, KLDS>), dim3(grid), dim3(kThreads), \
                       lds, s, pk, rp, col, val, nrows, H, sc, out, ntiles);                   \
    break;
    HKV_CASE(1) HKV_CASE(2) HKV_CASE(4) HKV_CASE(8) HKV_CASE(16) HKV_CASE(32)
#undef HKV_CASE
  }
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

}  // namespace

extern "C" size_t hkv_nuq_pack_compact_workspace_bytes(int64_t T, int H, int D) {
  if (T < 0 || H < 1 || !pow2_G(D)) return 0;
  return sizeof(PackWs) + sizeof(uint64_t) * (size_t)tiles_for(T * H, D);
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
  const size_t need = hkv_nuq_pack_compact_workspace_bytes(T, H, D);
  if (!workspace || workspace_bytes < need) return HKV_ERR_WORKSPACE;
  const int G = D / 8, R = kThreads / G;
  const unsigned ntiles = (unsigned)tiles_for(nrows, D);
  const bool kfix = (R % H) == 0;
  const uint32_t cap = (uint32_t)std::min<int64_t>(capacity, 0x7fffffff);
  PackWs* ws = (PackWs*)workspace;
  uint64_t* st = (uint64_t*)((char*)workspace + sizeof(PackWs));
  const hkv_nuq_scales sc = *scales;
  const int nb = nb_for_levels_host(sc.levels);
  auto x = (const uint16_t*)values;
  auto pk = (uint8_t*)packed;
#define HKV_ARGS kfix, G, ntiles, s, x, nrows, H, sc, pk, row_ptr, col, val, cap, ws, st
  if (bits == 4) {
    if (sc.per_token) {
      switch (nb) {
        case 0: launch_pack_k<0, true, 4>(HKV_ARGS); break;
        case 1: launch_pack_k<1, true, 4>(HKV_ARGS); break;
        case 2: launch_pack_k<2, true, 4>(HKV_ARGS); break;
        case 3: launch_pack_k<3, true, 4>(HKV_ARGS); break;
        default: launch_pack_k<4, true, 4>(HKV_ARGS); break;
      }
    } else {
      switch (nb) {
        case 0: launch_pack_k<0, false, 4>(HKV_ARGS); break;
        case 1: launch_pack_k<1, false, 4>(HKV_ARGS); break;
        case 2: launch_pack_k<2, false, 4>(HKV_ARGS); break;
        case 3: launch_pack_k<3, false, 4>(HKV_ARGS); break;
        default: launch_pack_k<4, false, 4>(HKV_ARGS); break;
      }
    }
  } else {
    if (sc.per_token) {
      switch (nb) {
        case 0: launch_pack_k<0, true, 2>(HKV_ARGS); break;
        case 1: launch_pack_k<1, true, 2>(HKV_ARGS); break;
        default: launch_pack_k<2, true, 2>(HKV_ARGS); break;
      }
    } else {
      switch (nb) {
        case 0: launch_pack_k<0, false, 2>(HKV_ARGS); break;
        case 1: launch_pack_k<1, false, 2>(HKV_ARGS); break;
        default: launch_pack_k<2, false, 2>(HKV_ARGS); break;
      }
    }
  }
#undef HKV_ARGS
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" int hkv_nuq_pack_compact_status(const void* workspace, void* stream) {
  if (!workspace) return HKV_ERR_ARG;
  uint32_t err = 0;
  if (hipMemcpyAsync(&err, (const char*)workspace + offsetof(PackWs, err), sizeof(err),
                     hipMemcpyDeviceToHost, (hipStream_t)stream) != hipSuccess)
    return -1;
  if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) return -1;
  return (int)err;
}

extern "C" int hkv_nuq_unpack_compact(const void* packed, const int32_t* row_ptr,
                                      const uint8_t* col, const uint16_t* val, int64_t T, int H,
                                      int D, int bits, const hkv_nuq_scales* scales, void* out,
                                      void* stream) {
  if (!scales || !scales->tables) return HKV_ERR_ARG;
  if (bits != 2 && bits != 4) return HKV_ERR_ARG;
  if (scales->per_token && scales->rows < 1) return HKV_ERR_SHAPE;
  if (T < 0 || H < 1 || !pow2_G(D)) return HKV_ERR_SHAPE;
  if (T == 0) return HKV_OK;
  if (!packed || !row_ptr || !out) return HKV_ERR_ARG;
  if (((uintptr_t)out & 15u) || ((uintptr_t)packed & 3u)) return HKV_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nrows = T * H;
  const int G = D / 8;
  const int TR = (kThreads / G) * kPasses;
  const unsigned ntiles = (unsigned)tiles_for(nrows, D);
  const unsigned grid = (unsigned)std::min<int64_t>(ntiles, (int64_t)num_cus() * 8);
  const hkv_nuq_scales sc = *scales;
  const size_t tile_bytes = (size_t)TR * D * 2;
  const size_t kpole_bytes = (size_t)H * 16 * D * 2;
  auto pk = (const uint8_t*)packed;
  auto o = (uint16_t*)out;
  if (sc.per_token) {
    const size_t lds = tile_bytes + (size_t)TR * 16 * 2;
    if (bits == 4) launch_unpack_g<true, 4, false>(G, grid, lds, s, pk, row_ptr, col, val, nrows, H, sc, o, ntiles);
    else launch_unpack_g<true, 2, false>(G, grid, lds, s, pk, row_ptr, col, val, nrows, H, sc, o, ntiles);
  } else if (tile_bytes + kpole_bytes <= 64 * 1024) {
    const size_t lds = tile_bytes + kpole_bytes;
    if (bits == 4) launch_unpack_g<false, 4, true>(G, grid, lds, s, pk, row_ptr, col, val, nrows, H, sc, o, ntiles);
    else launch_unpack_g<false, 2, true>(G, grid, lds, s, pk, row_ptr, col, val, nrows, H, sc, o, ntiles);
  } else {
    const size_t lds = tile_bytes;
    if (bits == 4) launch_unpack_g<false, 4, false>(G, grid, lds, s, pk, row_ptr, col, val, nrows, H, sc, o, ntiles);
    else launch_unpack_g<false, 2, false>(G, grid, lds, s, pk, row_ptr, col, val, nrows, H, sc, o, ntiles);
  }
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
