// decode.hip -- fused dequant + Quest-sparse decode attention (batch 1).
//
// Replaces the reference's decode path unpack_to_staging + flash_attn_varlen_
// func over an fp16 staging copy (src/kvquant/compact_backend.py:233-299):
// the selected pages are read straight from the compact format (bit-packed
// nuq2/nuq4 codes + CSR outliers, as written by hkv_nuq_pack_compact over
// rows t*H + h), dequantised in LDS and fed to MFMA.  Semantics: for query
// head hq (KV head g = hq / group), softmax(q . K^T * scale) . V over the
// tokens of the pages sel[0..nsel)[g] (page p = tokens [16p, 16p+16), tokens
// >= T masked), with an fp32 softmax -- the dense restatement
// src/quest/reference.py:136-168 with the standard GQA head map.
//
// Work: grid (splits, H); a split is a run of pps consecutive selected pages
// of one KV head; each of the block's 4 waves takes every 4th page.  Per page
// a wave:
//   1. loads the 16 rows' packed K and V codes (16 B per lane),
//   2. dequantises them through LUTs in LDS (K: per-channel poles of head g,
//      staged once per block; V: the rows' per-token poles, row
//      min(t, rows-1)), into padded fp16 tiles [16 keys][136],
//   3. patches the rows' CSR outliers into the tiles,
//   4. S^T = K Q^T with 8 v_mfma_f32_16x16x16f16 (lane l: query head l%16 of
//      the group, keys 4*(l/16)..+3), online softmax per query head (lanes
//      l, l^16, l^32, l^48 share a head),
//   5. O^T += V^T P^T with 8 more MFMAs; P comes straight from S's registers.
// The 4 waves' (m, l, O) are merged through LDS into one partial per split;
// merge_kernel combines the splits (flash-decoding) and normalises.
#include "hkv_common.h"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));

constexpr int kDT = 256;       // threads per block
constexpr int kW = kDT / 64;   // waves per block
constexpr int kHD = 128;       // head dim
constexpr int kPS = 16;        // tokens per page
constexpr int kTS = kHD + 8;   // padded tile row (halves): conflict-free MFMA operand reads

struct Side {  // one of K / V in the compact format
  const uint8_t* packed;   // (T, H, D*bits/8)
  const int32_t* row_ptr;  // (T*H + 1)
  const uint8_t* col;      // (cap)
  const uint16_t* val;     // (cap)
  int64_t cap;
  const hkv_table_t* tabs; // decision tables: pf16 are the dequantised poles
  int64_t rows;            // per-token scale rows (V); unused for K
  int bits;
};

struct DecodeArgs {
  const uint16_t* q;  // (Hq, D) fp16
  Side k, v;
  int H, group;
  int64_t T;
  const int64_t* sel;  // (nsel, H)
  int64_t nsel;
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

// Dequantise one side of a page into tile[16][kTS]: lane l owns row l/4 and
// channels [32*(l%4), +32).  lut(row, ch, code) gives the fp16 bits.
template <typename Lut>
HKV_DEV void dequant_page(const Side& sd, int64_t t0, int64_t T, int H, int g, int lane,
                          uint16_t* tile, Lut lut) {
  const int row = lane >> 2, c0 = 32 * (lane & 3);
  const int64_t t = t0 + row;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  if (t < T) {
    const int64_t r = t * H + g;
    if (sd.bits == 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(sd.packed + r * (kHD / 2) + c0 / 2);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(sd.packed + r * (kHD / 4) + c0 / 4);
      w[0] = v.x; w[1] = v.y;
    }
  }
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
        if (sd.bits == 4) code = (w[e >> 3] >> (4 * (e & 7))) & 15u;
        else code = (w[e >> 4] >> (2 * (e & 15))) & 3u;
        pr |= (uint32_t)lut(row, c0 + e, code) << (16 * e2);
      }
      h[j] = t < T ? pr : 0u;  // rows past the context read as zeros
    }
    *reinterpret_cast<uint4*>(tile + row * kTS + c0 + 8 * k) = make_uint4(h[0], h[1], h[2], h[3]);
  }
}

// The page's CSR outliers over the tile (after dequant_page, before use):
// lane l handles row l/4, entries (l%4), +4, ...
HKV_DEV void patch_page(const Side& sd, int64_t t0, int64_t T, int H, int g, int lane,
                        uint16_t* tile) {
  const int row = lane >> 2;
  const int64_t t = t0 + row;
  if (t >= T) return;
  const int64_t r = t * H + g;
  int32_t a = sd.row_ptr[r], b = sd.row_ptr[r + 1];
  if (a < 0) a = 0;
  if ((int64_t)b > sd.cap) b = (int32_t)sd.cap;
  for (int32_t i = a + (lane & 3); i < b; i += 4) {
    const uint32_t d = sd.col[i];
    if (d < (uint32_t)kHD) tile[row * kTS + d] = sd.val[i];
  }
}

__global__ void __launch_bounds__(kDT)
decode_kernel(DecodeArgs A) {
  __shared__ uint16_t s_klut[16 * kHD];           // [level][channel] of head g
  __shared__ __align__(16) uint16_t s_vlut[kW][kPS * 16];  // [row][level] of the wave's page
  __shared__ __align__(16) uint16_t s_tiles[kW][2][kPS * kTS];
  __shared__ float s_m[kW][16], s_l[kW][16];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int g = blockIdx.y, H = A.H, group = A.group;
  const int64_t j0 = (int64_t)blockIdx.x * A.pps;
  const int64_t j1 = j0 + A.pps < A.nsel ? j0 + A.pps : A.nsel;

  for (int i = tid; i < 16 * kHD; i += kDT) {
    const int l = i / kHD, d = i % kHD;
    s_klut[i] = A.k.tabs[(int64_t)g * kHD + d].pf16[l];
  }
  __syncthreads();

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
  const float sl2 = A.scale * 1.4426950408889634f;  // scale * log2(e)

  uint16_t* kt = s_tiles[wv][0];
  uint16_t* vt = s_tiles[wv][1];
  uint16_t* vl = s_vlut[wv];
  for (int64_t j = j0 + wv; j < j1; j += kW) {
    const int64_t p = A.sel[j * H + g];
    if (p < 0 || p >= (A.T + kPS - 1) / kPS) continue;  // no such page: nothing to attend
    const int64_t t0 = p * kPS;
    // V row tables: lanes 0..15 stage row `lane`'s 16 poles
    if (lane < kPS) {
      const int64_t t = t0 + lane;
      const int64_t row = t < A.v.rows ? t : A.v.rows - 1;
      const uint4* src = reinterpret_cast<const uint4*>(A.v.tabs[(int64_t)g * A.v.rows + row].pf16);
      reinterpret_cast<uint4*>(vl + lane * 16)[0] = src[0];
      reinterpret_cast<uint4*>(vl + lane * 16)[1] = src[1];
    }
    wave_sync();
    dequant_page(A.k, t0, A.T, H, g, lane, kt,
                 [&](int, int ch, uint32_t c) { return s_klut[c * kHD + ch]; });
    dequant_page(A.v, t0, A.T, H, g, lane, vt,
                 [&](int row, int, uint32_t c) { return vl[row * 16 + c]; });
    wave_sync();
    patch_page(A.k, t0, A.T, H, g, lane, kt);
    patch_page(A.v, t0, A.T, H, g, lane, vt);
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
    const float mn = fmaxf(m, mp);  // finite: every selected page holds a token < T
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
    wave_sync();  // the tiles are rewritten by the wave's next page
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
  const int64_t split = blockIdx.x;
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

// out[hq] = sum_s exp2(m_s - M) o_s / sum_s exp2(m_s - M) l_s  (m in log2 units)
__global__ void __launch_bounds__(kHD)
merge_kernel(const float* __restrict__ pm, const float* __restrict__ pl,
             const float* __restrict__ po, int64_t splits, int Hq, int H, int group,
             int64_t pps, int64_t nsel, void* out, int odt) {
  const int hq = blockIdx.x, d = threadIdx.x;
  (void)H;
  (void)group;
  (void)pps;
  (void)nsel;
  float M = -__builtin_inff();
  for (int64_t s = 0; s < splits; ++s) M = fmaxf(M, pm[s * Hq + hq]);
  float acc = 0.0f, L = 0.0f;
  if (M != -__builtin_inff()) {
    for (int64_t s = 0; s < splits; ++s) {
      const float ms = pm[s * Hq + hq];
      if (ms == -__builtin_inff()) continue;
      const float f = exp2f(ms - M);
      acc += f * po[(s * Hq + hq) * kHD + d];
      L += f * pl[s * Hq + hq];
    }
  }
  const float r = L > 0.0f ? acc / L : 0.0f;
  if (odt == HKV_DT_F32) ((float*)out)[(int64_t)hq * kHD + d] = r;
  else ((uint16_t*)out)[(int64_t)hq * kHD + d] = f2h(r);
}

}  // namespace

extern "C" size_t hkv_decode_workspace_bytes(int64_t nsel, int Hq, int pages_per_split) {
  if (nsel < 0 || Hq < 1 || pages_per_split < 1) return 0;
  const int64_t splits = nsel == 0 ? 1 : (nsel + pages_per_split - 1) / pages_per_split;
  return sizeof(float) * (size_t)splits * Hq * (2 + kHD);
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
  if (H < 1 || H > 65535 || Hq < H || Hq % H || Hq / H > 16 || T < 1 || nsel < 0 ||
      pages_per_split < 1)
    return HKV_ERR_SHAPE;
  if ((k_bits != 2 && k_bits != 4) || (v_bits != 2 && v_bits != 4)) return HKV_ERR_ARG;
  if (out_dtype != HKV_DT_F16 && out_dtype != HKV_DT_F32) return HKV_ERR_DTYPE;
  if (v_rows < 1 || k_cap < 0 || v_cap < 0) return HKV_ERR_ARG;
  if (T * H * D >= ((int64_t)1 << 31)) return HKV_ERR_SHAPE;
  if (!q || !k_packed || !k_row_ptr || !k_tables || !v_packed || !v_row_ptr || !v_tables || !out)
    return HKV_ERR_ARG;
  if ((k_cap > 0 && (!k_col || !k_val)) || (v_cap > 0 && (!v_col || !v_val))) return HKV_ERR_ARG;
  if (nsel > 0 && !sel) return HKV_ERR_ARG;
  if ((((uintptr_t)k_packed | (uintptr_t)v_packed) & 15u) || ((uintptr_t)q & 7u))
    return HKV_ERR_ARG;
  const size_t need = hkv_decode_workspace_bytes(nsel, Hq, pages_per_split);
  if (!workspace || workspace_bytes < need) return HKV_ERR_WORKSPACE;
  const int64_t splits = nsel == 0 ? 1 : (nsel + pages_per_split - 1) / pages_per_split;
  if (splits > 0x7fffffff) return HKV_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  float* pm = (float*)workspace;
  float* pl = pm + splits * Hq;
  float* po = pl + splits * Hq;
  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.k = Side{(const uint8_t*)k_packed, k_row_ptr, k_col, k_val, k_cap,
             (const hkv_table_t*)k_tables, 0, k_bits};
  a.v = Side{(const uint8_t*)v_packed, v_row_ptr, v_col, v_val, v_cap,
             (const hkv_table_t*)v_tables, v_rows, v_bits};
  a.H = H;
  a.group = Hq / H;
  a.T = T;
  a.sel = sel;
  a.nsel = nsel;
  a.pps = pages_per_split;
  a.scale = scale;
  a.part_m = pm;
  a.part_l = pl;
  a.part_o = po;
  hipLaunchKernelGGL(decode_kernel, dim3((unsigned)splits, (unsigned)H), dim3(kDT), 0, s, a);
  HKV_CHECK_LAUNCH();
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)Hq), dim3(kHD), 0, s, pm, pl, po, splits, Hq, H,
                     a.group, (int64_t)pages_per_split, nsel, out, out_dtype);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
