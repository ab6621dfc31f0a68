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
// staged once per block; V: the slots' per-token poles), applies its slot's
// CSR outliers in registers, and writes 64 contiguous bytes.
#include "hkv_common.h"

namespace {

constexpr int kGT = 256;
constexpr int kGW = kGT / 64;
constexpr int kGD = 128;        // head dim
constexpr int kGPS = 16;        // page size (tokens)
constexpr int kMaxSeqsG = 64;

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

template <int NB, bool PT>
__global__ void __launch_bounds__(kGT)
gather_pages_kernel(GArgs A, const GSegs sg) {
  extern __shared__ __align__(16) uint16_t g_lds[];  // K: [H][kGD*16+64]; V: [kGW][16][16]
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int H = A.H;
  if constexpr (!PT) {
    for (int i = tid; i < H * kGD * 16; i += kGT) {
      const int h = i / (kGD * 16), d = (i / 16) % kGD, l = i % 16;
      g_lds[glut_index(h, d, l)] = A.tabs[(int64_t)h * kGD + d].pf16[l];
    }
    __syncthreads();
  }
  uint16_t* vl = g_lds + wv * (kGPS * 16);
  const int row = lane >> 2, q = lane & 3;
  const int64_t items = A.nrows * H;
  for (int64_t it = (int64_t)blockIdx.x * kGW + wv; it < items; it += (int64_t)gridDim.x * kGW) {
    const int64_t i = it / H;
    const int h = (int)(it - i * H);
    int b = 0;  // sequence of selection row i (uniform)
    while (b + 1 < sg.nseg && sg.out_off[b + 1] <= i) ++b;
    const int64_t P = sg.off[b + 1] - sg.off[b];
    const int64_t lp = A.sel[i * H + h];
    const bool page_ok = lp >= 0 && lp < P;
    const int64_t t = (sg.off[b] + (page_ok ? lp : 0)) * kGPS + row;
    const bool ok = page_ok && t < A.T;
    const int64_t r = (ok ? t : 0) * H + h;
    uint32_t w[NB];
    if constexpr (NB == 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(A.packed + r * (kGD / 2) + q * 16);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(A.packed + r * (kGD / 4) + q * 8);
      w[0] = v.x; w[1] = v.y;
    }
    const int2 rb = *reinterpret_cast<const int2*>(A.row_ptr + r);
    if constexpr (PT) {
      const int64_t pos = (page_ok ? lp : 0) * kGPS + row;
      const int64_t vrow = pos < A.rows ? pos : A.rows - 1;
      const uint2 tv = *reinterpret_cast<const uint2*>(A.tabs[(int64_t)h * A.rows + vrow].pf16 + 4 * q);
      *reinterpret_cast<uint2*>(vl + row * 16 + 4 * q) = tv;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    uint32_t o[16];
#pragma unroll
    for (int e2 = 0; e2 < 16; ++e2) {
      uint32_t pr = 0;
#pragma unroll
      for (int hl = 0; hl < 2; ++hl) {
        const int e = 2 * e2 + hl;  // channel 32q + e
        uint32_t code;
        if constexpr (NB == 4) code = (w[e >> 3] >> (4 * (e & 7))) & 15u;
        else code = (w[e >> 4] >> (2 * (e & 15))) & 3u;
        uint16_t v;
        if constexpr (PT) v = vl[row * 16 + (int)code];
        else v = g_lds[glut_index(h, 32 * q + e, (int)code)];
        pr |= (uint32_t)v << (16 * hl);
      }
      o[e2] = ok ? pr : 0u;
    }
    if (ok) {  // this slot's outliers in channels [32q, 32q+32)
      const int64_t a = rb.x < 0 ? 0 : rb.x;
      const int64_t e = rb.y < A.cap ? rb.y : A.cap;
      for (int64_t k = a; k < e; ++k) {
        const int d = (int)A.col[k] - 32 * q;
        if (d >= 0 && d < 32) {
          const uint32_t v = A.val[k];
#pragma unroll
          for (int j = 0; j < 16; ++j)
            if (j == (d >> 1)) o[j] = (d & 1) ? ((o[j] & 0xffffu) | (v << 16)) : ((o[j] & 0xffff0000u) | v);
        }
      }
    }
    uint4* dst = reinterpret_cast<uint4*>(A.out + ((i * kGPS + row) * H + h) * kGD + 32 * q);
#pragma unroll
    // plain stores: a store instruction covers 16-byte pieces of several
    // lines, which L2 merges (streaming stores would write them out partial)
    for (int k = 0; k < 4; ++k) dst[k] = make_uint4(o[4 * k], o[4 * k + 1], o[4 * k + 2], o[4 * k + 3]);
    if constexpr (PT) {  // the V LUT is rewritten by the wave's next item
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
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
  const size_t lds = pt ? sizeof(uint16_t) * kGW * kGPS * 16 : sizeof(uint16_t) * H * (kGD * 16 + 64);
  if (lds > 64 * 1024) return HKV_ERR_SHAPE;
  GArgs a;
  a.packed = (const uint8_t*)packed;
  a.row_ptr = row_ptr;
  a.col = col;
  a.val = val;
  a.cap = capacity;
  a.tabs = (const hkv_table_t*)scales->tables;
  a.rows = scales->rows;
  a.T = T;
  a.H = H;
  a.sel = sel;
  a.nrows = nrows;
  a.out = (uint16_t*)out;
  const int64_t items = nrows * H;
  const unsigned grid =
      (unsigned)std::min<int64_t>((items + kGW - 1) / kGW, (int64_t)gather_cus() * 8);
  hipStream_t s = (hipStream_t)stream;
  if (bits == 4) {
    if (pt) hipLaunchKernelGGL((gather_pages_kernel<4, true>), dim3(grid), dim3(kGT), lds, s, a, sg);
    else hipLaunchKernelGGL((gather_pages_kernel<4, false>), dim3(grid), dim3(kGT), lds, s, a, sg);
  } else {
    if (pt) hipLaunchKernelGGL((gather_pages_kernel<2, true>), dim3(grid), dim3(kGT), lds, s, a, sg);
    else hipLaunchKernelGGL((gather_pages_kernel<2, false>), dim3(grid), dim3(kGT), lds, s, a, sg);
  }
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
