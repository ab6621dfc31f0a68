// nuq_generic.hip -- broadcasting nuq quantise / dequantise with the
// reference CPU spec's dtype semantics (src/kvquant/nuq.py:22-156).
//
// quantise: per element of a broadcast shape (<= 6 dims),
//   diff_l = round_cdt(v - pole_l)   (cdt = promoted dtype of values and poles:
//                                     the fp32 difference rounded to fp16/bf16
//                                     when that is the promoted type)
//   code   = first argmin_l |diff_l|                 (nuq.py:36-37)
//   mask   = v < lower || v > upper  (exact fp32 compare, nuq.py:72)
//   recon  = mask ? v : pole[code], stored in the promoted dtype (nuq.py:131)
// dequantise: out = mask ? outliers : pole[code], in the outliers' dtype
//   (nuq.py:155-156).
#include "hkv_common.h"

namespace {

constexpr int kMaxDims = 6;

struct Shape {
  int ndim;
  int64_t size[kMaxDims];
};

HKV_DEV float load_any(const void* p, int dt, int64_t i) {
  switch (dt) {
    case HKV_DT_F32: return ((const float*)p)[i];
    case HKV_DT_BF16: return __builtin_bit_cast(float, (uint32_t)((const uint16_t*)p)[i] << 16);
    case HKV_DT_F16: return h2f(((const uint16_t*)p)[i]);
    case HKV_DT_I64: return (float)((const int64_t*)p)[i];
    case HKV_DT_I32: return (float)((const int32_t*)p)[i];
    default: return (float)((const uint8_t*)p)[i];
  }
}

HKV_DEV int64_t load_index(const void* p, int dt, int64_t i) {
  switch (dt) {
    case HKV_DT_I64: return ((const int64_t*)p)[i];
    case HKV_DT_I32: return ((const int32_t*)p)[i];
    default: return ((const uint8_t*)p)[i];
  }
}

// float -> bf16 round to nearest even (NaN kept quiet).
HKV_DEV uint16_t f2bf(float f) {
  uint32_t b = __builtin_bit_cast(uint32_t, f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  b += 0x7fffu + ((b >> 16) & 1u);
  return (uint16_t)(b >> 16);
}

HKV_DEV float round_to(float f, int dt) {
  if (dt == HKV_DT_F16) return h2f(f2h(f));
  if (dt == HKV_DT_BF16) return __builtin_bit_cast(float, (uint32_t)f2bf(f) << 16);
  return f;
}

HKV_DEV void store_float(void* p, int dt, int64_t i, float v) {
  if (dt == HKV_DT_F32) ((float*)p)[i] = v;
  else if (dt == HKV_DT_BF16) ((uint16_t*)p)[i] = f2bf(v);
  else ((uint16_t*)p)[i] = f2h(v);
}

HKV_DEV int64_t offset(const Shape& s, const int64_t* st, int64_t i) {
  int64_t off = 0;
  for (int d = s.ndim - 1; d >= 0; --d) {
    const int64_t k = i % s.size[d];
    i /= s.size[d];
    off += k * st[d];
  }
  return off;
}

__global__ void __launch_bounds__(256)
quantize_generic(Shape s, int64_t n, hkv_tensor_desc v, hkv_tensor_desc p, int64_t lstride, int L,
                 hkv_tensor_desc up, hkv_tensor_desc lo, int cdt, int64_t* codes, void* recon,
                 int rdt, uint8_t* mask) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const float x = load_any(v.data, v.dtype, offset(s, v.strides, i));
    const int64_t pb = offset(s, p.strides, i);
    float best = __builtin_inff();
    int idx = 0;
    bool any = false;
    for (int l = 0; l < L; ++l) {
      const float d = __builtin_fabsf(round_to(__fsub_rn(x, load_any(p.data, p.dtype, pb + l * lstride)), cdt));
      // argmin over a row whose entries are all NaN returns the first NaN;
      // otherwise NaN entries never win (torch's argmin propagates NaN: the
      // first NaN is returned).  Track NaN explicitly.
      if (__builtin_isnan(d)) {
        if (!any) { idx = l; any = true; best = d; }
        continue;
      }
      if (!any && d < best) { best = d; idx = l; }
    }
    bool m = false;
    if (up.data) {
      const float u = load_any(up.data, up.dtype, offset(s, up.strides, i));
      const float w = load_any(lo.data, lo.dtype, offset(s, lo.strides, i));
      m = (x < w) || (x > u);
    }
    if (codes) codes[i] = idx;
    if (mask) mask[i] = m;
    if (recon) {
      const float q = load_any(p.data, p.dtype, pb + (int64_t)idx * lstride);
      store_float(recon, rdt, i, m ? x : q);
    }
  }
}

__global__ void __launch_bounds__(256)
dequantize_generic(Shape s, int64_t n, hkv_tensor_desc c, hkv_tensor_desc ov, hkv_tensor_desc om,
                   hkv_tensor_desc p, int64_t lstride, int L, void* out, int odt, int32_t* err) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const bool m = load_index(om.data, om.dtype, offset(s, om.strides, i)) != 0;
    float r;
    if (m) {
      r = load_any(ov.data, ov.dtype, offset(s, ov.strides, i));
    } else {
      int64_t code = load_index(c.data, c.dtype, offset(s, c.strides, i));
      if (code < 0 || code >= L) { atomicOr(err, 1); code = 0; }
      // the pole is first rounded to the outliers' dtype (nuq.py:156)
      r = round_to(load_any(p.data, p.dtype, offset(s, p.strides, i) + code * lstride), odt);
    }
    store_float(out, odt, i, r);
  }
}

int blocks_for(int64_t n) {
  return (int)std::min<int64_t>((n + 255) / 256, 65536);
}

bool float_dt(int dt) { return dt == HKV_DT_F16 || dt == HKV_DT_F32 || dt == HKV_DT_BF16; }
bool index_dt(int dt) { return dt == HKV_DT_I64 || dt == HKV_DT_I32 || dt == HKV_DT_U8; }

}  // namespace

extern "C" int hkv_nuq_quantize_generic(int ndim, const int64_t* shape, const hkv_tensor_desc* values,
                                        const hkv_tensor_desc* poles, int64_t level_stride,
                                        int levels, const hkv_tensor_desc* upper,
                                        const hkv_tensor_desc* lower, int compute_dtype,
                                        int64_t* codes, void* recon, int recon_dtype,
                                        uint8_t* mask, void* stream) {
  if (ndim < 0 || ndim > kMaxDims || !shape || !values || !poles) return HKV_ERR_ARG;
  if (levels < 1 || (upper == nullptr) != (lower == nullptr)) return HKV_ERR_ARG;
  if (!float_dt(values->dtype) || !float_dt(poles->dtype) || !float_dt(compute_dtype))
    return HKV_ERR_DTYPE;
  if (recon && !float_dt(recon_dtype)) return HKV_ERR_DTYPE;
  if (upper && (!float_dt(upper->dtype) || !float_dt(lower->dtype))) return HKV_ERR_DTYPE;
  Shape s;
  s.ndim = ndim;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) return HKV_ERR_SHAPE;
    s.size[d] = shape[d];
    n *= shape[d];
  }
  if (n == 0) return HKV_OK;
  hkv_tensor_desc none{};
  hipLaunchKernelGGL(quantize_generic, dim3(blocks_for(n)), dim3(256), 0, (hipStream_t)stream, s, n,
                     *values, *poles, level_stride, levels, upper ? *upper : none,
                     lower ? *lower : none, compute_dtype, codes, recon, recon_dtype, mask);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}

extern "C" int hkv_nuq_dequantize_generic(int ndim, const int64_t* shape, const hkv_tensor_desc* codes,
                                          const hkv_tensor_desc* outliers,
                                          const hkv_tensor_desc* outlier_mask,
                                          const hkv_tensor_desc* poles, int64_t level_stride,
                                          int levels, void* out, int out_dtype, int32_t* err,
                                          void* stream) {
  if (ndim < 0 || ndim > kMaxDims || !shape || !codes || !outliers || !outlier_mask || !poles ||
      !err)
    return HKV_ERR_ARG;
  if (!index_dt(codes->dtype) || !index_dt(outlier_mask->dtype) || !float_dt(outliers->dtype) ||
      !float_dt(poles->dtype) || !float_dt(out_dtype))
    return HKV_ERR_DTYPE;
  Shape s;
  s.ndim = ndim;
  int64_t n = 1;
  for (int d = 0; d < ndim; ++d) {
    if (shape[d] < 0) return HKV_ERR_SHAPE;
    s.size[d] = shape[d];
    n *= shape[d];
  }
  if (n == 0) return HKV_OK;
  hipLaunchKernelGGL(dequantize_generic, dim3(blocks_for(n)), dim3(256), 0, (hipStream_t)stream, s,
                     n, *codes, *outliers, *outlier_mask, *poles, level_stride, levels, out,
                     out_dtype, err);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
