// nuq_tables.hip -- nearest-pole decision tables.
//
// A table replaces the L-level scan of the reference's pack kernels
// (src/kvquant/triton_batched.py:65-72: strict '<' over fp32 |v - pole|,
// lowest index on ties) by a binary search over L-1 sorted fp16 breakpoints.
// The construction: if the poles are finite and sorted with smallest distinct
// gap delta >= 2^E, then for |x| <= xsafe (xsafe + max|p| < 2^(E+23)) every
// |x - p| rounds with error < delta/2, so only the two nearest distinct poles
// compete and the scan's code is a non-decreasing step function of x.  Each
// breakpoint is the smallest fp16 x whose scanned code reaches c, found by
// bisection with the scan itself.  Inputs outside the safe range, and tables
// that fail the criterion, are decided by the scan at pack time.
#include "hkv_common.h"

namespace {

HKV_DEV float hval(int32_t k) { return h2f(hkey_inv(k)); }

// Smallest fp16 value (over -inf..+inf) >= t; NaN -> -inf.
HKV_DEV uint16_t h_ceil(float t) {
  if (__builtin_isnan(t)) return 0xfc00u;
  int32_t lo = hkey(0xfc00u), hi = hkey(0x7c00u);
  if (!(hval(hi) >= t)) return 0x7c00u;
  while (lo < hi) {
    int32_t mid = lo + (hi - lo) / 2;
    if (hval(mid) >= t) hi = mid; else lo = mid + 1;
  }
  return hkey_inv(lo);
}

// Largest fp16 value (over -inf..+inf) <= t; NaN -> +inf; zero -> +0.
HKV_DEV uint16_t h_floor(float t) {
  if (__builtin_isnan(t)) return 0x7c00u;
  int32_t lo = hkey(0xfc00u), hi = hkey(0x7c00u);
  if (!(hval(lo) <= t)) return 0xfc00u;
  while (lo < hi) {
    int32_t mid = hi - (hi - lo) / 2;
    if (hval(mid) <= t) lo = mid; else hi = mid - 1;
  }
  uint16_t r = hkey_inv(lo);
  return r == 0x8000u ? 0x0000u : r;
}

HKV_DEV int scan_local(float v, const float* p, int L) {
  float best = __builtin_inff();
  int idx = 0;
  for (int l = 0; l < L; ++l) {
    float d = __builtin_fabsf(__fsub_rn(v, p[l]));
    if (d < best) { best = d; idx = l; }
  }
  return idx;
}

__global__ void __launch_bounds__(256)
build_tables_kernel(const void* poles, int pdt, const void* upper, const void* lower, int tdt,
                    int64_t n, int L, hkv_table_t* out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float p[16];
  for (int l = 0; l < L; ++l) p[l] = load_scale(poles, pdt, i * L + l);
  const float up = load_scale(upper, tdt, i), lo = load_scale(lower, tdt, i);

  hkv_table_t t;
  for (int c = 0; c < 16; ++c) { t.bp[c] = 0x7c00u; t.pf16[c] = 0; }
  for (int l = 0; l < L; ++l) t.pf16[l] = f2h(p[l]);
  t.lo = h_ceil(lo);
  if (t.lo == 0x0000u) t.lo = 0x8000u;
  t.up = h_floor(up);
  t.levels = (uint16_t)L;
  t.pad[0] = t.pad[1] = t.pad[2] = 0;
  t.flags = 0;
  t.xsafe = 0;

  bool ok = L >= 1 && L <= 16;
  double pmax = 0.0, delta = __builtin_inf();
  for (int l = 0; l < L && ok; ++l) {
    if (!__builtin_isfinite(p[l])) { ok = false; break; }
    double a = __builtin_fabs((double)p[l]);
    if (a > pmax) pmax = a;
    if (l > 0) {
      if (p[l] < p[l - 1]) ok = false;
      else if (p[l] > p[l - 1] && (double)p[l] - (double)p[l - 1] < delta)
        delta = (double)p[l] - (double)p[l - 1];
    }
  }
  double bound = 65504.0;
  if (ok && __builtin_isfinite(delta)) {
    int E;
    frexp(delta, &E);
    double lim = ldexp(1.0, (E - 1) + 23) - pmax;
    if (lim < bound) bound = lim;
  }
  if (ok && bound > 0.0) {
    uint16_t xs = h_floor((float)bound);
    if (!((xs & 0x8000u) || h2f(xs) < 0.0f)) {
      while ((double)h2f(xs) >= bound && xs > 0) xs--;
      if (xs >= 0x7c00u) xs = 0x7bffu;
      t.xsafe = xs;
      t.flags = 1;
      int32_t klo = hkey((uint16_t)(xs | 0x8000u)), khi = hkey(xs);
      for (int c = 1; c < L; ++c) {
        if (scan_local(hval(khi), p, L) < c) { t.bp[c - 1] = 0x7c00u; continue; }
        int32_t a = klo, b = khi;
        while (a < b) {
          int32_t mid = a + (b - a) / 2;
          if (scan_local(hval(mid), p, L) >= c) b = mid; else a = mid + 1;
        }
        t.bp[c - 1] = hkey_inv(a);
      }
    }
  }
  out[i] = t;
}

}  // namespace

extern "C" const char* hkv_version(void) { return "helix_kv 0.1 (gfx950)"; }

extern "C" const char* hkv_status_string(int s) {
  switch (s) {
    case HKV_OK: return "ok";
    case HKV_ERR_ARG: return "invalid argument";
    case HKV_ERR_SHAPE: return "unsupported or inconsistent shape";
    case HKV_ERR_DTYPE: return "unsupported dtype";
    case HKV_ERR_CAPACITY: return "output capacity too small";
    case HKV_ERR_LAUNCH: return "kernel launch failed";
    case HKV_ERR_WORKSPACE: return "workspace missing or too small";
    case HKV_ERR_SCRATCH: return "problem exceeds the fixed scratch of the no-allocation entry point";
    default: return "unknown status";
  }
}

static bool dtype_ok(int dt) { return dt == HKV_DT_F16 || dt == HKV_DT_F32 || dt == HKV_DT_BF16; }

extern "C" int hkv_nuq_build_tables(const void* poles, int poles_dtype, const void* upper,
                                    const void* lower, int thr_dtype, int64_t n_tables, int levels,
                                    void* tables_out, void* stream) {
  if (n_tables < 0 || levels < 1 || levels > 16) return HKV_ERR_ARG;
  if (!dtype_ok(poles_dtype) || !dtype_ok(thr_dtype)) return HKV_ERR_DTYPE;
  if (n_tables == 0) return HKV_OK;
  if (!poles || !upper || !lower || !tables_out) return HKV_ERR_ARG;
  const int threads = 256;
  const int64_t blocks = (n_tables + threads - 1) / threads;
  hipLaunchKernelGGL(build_tables_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                     (hipStream_t)stream, poles, poles_dtype, upper, lower, thr_dtype, n_tables,
                     levels, (hkv_table_t*)tables_out);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
