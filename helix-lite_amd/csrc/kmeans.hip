// kmeans.hip -- batched 1-D k-means (Lloyd) for nuq calibration.
//
// The calibration step either side of the hot path: the reference fits one
// 1-D k-means per (head, channel) of K and per (head, position) of V with
// sklearn on the CPU (src/kvquant/calibration.py:106-188, _kmeans_1d inside
// the _calibrate_keys / _calibrate_values loops), some 17,000 fits per layer.
// Here one block fits one problem, all problems of a layer in one launch.
//
// Problem p is values[offsets[p] .. offsets[p+1]) (fp32, finite).  Its k
// centres (k <= 16) start at order statistics of the problem's n values,
//   c_l = sorted[floor((2l + 1) n / 2k)]       (n <= kKmLds, sorted in LDS)
// or, for larger problems, evenly spread over [min, max]:
//   c_l = fl(min + fl(fl(max - min) * fl((2l + 1) / 2k)))
// and take `iters` Lloyd steps: every value joins the first centre of least
// fp32 |v - c| (the lowest index wins ties), then each centre with members
// moves to their mean -- a float64 sum over the members divided by their count,
// rounded to fp32 -- and a centre without members stays.  The centres are
// written sorted ascending.  As in the reference's _kmeans_1d
// (calibration.py:113-119): no values give k zeros; fewer than k values give
// the values and k - n zeros, sorted.
//
// The fp64 sums run per thread over a fixed stride of the values, then across
// the block in a fixed order, so the result does not depend on scheduling.
// A problem that fits (kKmLds floats) is staged in LDS once and sorted there
// by a bitonic network over the next power of two (padded with +inf); larger
// ones are re-read from global (L2) at each step.
#include "hkv_common.h"

namespace {

constexpr int kKmT = 256;
constexpr int kKmW = kKmT / 64;
constexpr int kKmMaxK = 16;
constexpr int kKmLds = 8192;  // a power of two: the bitonic sort's size

HKV_DEV double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
HKV_DEV int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Insertion sort of s[0..k) by one thread.
HKV_DEV void sort_small(float* s, int k) {
  for (int i = 1; i < k; ++i) {
    const float x = s[i];
    int j = i - 1;
    while (j >= 0 && s[j] > x) {
      s[j + 1] = s[j];
      --j;
    }
    s[j + 1] = x;
  }
}

__global__ void __launch_bounds__(kKmT)
kmeans_kernel(const float* __restrict__ values, const int64_t* __restrict__ offsets, int k,
              int iters, float* __restrict__ centers) {
  __shared__ float s_v[kKmLds];
  __shared__ float s_c[kKmMaxK];
  __shared__ double s_sum[kKmW][kKmMaxK];
  __shared__ int s_cnt[kKmW][kKmMaxK];
  __shared__ float s_mn[kKmW], s_mx[kKmW];

  const int64_t p = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t b = offsets[p], n64 = offsets[p + 1] - b;
  float* out = centers + p * k;
  if (n64 < 0 || n64 > 0x7fffffff) {  // malformed offsets: flag the problem
    if (tid < k) out[tid] = __builtin_nanf("");
    return;
  }
  const int n = (int)n64;
  const float* v = values + b;
  if (n < k) {  // the reference's padding case, including n == 0
    if (tid == 0) {
      for (int l = 0; l < k; ++l) s_c[l] = l < n ? v[l] : 0.0f;
      sort_small(s_c, k);
      for (int l = 0; l < k; ++l) out[l] = s_c[l];
    }
    return;
  }
  const bool staged = n <= kKmLds;
  float mn = __builtin_inff(), mx = -__builtin_inff();
  for (int i = tid; i < n; i += kKmT) {
    const float x = v[i];
    if (staged) s_v[i] = x;
    mn = fminf(mn, x);
    mx = fmaxf(mx, x);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  }
  if (lane == 0) {
    s_mn[wv] = mn;
    s_mx[wv] = mx;
  }
  __syncthreads();
  if (staged) {
    int sz = 2;  // the sort's size: the next power of two >= n
    while (sz < n) sz <<= 1;
    for (int i = n + tid; i < sz; i += kKmT) s_v[i] = __builtin_inff();
    __syncthreads();
    for (int size = 2; size <= sz; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int t = tid; t < sz / 2; t += kKmT) {
          const int i = 2 * t - (t & (stride - 1));  // low element of the pair
          const int j = i + stride;
          const bool up = (i & size) == 0;
          const float a = s_v[i], bv = s_v[j];
          if ((a > bv) == up) {
            s_v[i] = bv;
            s_v[j] = a;
          }
        }
        __syncthreads();
      }
    }
    if (tid < k) s_c[tid] = s_v[((2 * tid + 1) * n) / (2 * k)];
  } else if (tid < k) {
    float a = s_mn[0], z = s_mx[0];
    for (int w = 1; w < kKmW; ++w) {
      a = fminf(a, s_mn[w]);
      z = fmaxf(z, s_mx[w]);
    }
    const float frac = (float)(2 * tid + 1) / (float)(2 * k);
    s_c[tid] = __fadd_rn(a, __fmul_rn(__fsub_rn(z, a), frac));
  }
  __syncthreads();

  for (int it = 0; it < iters; ++it) {
    float c[kKmMaxK];
    double sum[kKmMaxK];
    int cnt[kKmMaxK];
#pragma unroll
    for (int l = 0; l < kKmMaxK; ++l) {
      c[l] = l < k ? s_c[l] : 0.0f;
      sum[l] = 0.0;
      cnt[l] = 0;
    }
    for (int i = tid; i < n; i += kKmT) {
      const float x = staged ? s_v[i] : v[i];
      float best = __builtin_fabsf(__fsub_rn(x, c[0]));
      int bl = 0;
#pragma unroll
      for (int l = 1; l < kKmMaxK; ++l) {
        const float d = __builtin_fabsf(__fsub_rn(x, c[l]));
        if (l < k && d < best) {
          best = d;
          bl = l;
        }
      }
#pragma unroll
      for (int l = 0; l < kKmMaxK; ++l) {
        if (l == bl) {
          sum[l] += (double)x;
          cnt[l] += 1;
        }
      }
    }
#pragma unroll
    for (int l = 0; l < kKmMaxK; ++l) {
      if (l < k) {
        const double s = wave_sum_f64(sum[l]);
        const int m = wave_sum_i32(cnt[l]);
        if (lane == 0) {
          s_sum[wv][l] = s;
          s_cnt[wv][l] = m;
        }
      }
    }
    __syncthreads();
    if (tid < k) {
      double s = 0.0;
      int m = 0;
      for (int w = 0; w < kKmW; ++w) {
        s += s_sum[w][tid];
        m += s_cnt[w][tid];
      }
      if (m > 0) s_c[tid] = (float)(s / (double)m);
    }
    __syncthreads();
  }
  if (tid == 0) {
    sort_small(s_c, k);
    for (int l = 0; l < k; ++l) out[l] = s_c[l];
  }
}

}  // namespace

extern "C" int hkv_kmeans_1d(const float* values, const int64_t* offsets, int64_t n_problems,
                             int k, int iters, float* centers, void* stream) {
  if (n_problems < 0 || n_problems > 0x7fffffff) return HKV_ERR_SHAPE;
  if (k < 1 || k > kKmMaxK || iters < 0) return HKV_ERR_ARG;
  if (!values || !offsets || !centers) return HKV_ERR_ARG;
  if (n_problems == 0) return HKV_OK;
  hipLaunchKernelGGL(kmeans_kernel, dim3((unsigned)n_problems), dim3(kKmT), 0,
                     (hipStream_t)stream, values, offsets, k, iters, centers);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
