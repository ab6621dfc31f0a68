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


// ------------------------------------------------------ optimal 1-D k-means
//
// The k-means objective in one dimension has an exact solution by dynamic
// programming over the sorted values (Wang & Song, "Ckmeans.1d.dp", R Journal
// 2011; Groenlund et al., "Fast exact k-means, k-medians and Bregman
// divergence clustering in 1D", 2017): with x sorted ascending and
//   cost(j, i) = sum_{t=j..i} x_t^2 - (sum_{t=j..i} x_t)^2 / (i - j + 1)
// (from fp64 prefix sums S1, S2 of x and x^2),
//   D[0][i] = cost(0, i)
//   D[m][i] = min_{m <= j <= i} D[m-1][j-1] + cost(j, i)        (m = 1..k-1)
// the optimum is D[k-1][n-1], and clusters are recovered from the argmins.
// Each D row is rounded to fp32 (the candidate sums are fp64), the leftmost
// argmin wins ties.  The argmin of a row is non-decreasing in i (the cost has
// the quadrangle inequality), so a row is computed by divide and conquer over
// i: the middle i of a range searches j between the argmins of its range's
// neighbours, which are ancestors in the fixed halving tree; the tree is
// walked level by level, each node searched by a group of lanes
// (min(64, 256 >> level)) with a shuffle reduction.  Centres are the
// clusters' means (fp64 sum / count, rounded to fp32), ascending.
//
// One block fits one problem at a time (a persistent grid over problems).
// LDS holds S1, S2 (fp64), two D rows (fp32) and the row's argmins (int16)
// for n <= kDpMax values (the sorting buffer reuses the D rows); every row's
// argmins also go to the block's slice of the workspace for the backward walk.
// Problems of more than kDpMax values are not solved: their centres are NaN.
// Fewer than k values give the reference's padding (the values and k - n
// zeros, sorted), as hkv_kmeans_1d.
constexpr int kDpMax = 6144;
constexpr int kDpT = 256;
constexpr size_t kDpLds = 2 * 8 * (kDpMax + 1) + 2 * 4 * kDpMax + 2 * kDpMax;

HKV_DEV double dp_cost(const double* S1, const double* S2, int j, int i) {
  const double s = S1[i + 1] - S1[j];
  const double q = S2[i + 1] - S2[j];
  return q - s * s / (double)(i - j + 1);
}

__global__ void __launch_bounds__(kDpT)
kmeans_dp_kernel(const float* __restrict__ values, const int64_t* __restrict__ offsets,
                 int64_t n_problems, int k, float* __restrict__ centers,
                 int16_t* __restrict__ ws_opt) {
  extern __shared__ __align__(16) unsigned char dp_lds[];
  double* S1 = reinterpret_cast<double*>(dp_lds);
  double* S2 = S1 + (kDpMax + 1);
  float* Dp = reinterpret_cast<float*>(S2 + (kDpMax + 1));
  float* Dc = Dp + kDpMax;
  int16_t* opt = reinterpret_cast<int16_t*>(Dc + kDpMax);
  float* sbuf = Dp;  // the sort's buffer (8192 floats = both D rows)
  __shared__ float s_c[kKmMaxK];
  const int tid = threadIdx.x;
  int16_t* gopt = ws_opt + (int64_t)blockIdx.x * (kKmMaxK - 1) * kDpMax;

  for (int64_t p = blockIdx.x; p < n_problems; p += gridDim.x) {
    const int64_t b = offsets[p], n64 = offsets[p + 1] - b;
    float* out = centers + p * k;
    if (n64 < 0 || n64 > kDpMax) {  // malformed, or too large for the exact fit
      if (tid < k) out[tid] = __builtin_nanf("");
      continue;
    }
    const int n = (int)n64;
    const float* v = values + b;
    if (n < k) {  // the reference's padding case, including n == 0
      if (tid == 0) {
        for (int l = 0; l < k; ++l) s_c[l] = l < n ? v[l] : 0.0f;
        sort_small(s_c, k);
        for (int l = 0; l < k; ++l) out[l] = s_c[l];
      }
      __syncthreads();
      continue;
    }
    // sort (bitonic over the next power of two, +inf padding)
    int sz = 2;
    while (sz < n) sz <<= 1;
    for (int i = tid; i < sz; i += kDpT) sbuf[i] = i < n ? v[i] : __builtin_inff();
    __syncthreads();
    for (int size = 2; size <= sz; size <<= 1) {
      for (int stride = size >> 1; stride > 0; stride >>= 1) {
        for (int t = tid; t < sz / 2; t += kDpT) {
          const int i = 2 * t - (t & (stride - 1));
          const int j = i + stride;
          const bool up = (i & size) == 0;
          const float a = sbuf[i], bv = sbuf[j];
          if ((a > bv) == up) {
            sbuf[i] = bv;
            sbuf[j] = a;
          }
        }
        __syncthreads();
      }
    }
    // prefix sums S1, S2 (fp64): a block scan, chunks of the sorted values
    // summed in order per thread, then the threads' totals in order
    {
      const int per = (n + kDpT - 1) / kDpT;
      const int i0 = tid * per, i1 = i0 + per < n ? i0 + per : n;
      double a1 = 0.0, a2 = 0.0;
      for (int i = i0; i < i1; ++i) {
        const double x = (double)sbuf[i];
        a1 += x;
        a2 += x * x;
      }
      // exclusive scan of the threads' totals, through the front of S1 / S2
      // (written with the prefix sums only after every thread has read them)
      __syncthreads();
      double* t1 = S1;  // thread totals, temporarily at the front
      double* t2 = S2;
      t1[tid] = a1;
      t2[tid] = a2;
      __syncthreads();
      double b1 = 0.0, b2 = 0.0;
      for (int t = 0; t < tid; ++t) {
        b1 += t1[t];
        b2 += t2[t];
      }
      __syncthreads();
      double c1 = b1, c2 = b2;
      if (tid == 0) {
        S1[0] = 0.0;
        S2[0] = 0.0;
      }
      for (int i = i0; i < i1; ++i) {
        const double x = (double)sbuf[i];
        c1 += x;
        c2 += x * x;
        S1[i + 1] = c1;
        S2[i + 1] = c2;
      }
    }
    __syncthreads();
    // row 0: one cluster over x[0..i]
    for (int i = tid; i < n; i += kDpT) Dp[i] = (float)dp_cost(S1, S2, 0, i);
    __syncthreads();
    const int last = k - 1;
    for (int m = 1; m <= last; ++m) {
      // i runs over [m, n - 1 - (last - m)] (enough values for the later
      // clusters); the last row needs only i = n - 1
      const int ilo = m == last ? n - 1 : m;
      const int ihi = n - 1 - (last - m);
      const int span = ihi - ilo + 1;
      int levels = 0;
      while ((1 << levels) < span + 1) ++levels;
      for (int L = 0; L < levels; ++L) {
        const int g = (kDpT >> L) < 64 ? ((kDpT >> L) > 0 ? (kDpT >> L) : 1) : 64;
        const int nodes = 1 << L;
        const int per_pass = kDpT / g;
        for (int t0 = 0; t0 < nodes; t0 += per_pass) {
          const int t = t0 + tid / g, gl = tid % g;
          int a = ilo, z = ihi;
          bool live = t < nodes;
          for (int bit = L - 1; bit >= 0 && live; --bit) {
            const int mid = (a + z) >> 1;
            if ((t >> bit) & 1) a = mid + 1;
            else z = mid - 1;
            live = a <= z;
          }
          double best = __builtin_inf();
          int bj = 0x7fffffff;
          int mid = (a + z) >> 1;
          if (live) {
            const int jlo = a - 1 >= ilo ? opt[a - 1] : m;
            int jhi = z + 1 <= ihi ? opt[z + 1] : mid;
            jhi = jhi < mid ? jhi : mid;
            for (int j = jlo + gl; j <= jhi; j += g) {
              const double c = (double)Dp[j - 1] + dp_cost(S1, S2, j, mid);
              if (c < best) {
                best = c;
                bj = j;
              }
            }
          }
          // leftmost minimum over the group (xor offsets below g stay in it)
          for (int o = 1; o < g; o <<= 1) {
            const double ob = __shfl_xor(best, o, 64);
            const int oj = __shfl_xor(bj, o, 64);
            if (ob < best || (ob == best && oj < bj)) {
              best = ob;
              bj = oj;
            }
          }
          if (live && gl == 0) {
            Dc[mid] = (float)best;
            opt[mid] = (int16_t)bj;
            gopt[(int64_t)(m - 1) * kDpMax + mid] = (int16_t)bj;
          }
        }
        __syncthreads();
      }
      float* tmp = Dp;
      Dp = Dc;
      Dc = tmp;
      sbuf = Dp;
    }
    // backward walk: cluster m is [j, i] with j = argmin of row m at i
    __syncthreads();
    if (tid == 0) {
      int i = n - 1;
      for (int m = last; m >= 1; --m) {
        const int j = gopt[(int64_t)(m - 1) * kDpMax + i];
        s_c[m] = (float)((S1[i + 1] - S1[j]) / (double)(i - j + 1));
        i = j - 1;
      }
      s_c[0] = (float)(S1[i + 1] / (double)(i + 1));
      for (int l = 0; l < k; ++l) out[l] = s_c[l];
    }
    __syncthreads();
    Dp = reinterpret_cast<float*>(S2 + (kDpMax + 1));
    Dc = Dp + kDpMax;
    sbuf = Dp;
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

extern "C" size_t hkv_kmeans_1d_optimal_workspace_bytes(void) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kmeans_dp_kernel, kDpT, kDpLds) != hipSuccess ||
      per_cu < 1)
    per_cu = 1;
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = 256;
  return (size_t)per_cu * cus * (kKmMaxK - 1) * kDpMax * sizeof(int16_t);
}

extern "C" int hkv_kmeans_1d_optimal(const float* values, const int64_t* offsets, int64_t n_problems,
                                     int k, float* centers, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (n_problems < 0 || n_problems > 0x7fffffff) return HKV_ERR_SHAPE;
  if (k < 1 || k > kKmMaxK) return HKV_ERR_ARG;
  if (!values || !offsets || !centers) return HKV_ERR_ARG;
  if (n_problems == 0) return HKV_OK;
  const size_t slice = (size_t)(kKmMaxK - 1) * kDpMax * sizeof(int16_t);
  if (!workspace || workspace_bytes < slice) return HKV_ERR_WORKSPACE;
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute((const void*)kmeans_dp_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)kDpLds) != hipSuccess)
      return HKV_ERR_LAUNCH;
    attr = true;
  }
  const int64_t slots = (int64_t)(workspace_bytes / slice);
  const unsigned grid = (unsigned)std::min<int64_t>(n_problems, slots);
  hipLaunchKernelGGL(kmeans_dp_kernel, dim3(grid), dim3(kDpT), kDpLds, (hipStream_t)stream, values,
                     offsets, n_problems, k, centers, (int16_t*)workspace);
  HKV_CHECK_LAUNCH();
  return HKV_OK;
}
