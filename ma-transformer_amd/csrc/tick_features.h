// tick_features.h -- GPU-resident microstructure features of raw ticks.
//
// The reference computes, per tick i, in pandas float64
// (/root/reference src/data_loader.py:15-28):
//   spread_i = ask_i - bid_i
//   wap_i    = (bid_i * askv_i + ask_i * bidv_i) / (bidv_i + askv_i)
//   obi_i    = bidv_i / (bidv_i + askv_i)
//   dt_i     = ts_i - ts_{i-1}  (dt_0 = 0: diff().fillna(0))
// then z-scores each of [price, spread, wap, obi, dt] with the column mean
// and the sample standard deviation (ddof 1), and hands float32 rows to the
// model.  Here the columns stay on the device (structure of arrays, float64)
// and three launches produce the float32 [n, 5] rows:
//   features_stats   grid-stride pass: per-thread shifted sums turned into
//                    (count, mean, M2) of each feature, combined across a
//                    block's threads in a fixed tree (Chan et al.'s
//                    pairwise update);
//   features_finish  one wave per feature: combines the per-block partials
//                    (strided per lane, then a fixed shuffle tree) into
//                    mean and std (float64 [2][5]);
//   features_write   grid-stride pass: (f - mean) / std, rounded once to
//                    float32.
// Each feature is formed with explicitly rounded float64 operations
// (__dmul_rn / __dadd_rn / ...), in the reference's operation order, so the
// per-tick values are the pandas values bit for bit; the statistics differ
// from pandas' summation order only in the last bits.  HBM traffic: the six
// columns are read twice (48 B per tick each pass) and 20 B per tick written.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ma_feat {

constexpr int kFeatures = 5;
constexpr int kStatThreads = 256;
constexpr int kStatBlocks = 1024;  // upper bound on the first pass's grid

struct TickCols {
  const double* ts;
  const double* price;
  const double* bid;
  const double* ask;
  const double* bidv;
  const double* askv;
};

__device__ __forceinline__ void tick_features(const TickCols& c, int64_t i, double (&f)[kFeatures]) {
  const double bid = c.bid[i], ask = c.ask[i], bv = c.bidv[i], av = c.askv[i];
  const double vol = __dadd_rn(bv, av);
  f[0] = c.price[i];
  f[1] = __dsub_rn(ask, bid);
  f[2] = __ddiv_rn(__dadd_rn(__dmul_rn(bid, av), __dmul_rn(ask, bv)), vol);
  f[3] = __ddiv_rn(bv, vol);
  f[4] = i > 0 ? __dsub_rn(c.ts[i], c.ts[i - 1]) : 0.0;
}

// (count, mean, M2) of a set; merge of two sets (Chan, Golub, LeVeque 1979).
struct Moments {
  double n, mean, m2;
};

__device__ __forceinline__ Moments merge(const Moments& a, const Moments& b) {
  if (a.n == 0.0) return b;
  if (b.n == 0.0) return a;
  const double n = a.n + b.n;
  const double inv = 1.0 / n;
  const double d = b.mean - a.mean;
  Moments r;
  r.n = n;
  r.mean = a.mean + d * (b.n * inv);
  r.m2 = a.m2 + b.m2 + d * d * (a.n * b.n * inv);
  return r;
}

// Merge of one Moments per thread across a block of kStatThreads threads in a
// fixed pairwise tree (thread t with t + w, w = 128, 64, ..., 1), so the
// result does not depend on scheduling.  Valid in thread 0; sh is reusable
// after the final barrier.
__device__ __forceinline__ Moments block_merge(Moments m, double (*sh)[3]) {
  const int t = threadIdx.x;
  sh[t][0] = m.n;
  sh[t][1] = m.mean;
  sh[t][2] = m.m2;
  __syncthreads();
  for (int w = kStatThreads / 2; w > 0; w >>= 1) {
    if (t < w) {
      m = merge(m, Moments{sh[t + w][0], sh[t + w][1], sh[t + w][2]});
      sh[t][0] = m.n;
      sh[t][1] = m.mean;
      sh[t][2] = m.m2;
    }
    __syncthreads();
  }
  return m;
}

__global__ __launch_bounds__(kStatThreads) void features_stats(TickCols c, int64_t n, double* partial) {
  __shared__ double sh[kStatThreads][3];
  // Shifted sums per thread (the shifted-data algorithm): s1 = sum(f - K),
  // s2 = sum((f - K)^2) with K the thread's first value of the feature, so
  // the loop has no division; M2 = s2 - s1^2 / cnt loses about
  // eps * (1 + cnt (mean - K)^2 / M2) relative, O(eps) for K drawn from the
  // column itself.
  double shift[kFeatures], s1[kFeatures], s2[kFeatures];
#pragma unroll
  for (int k = 0; k < kFeatures; ++k) shift[k] = s1[k] = s2[k] = 0.0;
  double cnt = 0.0;
  const int64_t stride = (int64_t)gridDim.x * kStatThreads;
  const int64_t i0 = (int64_t)blockIdx.x * kStatThreads + threadIdx.x;
  if (i0 < n) tick_features(c, i0, shift);
  for (int64_t i = i0; i < n; i += stride) {
    double f[kFeatures];
    tick_features(c, i, f);
    cnt += 1.0;
#pragma unroll
    for (int k = 0; k < kFeatures; ++k) {
      const double d = f[k] - shift[k];
      s1[k] += d;
      s2[k] = fma(d, d, s2[k]);
    }
  }
  for (int k = 0; k < kFeatures; ++k) {
    Moments own{0.0, 0.0, 0.0};
    if (cnt > 0.0) {
      const double dm = s1[k] / cnt;
      own = Moments{cnt, shift[k] + dm, fmax(s2[k] - s1[k] * dm, 0.0)};
    }
    const Moments m = block_merge(own, sh);
    if (threadIdx.x == 0) {
      double* p = partial + ((int64_t)blockIdx.x * kFeatures + k) * 3;
      p[0] = m.n;
      p[1] = m.mean;
      p[2] = m.m2;
    }
  }
}

// One wave per feature (kFeatures waves): lane l merges partials l, l + 64,
// ... in order, then a fixed shuffle tree across the wave (lane l with
// l + w, w = 32, ..., 1).  stats: [0..4] means, [5..9] sample standard
// deviations (ddof 1; NaN for fewer than two ticks, as pandas).
constexpr int kFinishThreads = 64 * kFeatures;

__global__ __launch_bounds__(kFinishThreads) void features_finish(const double* partial, int blocks, double* stats) {
  const int k = threadIdx.x >> 6, l = threadIdx.x & 63;
  // the lane's partials are loaded before the first merge (kStatBlocks / 64 at most)
  Moments part[kStatBlocks / 64];
#pragma unroll
  for (int j = 0; j < kStatBlocks / 64; ++j) {
    const int b = l + 64 * j;
    const double* p = partial + ((int64_t)b * kFeatures + k) * 3;
    part[j] = b < blocks ? Moments{p[0], p[1], p[2]} : Moments{0.0, 0.0, 0.0};
  }
  Moments m = part[0];
#pragma unroll
  for (int j = 1; j < kStatBlocks / 64; ++j) m = merge(m, part[j]);
  for (int w = 32; w > 0; w >>= 1) {
    const Moments o{__shfl_down(m.n, w), __shfl_down(m.mean, w), __shfl_down(m.m2, w)};
    if (l < w) m = merge(m, o);
  }
  if (l == 0) {
    stats[k] = m.mean;
    stats[kFeatures + k] = m.n > 1.0 ? sqrt(m.m2 / (m.n - 1.0)) : __builtin_nan("");
  }
}

__global__ __launch_bounds__(256) void features_write(TickCols c, int64_t n, const double* stats, float* out) {
  double mean[kFeatures], sd[kFeatures];
#pragma unroll
  for (int k = 0; k < kFeatures; ++k) {
    mean[k] = stats[k];
    sd[k] = stats[kFeatures + k];
  }
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    double f[kFeatures];
    tick_features(c, i, f);
#pragma unroll
    for (int k = 0; k < kFeatures; ++k) out[i * kFeatures + k] = (float)__ddiv_rn(__dsub_rn(f[k], mean[k]), sd[k]);
  }
}

}  // namespace ma_feat
