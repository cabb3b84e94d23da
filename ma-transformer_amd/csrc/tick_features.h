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
//   features_stats   grid-stride pass: per-block (count, mean, M2) of each
//                    feature, combined across a block's threads in a fixed
//                    tree (Chan et al.'s pairwise update);
//   features_finish  one block: combines the per-block partials in block
//                    order into mean and std (float64 [2][5]);
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
  const double d = b.mean - a.mean;
  Moments r;
  r.n = n;
  r.mean = a.mean + d * (b.n / n);
  r.m2 = a.m2 + b.m2 + d * d * (a.n * b.n / n);
  return r;
}

__global__ __launch_bounds__(kStatThreads) void features_stats(TickCols c, int64_t n, double* partial) {
  __shared__ double sh[kStatThreads][3];
  Moments acc[kFeatures];
#pragma unroll
  for (int k = 0; k < kFeatures; ++k) acc[k] = Moments{0.0, 0.0, 0.0};
  const int64_t stride = (int64_t)gridDim.x * kStatThreads;
  for (int64_t i = (int64_t)blockIdx.x * kStatThreads + threadIdx.x; i < n; i += stride) {
    double f[kFeatures];
    tick_features(c, i, f);
#pragma unroll
    for (int k = 0; k < kFeatures; ++k) {  // Welford update
      acc[k].n += 1.0;
      const double d = f[k] - acc[k].mean;
      acc[k].mean += d / acc[k].n;
      acc[k].m2 += d * (f[k] - acc[k].mean);
    }
  }
  for (int k = 0; k < kFeatures; ++k) {
    sh[threadIdx.x][0] = acc[k].n;
    sh[threadIdx.x][1] = acc[k].mean;
    sh[threadIdx.x][2] = acc[k].m2;
    __syncthreads();
    for (int w = kStatThreads / 2; w > 0; w >>= 1) {
      if ((int)threadIdx.x < w) {
        const Moments a{sh[threadIdx.x][0], sh[threadIdx.x][1], sh[threadIdx.x][2]};
        const Moments b{sh[threadIdx.x + w][0], sh[threadIdx.x + w][1], sh[threadIdx.x + w][2]};
        const Moments m = merge(a, b);
        sh[threadIdx.x][0] = m.n;
        sh[threadIdx.x][1] = m.mean;
        sh[threadIdx.x][2] = m.m2;
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      double* p = partial + ((int64_t)blockIdx.x * kFeatures + k) * 3;
      p[0] = sh[0][0];
      p[1] = sh[0][1];
      p[2] = sh[0][2];
    }
    __syncthreads();
  }
}

// stats: [0..4] means, [5..9] sample standard deviations (ddof 1)
__global__ __launch_bounds__(64) void features_finish(const double* partial, int blocks, double* stats) {
  const int k = threadIdx.x;
  if (k >= kFeatures) return;
  Moments m{0.0, 0.0, 0.0};
  for (int b = 0; b < blocks; ++b) {
    const double* p = partial + ((int64_t)b * kFeatures + k) * 3;
    m = merge(m, Moments{p[0], p[1], p[2]});
  }
  stats[k] = m.mean;
  stats[kFeatures + k] = m.n > 1.0 ? sqrt(m.m2 / (m.n - 1.0)) : __builtin_nan("");
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
