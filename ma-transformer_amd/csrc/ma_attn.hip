// ma_attn.hip -- MI355X (gfx950) sparse-attention forward engine behind the
// C-ABI of include/ma_attn.h.
//
// Kernels
//   band_kernel<T>   bf16/fp16, head_dim 64, SLIDING (any dilation): one
//                    workgroup per 64-query tile of one (batch, head, residue
//                    class); the K/V band of the tile is staged in LDS (K row
//                    major, V transposed) and both contractions run on MFMA
//                    (16x16x32 for Q.K^T, 16x16x16 for P.V) with an online
//                    softmax held in registers.  One O store per row.
//   gather_rows_kernel<T>  head_dim 64, any key set (index sets among them)
//                    the tiled kernels do not take: one wave per query row,
//                    8 whole K or V rows per load instruction.
//   rows_kernel<T>   every pattern / dtype / head_dim: one wave per query
//                    row, lanes over keys for the scores, lanes over head_dim
//                    for P.V (above 512, in passes of 512 output columns).
//                    Used where no other kernel applies.
//
// Semantics follow ma_core::compute_sparse_attention
// (/root/reference src/csrc/ma_core.cpp:160-246): softmax over the row's key
// set with scale 1/sqrtf(D), empty set => zero row.  The reference GPU
// launcher this replaces is sparse_forward_cuda
// (src/cuda/sparse_attention_kernel.cu:423-458).
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <algorithm>
#include <atomic>
#include <cstring>
#include <mutex>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "../../include/ma_attn.h"
#include "../../include/ma_features.h"
#include "device_common.h"
#include "pattern.h"
#include "stream_kernel.h"
#include "block_kernel.h"
#include "backward_kernel.h"
#include "bwd_fused_kernel.h"
#include "bwd_longformer_kernel.h"
#include "tile_kernel.h"
#include "tick_features.h"

// Scratch of ma_attn_forward_noalloc: device memory the library owns, one
// copy per GPU (each at its own address), held until the process ends.  Host
// code never names this array in a launch or a copy: its name is a host-side
// stand-in, not a device address.  scratch_of_stream() gives the address on
// the stream's device (hipGetSymbolAddress, once per device).
static __device__ __align__(256) unsigned char scratch[MA_ATTN_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return 1;
}

}  // namespace

// The library's one error channel, shared with the other translation units
// (ma_attn_last_error() reads it).
namespace ma_host {
void clear_error() { g_last_error.clear(); }
int set_error(const char* msg) {
  g_last_error = msg;
  return 1;
}
}  // namespace ma_host

namespace {

// ------------------------------------------------------------------ options
//
// Kernel-selection switches for tests and A/B timing, read from the
// environment once, when the library loads (ma_attn_reload_options reads
// them again):
//   MA_ATTN_KERNEL=rows     every launch on the generic row kernels
//   MA_ATTN_KERNEL=band     16-bit windows on the band kernel, not the stream kernel
//   MA_ATTN_NO_FIXED=1      forward windows on the generic stream tiles
//   MA_ATTN_BWD_NO_FIXED=1  backward windows on the generic stream tiles
//   MA_ATTN_BWD_UNFUSED=1   the fixed-window 16-bit backward as two launches (dQ, then dK/dV)
struct Options {
  bool force_rows, force_band, no_fixed, bwd_no_fixed, bwd_unfused;
};

Options read_options() {
  const char* k = getenv("MA_ATTN_KERNEL");
  Options o;
  o.force_rows = k && strcmp(k, "rows") == 0;
  o.force_band = k && strcmp(k, "band") == 0;
  o.no_fixed = getenv("MA_ATTN_NO_FIXED") != nullptr;
  o.bwd_no_fixed = getenv("MA_ATTN_BWD_NO_FIXED") != nullptr;
  o.bwd_unfused = getenv("MA_ATTN_BWD_UNFUSED") != nullptr;
  return o;
}

Options g_opt = read_options();

// ------------------------------------------------------------------ devices
//
// The device a launch runs on is its stream's (the null stream: the current
// device's).
int stream_device(hipStream_t st, int* dev) {
  const hipError_t e = st ? hipStreamGetDevice(st, dev) : hipGetDevice(dev);
  if (e != hipSuccess) return fail("ma_attn: cannot query the stream's device: %s", hipGetErrorString(e));
  return 0;
}

// Raises a kernel's dynamic-LDS limit to `shm` bytes once per (kernel,
// device), with that device current; safe from any number of threads.
int reserve_lds(const void* kern, size_t shm, hipStream_t st) {
  int dev = 0;
  if (stream_device(st, &dev)) return 1;
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({kern, dev})) return 0;
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return fail("ma_attn: hipGetDevice failed");
  if (cur != dev && hipSetDevice(dev) != hipSuccess) return fail("ma_attn: cannot select device %d", dev);
  const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
  if (cur != dev) (void)hipSetDevice(cur);
  if (e != hipSuccess) return fail("ma_attn: cannot reserve %zu B of LDS: %s", shm, hipGetErrorString(e));
  done.insert({kern, dev});
  return 0;
}

using namespace ma_dev;

// ------------------------------------------------------------------ launches
//
// Events of the current ma_attn_*_timed call (null otherwise): the call's
// first kernel takes the start event and its last kernel the stop event, so
// they bracket the kernels' own execution (hipExtLaunchKernel stamps them on
// the dispatch packets; no extra queue packets).
thread_local hipEvent_t g_ev_start = nullptr;
thread_local hipEvent_t g_ev_stop = nullptr;

template <typename F, typename... Args>
void launch(bool last, F kernel, dim3 grid, dim3 block, uint32_t shm, hipStream_t st, Args... args) {
  hipEvent_t e0 = g_ev_start, e1 = last ? g_ev_stop : nullptr;
  if (e0 || e1) {
    g_ev_start = nullptr;
    if (last) g_ev_stop = nullptr;
    hipExtLaunchKernelGGL(kernel, grid, block, shm, st, e0, e1, 0u, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shm, st, args...);
  }
}

// ------------------------------------------------------------------ element access

template <typename T>
__device__ __forceinline__ float ld_f(const T* p) {
  return static_cast<float>(*p);
}

template <typename T>
__device__ __forceinline__ T cvt_out(float x) {
  return static_cast<T>(x);
}

// ------------------------------------------------------------------ wave64 reductions

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m, 64));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

__device__ __forceinline__ float bcast_f(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

__device__ __forceinline__ int bcast_i(int x, int lane) {
  return __builtin_amdgcn_readlane(x, lane);
}

// ------------------------------------------------------------------ rows_kernel

constexpr int kRowsWaves = 4;

// One wave per query row (row = (b*N + i)*H + h).  Scores: lane t of a
// 64-key chunk owns key key_at(t); online softmax across chunks (m, l, acc).
// P.V: lanes own head_dim slots d = lane + 64*c.
// STATS (backward): instead of O, writes the row's softmax statistics
// stats[row] = {lse, delta}: lse = m + log(l) of the scaled scores, delta =
// dout . O with O kept in fp32.
// WIDE (head_dim above 64*DPL): the query row is read from memory rather
// than LDS, and the output columns are done in passes of 64*DPL, each pass
// recomputing the row's scores over the whole head_dim.
struct RowStat {
  float lse, delta;
};

template <typename T, int DPL, bool STATS = false, bool WIDE = false>
__global__ __launch_bounds__(256) void rows_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                   const T* __restrict__ v, T* __restrict__ o,
                                                   int64_t B, int64_t H, int64_t D,
                                                   ma::PatternParams pp, float scale,
                                                   const T* __restrict__ dout = nullptr,
                                                   RowStat* __restrict__ stats = nullptr) {
  extern __shared__ float q_lds[];  // kRowsWaves * D floats (not WIDE)
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t N = pp.n;
  const int64_t row = (int64_t)blockIdx.x * kRowsWaves + wv;
  const bool row_ok = row < B * N * H;
  const int64_t rr = row_ok ? row : 0;
  const int64_t h = rr % H;
  const int64_t bi = rr / H;
  const int64_t i = bi % N;
  const int64_t b = bi / N;
  const int64_t rs = H * D;  // elements between consecutive tokens

  float* qw = q_lds + wv * D;
  if constexpr (!WIDE) {
    for (int64_t d = lane; d < D; d += 64) qw[d] = row_ok ? ld_f(q + rr * D + d) : 0.0f;
    __syncthreads();
  }
  if (!row_ok) return;  // no barrier below this point
  auto qd = [&](int64_t d) -> float {
    if constexpr (WIDE)
      return ld_f(q + rr * D + d);
    else
      return qw[d];
  };

  const T* kb = k + (b * N * H + h) * D;
  const T* vb = v + (b * N * H + h) * D;
  const ma::RowKeys rk = ma::row_keys(pp, i);
  const int64_t cnt = rk.count;

  float m = -INFINITY, l = 0.0f, part = 0.0f;
  for (int64_t col0 = 0; col0 < (WIDE ? D : 1); col0 += 64 * DPL) {  // one pass unless WIDE
    m = -INFINITY;
    l = 0.0f;
    float acc[DPL];
#pragma unroll
    for (int c = 0; c < DPL; ++c) acc[c] = 0.0f;

    for (int64_t c0 = 0; c0 < cnt; c0 += 64) {
      const int64_t t = c0 + lane;
      const int64_t jk0 = t < cnt ? ma::key_at(pp, rk, i, t) : -1;
      // closed-form keys are always in range; an index set's are checked here
      const bool valid = jk0 >= 0 && jk0 < N;
      const int64_t j = valid ? jk0 : 0;
      float s = -INFINITY;
      if (valid) {
        const T* kr = kb + j * rs;
        float dot = 0.0f;
        for (int64_t d = 0; d < D; ++d) dot = fmaf(qd(d), ld_f(kr + d), dot);
        s = dot * scale;
      }
      // mn is -inf only while every key so far was skipped (index sets)
      const float mn = fmaxf(m, wave_max(s));
      const float mu = mn == -INFINITY ? 0.0f : mn;
      const float corr = expf(m - mu);
      const float p = valid ? expf(s - mu) : 0.0f;
      l = l * corr + wave_sum(p);
#pragma unroll
      for (int c = 0; c < DPL; ++c) acc[c] *= corr;
      const int nk = (int)ma::imin64(64, cnt - c0);
      for (int kk = 0; kk < nk; ++kk) {
        const float pk = bcast_f(p, kk);
        const int64_t jk = (int64_t)bcast_i((int)j, kk);
        const T* vr = vb + jk * rs;
#pragma unroll
        for (int c = 0; c < DPL; ++c) {
          const int64_t d = col0 + lane + 64 * c;
          if (d < D) acc[c] = fmaf(pk, ld_f(vr + d), acc[c]);
        }
      }
      m = mn;
    }
    const float inv = cnt > 0 && l != 0.0f ? 1.0f / l : 0.0f;
    if constexpr (STATS) {
#pragma unroll
      for (int c = 0; c < DPL; ++c) {
        const int64_t d = col0 + lane + 64 * c;
        if (d < D) part = fmaf(ld_f(dout + rr * D + d), acc[c] * inv, part);
      }
    } else {
      T* orow = o + rr * D;
#pragma unroll
      for (int c = 0; c < DPL; ++c) {
        const int64_t d = col0 + lane + 64 * c;
        if (d < D) orow[d] = cvt_out<T>(acc[c] * inv);
      }
    }
  }
  if constexpr (STATS) {
    const float delta = wave_sum(part);
    if (lane == 0) stats[rr] = RowStat{cnt > 0 && l > 0.0f ? m + logf(l) : 0.0f, delta};
  }
}

// ------------------------------------------------------------------ narrow_kernel
//
// Narrow heads (head_dim <= 32), SLIDING with dilation 1 and left, right >= 0:
// one workgroup (4 waves) per 64 consecutive queries of one (batch, head),
// one query per lane.  The K/V rows those queries read,
// [64w-left, 64w+63+right], are staged in LDS as fp32 rows of DP + 4 floats
// (DP = head_dim padded to 16 or 32; the 4-float pad makes the 16-byte reads
// of 16 consecutive rows hit 64 distinct banks).  Wave v takes the v-th
// quarter of each query's window, in groups of 16 keys (scores in registers,
// one rescale per group), lane l reading row l + step so that a wave reads
// consecutive rows; waves 1-3 leave (max, sum, acc) partials in LDS and wave
// 0 merges them (log-sum-exp) and writes O.
constexpr int kNarrowWaves = 4;

template <int DP>
constexpr int narrow_row() { return DP + 4; }

template <typename T, int DP>
__global__ __launch_bounds__(256) void narrow_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                     const T* __restrict__ v, T* __restrict__ o, int64_t N,
                                                     int64_t H, int D, int left, int right, float scale) {
  extern __shared__ __attribute__((aligned(16))) float band[];  // K rows, V rows, then wave partials
  constexpr int RS = narrow_row<DP>();
  constexpr int PS = DP + 2;  // partial: acc[DP], max, sum
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t tiles = (N + 63) / 64;
  const int64_t t = blockIdx.x % tiles;
  const int64_t bh = blockIdx.x / tiles;
  const int64_t h = bh % H, b = bh / H;
  const int64_t rs = H * D;  // elements between consecutive tokens
  const T* qb = q + (b * N * H + h) * D;
  const T* kb = k + (b * N * H + h) * D;
  const T* vb = v + (b * N * H + h) * D;
  T* ob = o + (b * N * H + h) * D;

  const int64_t i0 = 64 * t;
  const int64_t j0 = i0 - left > 0 ? i0 - left : 0;
  const int64_t j1 = i0 + 63 + right < N - 1 ? i0 + 63 + right : N - 1;
  const int rows = (int)(j1 - j0 + 1);
  float* kl = band;
  float* vl = band + (size_t)rows * RS;
  float* part = vl + (size_t)rows * RS;  // [wave 1..3][lane][PS]

  // The lane's query row is loaded first (it depends on nothing), then the
  // band in batches of 8 elements per thread: every load of a batch is
  // issued (indices clamped into range, so unconditionally) before the
  // stores that wait for them, and the causal-64 band at head_dim 16 (127 rows of 16) is one
  // batch -- a single global round trip before the barrier.
  const int64_t i = i0 + lane;
  const int64_t ic = i < N ? i : N - 1;
  float qv[DP];
#pragma unroll
  for (int d = 0; d < DP; ++d) qv[d] = ld_f(qb + ic * rs + (d < D ? d : D - 1));
  const int ne = rows * DP;
  for (int e0 = 0; e0 < ne; e0 += 256 * 8) {
    float kx[8], vx[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = min(e0 + tid + 256 * u, ne - 1);
      const int r = e / DP, d = min(e % DP, D - 1);
      const int64_t off = (j0 + r) * rs + d;
      kx[u] = ld_f(kb + off);
      vx[u] = ld_f(vb + off);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int e = e0 + tid + 256 * u;
      if (e < ne) {
        const int r = e / DP, d = e % DP;
        kl[r * RS + d] = d < D ? kx[u] : 0.0f;
        vl[r * RS + d] = d < D ? vx[u] : 0.0f;
      }
    }
  }
#pragma unroll
  for (int d = 0; d < DP; ++d) qv[d] = d < D ? qv[d] : 0.0f;
  __syncthreads();

  // this wave's quarter of the query's window
  const int64_t lo = i - left > 0 ? i - left : 0;
  const int64_t hi = ic + right < N - 1 ? ic + right : N - 1;
  const int64_t per = (hi - lo + kNarrowWaves) / kNarrowWaves;
  const int64_t plo = lo + wv * per;
  const int64_t phi = plo + per - 1 < hi ? plo + per - 1 : hi;
  const float sl2 = scale * 1.4426950408889634f;  // scores in log2 units, exp2 below
  float m = -INFINITY, l = 0.0f, acc[DP];
#pragma unroll
  for (int d = 0; d < DP; ++d) acc[d] = 0.0f;
  for (int64_t g0 = plo; g0 <= phi; g0 += 16) {
    float sc[16];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int64_t j = g0 + u;
      const float* kr = kl + (j <= phi ? j - j0 : 0) * RS;
      float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
#pragma unroll
      for (int d = 0; d < DP; d += 4) {
        const float4 kk = *reinterpret_cast<const float4*>(kr + d);
        d0 = fmaf(qv[d], kk.x, d0);
        d1 = fmaf(qv[d + 1], kk.y, d1);
        d2 = fmaf(qv[d + 2], kk.z, d2);
        d3 = fmaf(qv[d + 3], kk.w, d3);
      }
      sc[u] = j <= phi ? ((d0 + d1) + (d2 + d3)) * sl2 : -INFINITY;
      mx = fmaxf(mx, sc[u]);
    }
    const float mn = fmaxf(m, mx);  // finite: the group's first key is in the part
    const float corr = __builtin_amdgcn_exp2f(m - mn);
    l *= corr;
#pragma unroll
    for (int d = 0; d < DP; ++d) acc[d] *= corr;
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float p = __builtin_amdgcn_exp2f(sc[u] - mn);
      l += p;
      const float* vr = vl + (g0 + u <= phi ? g0 + u - j0 : 0) * RS;
#pragma unroll
      for (int d = 0; d < DP; d += 4) {
        const float4 vv = *reinterpret_cast<const float4*>(vr + d);
        acc[d] = fmaf(p, vv.x, acc[d]);
        acc[d + 1] = fmaf(p, vv.y, acc[d + 1]);
        acc[d + 2] = fmaf(p, vv.z, acc[d + 2]);
        acc[d + 3] = fmaf(p, vv.w, acc[d + 3]);
      }
    }
    m = mn;
  }
  if (wv > 0) {
    float* pw = part + ((wv - 1) * 64 + lane) * PS;
#pragma unroll
    for (int d = 0; d < DP; ++d) pw[d] = acc[d];
    pw[DP] = m;
    pw[DP + 1] = l;
  }
  __syncthreads();
  if (wv != 0 || i >= N) return;  // after the last barrier
  for (int w = 1; w < kNarrowWaves; ++w) {
    const float* pw = part + ((w - 1) * 64 + lane) * PS;
    const float mw = pw[DP];
    const float mn = fmaxf(m, mw);
    if (mn == -INFINITY) continue;  // both parts empty
    const float c0 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mn);
    const float c1 = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - mn);
    l = l * c0 + pw[DP + 1] * c1;
#pragma unroll
    for (int d = 0; d < DP; ++d) acc[d] = acc[d] * c0 + pw[d] * c1;
    m = mn;
  }
  const float inv = hi >= lo ? 1.0f / l : 0.0f;
#pragma unroll
  for (int d = 0; d < DP; ++d)
    if (d < D) ob[i * rs + d] = cvt_out<T>(acc[d] * inv);
}

// ------------------------------------------------------------------ backward row kernels
//
// Gradients of O = softmax(S) V, S = Q K^T * scale over each row's key set,
// as the reference's backward kernels define them
// (/root/reference src/cuda/sparse_attention_kernel.cu:265-346, dense
// :104-175): with p_ij = exp(s_ij - lse_i), dp_ij = dout_i . v_j and
// ds_ij = p_ij (dp_ij - delta_i),
//   dq_i = scale * sum_{j in S_i} ds_ij k_j
//   dk_j = scale * sum_{i in T_j} ds_ij q_i,   dv_j = sum_{i in T_j} p_ij dout_i
// where T_j = {i : j in S_i}, and delta_i = sum_j p_ij dp_ij = dout_i . O_i
// (the reference's s_dot, :306-316).  Three launches and no atomics: the
// statistics (rows_kernel<STATS>), dq per query row, dk/dv per key row.  For
// SLIDING (and DENSE, a window of N-1) T_j is itself a sliding set with left
// and right swapped, so the key-row kernel walks it with the same closed
// forms.  Same lane layout as rows_kernel: lanes over the set's entries for
// the dot products, lanes over head_dim for the accumulations.

// dq: one wave per query row; q_i and dout_i cached in LDS (WIDE: read from
// memory, and dq done in column passes of 64*DPL, each recomputing the
// row's scores and dP over the whole head_dim).
template <typename T, int DPL, bool WIDE = false>
__global__ __launch_bounds__(256) void bwd_dq_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                     const T* __restrict__ v, const T* __restrict__ dout,
                                                     const RowStat* __restrict__ stats, T* __restrict__ dq,
                                                     int64_t B, int64_t H, int64_t D, ma::PatternParams pp,
                                                     float scale) {
  extern __shared__ float row_lds[];  // kRowsWaves * 2 * D floats (not WIDE)
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t N = pp.n;
  const int64_t row = (int64_t)blockIdx.x * kRowsWaves + wv;
  const bool row_ok = row < B * N * H;
  const int64_t rr = row_ok ? row : 0;
  const int64_t h = rr % H;
  const int64_t bi = rr / H;
  const int64_t i = bi % N;
  const int64_t b = bi / N;
  const int64_t rs = H * D;

  float* qw = row_lds + wv * 2 * D;
  float* gw = qw + D;
  if constexpr (!WIDE) {
    for (int64_t d = lane; d < D; d += 64) {
      qw[d] = row_ok ? ld_f(q + rr * D + d) : 0.0f;
      gw[d] = row_ok ? ld_f(dout + rr * D + d) : 0.0f;
    }
    __syncthreads();
  }
  if (!row_ok) return;  // no barrier below this point
  auto qd = [&](int64_t d) -> float {
    if constexpr (WIDE)
      return ld_f(q + rr * D + d);
    else
      return qw[d];
  };
  auto gd = [&](int64_t d) -> float {
    if constexpr (WIDE)
      return ld_f(dout + rr * D + d);
    else
      return gw[d];
  };

  const T* kb = k + (b * N * H + h) * D;
  const T* vb = v + (b * N * H + h) * D;
  const ma::RowKeys rk = ma::row_keys(pp, i);
  const int64_t cnt = rk.count;
  const RowStat st = stats[rr];

  for (int64_t col0 = 0; col0 < (WIDE ? D : 1); col0 += 64 * DPL) {  // one pass unless WIDE
    float acc[DPL];
#pragma unroll
    for (int c = 0; c < DPL; ++c) acc[c] = 0.0f;
    for (int64_t c0 = 0; c0 < cnt; c0 += 64) {
      const int64_t t = c0 + lane;
      const int64_t j0 = t < cnt ? ma::key_at(pp, rk, i, t) : -1;
      const bool valid = j0 >= 0 && j0 < N;  // an index set's keys are checked here
      const int64_t j = valid ? j0 : 0;
      float ds = 0.0f;
      if (valid) {
        const T* kr = kb + j * rs;
        const T* vr = vb + j * rs;
        float sdot = 0.0f, pdot = 0.0f;
        for (int64_t d = 0; d < D; ++d) {
          sdot = fmaf(qd(d), ld_f(kr + d), sdot);
          pdot = fmaf(gd(d), ld_f(vr + d), pdot);
        }
        const float p = expf(sdot * scale - st.lse);
        ds = p * (pdot - st.delta);
      }
      const int nk = (int)ma::imin64(64, cnt - c0);
      for (int kk = 0; kk < nk; ++kk) {
        const float dsk = bcast_f(ds, kk);
        const T* kr = kb + (int64_t)bcast_i((int)j, kk) * rs;
#pragma unroll
        for (int c = 0; c < DPL; ++c) {
          const int64_t d = col0 + lane + 64 * c;
          if (d < D) acc[c] = fmaf(dsk, ld_f(kr + d), acc[c]);
        }
      }
    }
    T* out = dq + rr * D;
#pragma unroll
    for (int c = 0; c < DPL; ++c) {
      const int64_t d = col0 + lane + 64 * c;
      if (d < D) out[d] = cvt_out<T>(acc[c] * scale);
    }
  }
}

// dk, dv: one wave per key row j over the query set T_j (pt = the transposed
// pattern); k_j and v_j cached in LDS (WIDE: as bwd_dq_kernel).
template <typename T, int DPL, bool WIDE = false>
__global__ __launch_bounds__(256) void bwd_dkv_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                      const T* __restrict__ v, const T* __restrict__ dout,
                                                      const RowStat* __restrict__ stats, T* __restrict__ dk,
                                                      T* __restrict__ dv, int64_t B, int64_t H, int64_t D,
                                                      ma::PatternParams pt, float scale) {
  extern __shared__ float row_lds[];  // kRowsWaves * 2 * D floats (not WIDE)
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int64_t N = pt.n;
  const int64_t row = (int64_t)blockIdx.x * kRowsWaves + wv;
  const bool row_ok = row < B * N * H;
  const int64_t rr = row_ok ? row : 0;
  const int64_t h = rr % H;
  const int64_t bj = rr / H;
  const int64_t j = bj % N;
  const int64_t b = bj / N;
  const int64_t rs = H * D;

  float* kw = row_lds + wv * 2 * D;
  float* vw = kw + D;
  if constexpr (!WIDE) {
    for (int64_t d = lane; d < D; d += 64) {
      kw[d] = row_ok ? ld_f(k + rr * D + d) : 0.0f;
      vw[d] = row_ok ? ld_f(v + rr * D + d) : 0.0f;
    }
    __syncthreads();
  }
  if (!row_ok) return;  // no barrier below this point
  auto kd = [&](int64_t d) -> float {
    if constexpr (WIDE)
      return ld_f(k + rr * D + d);
    else
      return kw[d];
  };
  auto vd = [&](int64_t d) -> float {
    if constexpr (WIDE)
      return ld_f(v + rr * D + d);
    else
      return vw[d];
  };

  const T* qb = q + (b * N * H + h) * D;
  const T* gb = dout + (b * N * H + h) * D;
  const RowStat* sb = stats + b * N * H + h;
  const ma::RowKeys rq = ma::row_keys(pt, j);
  const int64_t cnt = rq.count;

  for (int64_t col0 = 0; col0 < (WIDE ? D : 1); col0 += 64 * DPL) {  // one pass unless WIDE
    float acc_k[DPL], acc_v[DPL];
#pragma unroll
    for (int c = 0; c < DPL; ++c) acc_k[c] = acc_v[c] = 0.0f;
    for (int64_t c0 = 0; c0 < cnt; c0 += 64) {
      const int64_t t = c0 + lane;
      const int64_t i0 = t < cnt ? ma::key_at(pt, rq, j, t) : -1;
      const bool valid = i0 >= 0 && i0 < N;  // a transposed index set's queries are checked here
      const int64_t i = valid ? i0 : 0;
      float p = 0.0f, ds = 0.0f;
      if (valid) {
        const T* qr = qb + i * rs;
        const T* gr = gb + i * rs;
        float sdot = 0.0f, pdot = 0.0f;
        for (int64_t d = 0; d < D; ++d) {
          sdot = fmaf(ld_f(qr + d), kd(d), sdot);
          pdot = fmaf(ld_f(gr + d), vd(d), pdot);
        }
        const RowStat st = sb[i * H];
        p = expf(sdot * scale - st.lse);
        ds = p * (pdot - st.delta);
      }
      const int nk = (int)ma::imin64(64, cnt - c0);
      for (int kk = 0; kk < nk; ++kk) {
        const float pk = bcast_f(p, kk);
        const float dsk = bcast_f(ds, kk);
        const int64_t ik = (int64_t)bcast_i((int)i, kk);
        const T* qr = qb + ik * rs;
        const T* gr = gb + ik * rs;
#pragma unroll
        for (int c = 0; c < DPL; ++c) {
          const int64_t d = col0 + lane + 64 * c;
          if (d < D) {
            acc_v[c] = fmaf(pk, ld_f(gr + d), acc_v[c]);
            acc_k[c] = fmaf(dsk, ld_f(qr + d), acc_k[c]);
          }
        }
      }
    }
    T* ok = dk + rr * D;
    T* ov = dv + rr * D;
#pragma unroll
    for (int c = 0; c < DPL; ++c) {
      const int64_t d = col0 + lane + 64 * c;
      if (d < D) {
        ok[d] = cvt_out<T>(acc_k[c] * scale);
        ov[d] = cvt_out<T>(acc_v[c]);
      }
    }
  }
}

// ------------------------------------------------------------------ band_kernel (MFMA)

constexpr int kBandD = 64;         // head_dim handled by band_kernel
constexpr int kBandQ = 64;         // queries per workgroup (4 waves x 16)
constexpr int kBandKC = 128;       // keys staged per LDS stage
constexpr int kKsStride = 72;      // K row in LDS: 64 + 8 pad (144 B: conflict-free 16 B reads)
constexpr int kVtStride = kBandKC + 8;  // V^T row in LDS: 136 (272 B: conflict-free 8 B reads)

struct BandArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t B, N, H;
  int64_t left, right, dil;
  int64_t tiles;     // query tiles per residue class (ceil(ceil(N/dil)/64))
  float scale_log2;  // scale * log2(e)
};

// Workgroup -> (b, tile, h, rho) with the dispatcher's round-robin over the
// 8 XCDs undone, so each XCD walks a contiguous run of tiles (the K/V halo of
// tile t+1 is the tile t block that the same XCD's L2 just fetched).
__device__ __forceinline__ int64_t xcd_linear(int64_t bid, int64_t nwg) {
  const int64_t xcd = bid & 7, idx = bid >> 3;
  const int64_t per = nwg >> 3, rem = nwg & 7;
  return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

template <typename T>
__global__ __launch_bounds__(256) void band_kernel(BandArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[kBandKC * kKsStride];
  __shared__ __attribute__((aligned(16))) uint16_t vt[kBandD * kVtStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int c = lane & 15;  // MFMA column: this lane's query within the wave tile
  const int g = lane >> 4;  // MFMA row group: keys 4g..4g+3 of a 16-key sub-tile

  int64_t lin = xcd_linear(blockIdx.x, gridDim.x);
  const int64_t rho = lin % a.dil;
  lin /= a.dil;
  const int64_t h = lin % a.H;
  lin /= a.H;
  const int64_t tile = lin % a.tiles;
  const int64_t b = lin / a.tiles;

  const int64_t Nr = (a.N - rho + a.dil - 1) / a.dil;  // length of residue class rho
  const int64_t m0 = tile * kBandQ;
  if (m0 >= Nr) return;  // whole workgroup: uniform exit before any barrier

  // element offset of (b, residue index m, h, 0)
  const int64_t tok_stride = a.dil * a.H * kBandD;
  const int64_t base = ((b * a.N + rho) * a.H + h) * kBandD;
  const uint16_t* Q = static_cast<const uint16_t*>(a.q) + base;
  const uint16_t* K = static_cast<const uint16_t*>(a.k) + base;
  const uint16_t* V = static_cast<const uint16_t*>(a.v) + base;
  uint16_t* O = static_cast<uint16_t*>(a.o) + base;

  // Q^T operand (B of the 16x16x32 MFMA): query column c, head_dim slice 8g..8g+7 (+32)
  const int64_t qa = m0 + 16 * wv;  // first query of this wave
  const int64_t qm = qa + c;        // this lane's query
  const bool wave_has_q = qa < Nr;
  const bool q_ok = qm < Nr;
  uint4 qb0 = make_uint4(0, 0, 0, 0), qb1 = make_uint4(0, 0, 0, 0);
  if (q_ok) {
    const uint16_t* qr = Q + qm * tok_stride + 8 * g;
    qb0 = *reinterpret_cast<const uint4*>(qr);
    qb1 = *reinterpret_cast<const uint4*>(qr + 32);
  }

  const int64_t need_lo = ma::imax64(qa - a.left, 0);
  const int64_t need_hi = ma::imin64(qa + 15 + a.right, Nr - 1);
  const int64_t band_lo = ma::imax64(m0 - a.left, 0);
  const int64_t band_hi = ma::imin64(m0 + kBandQ - 1 + a.right, Nr - 1);

  float m_run = -INFINITY;  // running max of scaled log2 scores for query qm
  float l_run = 0.0f;       // this lane's share of the softmax denominator
  f32x4 acc[4];             // O^T tiles: head_dim rows 16*dt + 4g + r, query column c
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int64_t s0 = band_lo; s0 <= band_hi; s0 += kBandKC) {
    __syncthreads();  // previous stage fully consumed
    // ---- stage K (row major) : 128 keys x 8 chunks of 16 B
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int idx = tid + 256 * r;
      const int key = idx >> 3, ch = idx & 7;
      const int64_t km = s0 + key;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (km <= band_hi) val = *reinterpret_cast<const uint4*>(K + km * tok_stride + 8 * ch);
      *reinterpret_cast<uint4*>(&ks[key * kKsStride + 8 * ch]) = val;
    }
    // ---- stage V transposed: V^T[d][key]; thread = key pair kp, head_dim chunks dc, dc+4
    {
      const int kp = tid & 63, dc = tid >> 6;
      const int64_t k0 = s0 + 2 * kp, k1 = k0 + 1;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ch = dc + 4 * half;
        uint4 x0 = make_uint4(0, 0, 0, 0), x1 = make_uint4(0, 0, 0, 0);
        if (k0 <= band_hi) x0 = *reinterpret_cast<const uint4*>(V + k0 * tok_stride + 8 * ch);
        if (k1 <= band_hi) x1 = *reinterpret_cast<const uint4*>(V + k1 * tok_stride + 8 * ch);
        const uint32_t w0[4] = {x0.x, x0.y, x0.z, x0.w};
        const uint32_t w1[4] = {x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = (w0[e] & 0xFFFFu) | (w1[e] << 16);
          const uint32_t hi = (w0[e] >> 16) | (w1[e] & 0xFFFF0000u);
          *reinterpret_cast<uint32_t*>(&vt[(8 * ch + 2 * e) * kVtStride + 2 * kp]) = lo;
          *reinterpret_cast<uint32_t*>(&vt[(8 * ch + 2 * e + 1) * kVtStride + 2 * kp]) = hi;
        }
      }
    }
    __syncthreads();
    if (!wave_has_q) continue;

    // ---- S^T = K . Q^T for the 16-key sub-tiles this wave needs
    f32x4 sc[kBandKC / 16];
#pragma unroll
    for (int st = 0; st < kBandKC / 16; ++st) {
      const int64_t k_lo = s0 + 16 * st;
      const bool active = (k_lo <= need_hi) && (k_lo + 15 >= need_lo);
      sc[st] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      if (active) {
        const uint16_t* kr = &ks[(16 * st + c) * kKsStride + 8 * g];
        const uint4 ka0 = *reinterpret_cast<const uint4*>(kr);
        const uint4 ka1 = *reinterpret_cast<const uint4*>(kr + 32);
        f32x4 z = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        z = Mma<T>::x32(ka0, qb0, z);
        z = Mma<T>::x32(ka1, qb1, z);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t km = k_lo + 4 * g + r;
          const bool ok = q_ok && km <= band_hi && ma::in_window(qm, km, a.left, a.right);
          sc[st][r] = ok ? z[r] * a.scale_log2 : -INFINITY;
        }
      }
    }
    // ---- online softmax update (stats per query column; 4 lane groups share a query)
    float mx = -INFINITY;
#pragma unroll
    for (int st = 0; st < kBandKC / 16; ++st)
#pragma unroll
      for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[st][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float corr = __builtin_amdgcn_exp2f(m_run - m_use);
    l_run *= corr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] *= corr;
    m_run = m_new;

    // ---- O^T += V^T . P^T
#pragma unroll
    for (int st = 0; st < kBandKC / 16; ++st) {
      const int64_t k_lo = s0 + 16 * st;
      const bool active = (k_lo <= need_hi) && (k_lo + 15 >= need_lo);
      if (!active) continue;
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = __builtin_amdgcn_exp2f(sc[st][r] - m_use);
        l_run += p[r];
      }
      uint2 pb;
      pb.x = Mma<T>::pack2(p[0], p[1]);
      pb.y = Mma<T>::pack2(p[2], p[3]);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint2 va = *reinterpret_cast<const uint2*>(&vt[(16 * dt + c) * kVtStride + 16 * st + 4 * g]);
        acc[dt] = Mma<T>::x16(va, pb, acc[dt]);
      }
    }
  }

  if (!q_ok) return;
  float l_tot = l_run + __shfl_xor(l_run, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  uint16_t* orow = O + qm * tok_stride;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    uint2 ov;
    ov.x = Mma<T>::pack2(acc[dt][0] * inv, acc[dt][1] * inv);
    ov.y = Mma<T>::pack2(acc[dt][2] * inv, acc[dt][3] * inv);
    *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * g) = ov;
  }
}

// ------------------------------------------------------------------ host side

size_t elt_size(int32_t dt) { return dt == MA_ATTN_F32 ? 4 : 2; }

ma::PatternParams params_of(const ma_attn_desc* d, const int32_t* table) {
  ma::PatternParams p;
  p.n = d->seq_len;
  p.pattern = d->pattern;
  p.causal = d->causal;
  p.left = d->left;
  p.right = d->right;
  p.dilation = d->dilation;
  p.block_size = d->block_size;
  p.table = table;
  p.bpr = d->blocks_per_row;
  p.num_global = d->num_global;
  p.offsets = d->index_offsets;
  p.keys = d->index_keys;
  p.nnz = d->num_indices;
  return p;
}

int validate(const ma_attn_desc* d) {
  if (!d) return fail("ma_attn: null descriptor");
  if (d->batch < 0 || d->seq_len < 0 || d->num_heads < 0 || d->head_dim < 0)
    return fail("ma_attn: negative dimension (B=%lld N=%lld H=%lld D=%lld)", (long long)d->batch,
                (long long)d->seq_len, (long long)d->num_heads, (long long)d->head_dim);
  if (d->dtype != MA_ATTN_F32 && d->dtype != MA_ATTN_BF16 && d->dtype != MA_ATTN_F16)
    return fail("ma_attn: unsupported dtype %d (float32, bfloat16, float16 only)", d->dtype);
  if (d->head_dim > (1LL << 24)) return fail("ma_attn: head_dim %lld above 2^24", (long long)d->head_dim);
  if (d->seq_len > (int64_t)INT32_MAX) return fail("ma_attn: seq_len exceeds int32 range");
  switch (d->pattern) {
    case MA_ATTN_SLIDING:
      if (d->dilation < 1) return fail("ma_attn: dilation must be >= 1 (got %lld)", (long long)d->dilation);
      break;
    case MA_ATTN_DENSE:
      break;
    case MA_ATTN_BLOCK_SPARSE:
      if (d->block_size < 1) return fail("ma_attn: block_size must be >= 1");
      if (d->blocks_per_row < 1 || d->blocks_per_row > 64)
        return fail("ma_attn: blocks_per_row must be in [1, 64]");
      if (!d->block_table && d->seq_len > 0) return fail("ma_attn: block_table is null");
      break;
    case MA_ATTN_LONGFORMER:
      if (d->num_global < 0) return fail("ma_attn: num_global must be >= 0");
      break;
    case MA_ATTN_INDEX_SET:
      if (d->num_indices < 0) return fail("ma_attn: num_indices must be >= 0");
      if (d->tile_header && !d->tile_plan) return fail("ma_attn: tile_header given without tile_plan");
      if (d->tile_header && (d->tile_header->seq_len != d->seq_len || d->tile_header->num_tiles != (d->seq_len + 63) / 64 ||
                             d->tile_header->num_entries < 0 || d->tile_header->num_q_items < (d->seq_len + 63) / 64 ||
                             d->tile_header->num_k_items < (d->seq_len + 63) / 64 || d->tile_header->num_q_partials < 0 ||
                             d->tile_header->num_k_partials < 0 || d->tile_header->num_q_split < 0 ||
                             d->tile_header->num_k_split < 0 || d->tile_header->num_masked < -1 ||
                             d->tile_header->num_masked > d->tile_header->num_entries))
        return fail("ma_attn: the tile plan does not belong to a set of seq_len %lld", (long long)d->seq_len);
      if (!d->index_offsets && d->seq_len > 0) return fail("ma_attn: index_offsets is null");
      if (!d->index_keys && d->num_indices > 0) return fail("ma_attn: index_keys is null");
      break;
    default:
      return fail("ma_attn: unknown pattern %d", d->pattern);
  }
  if (!(d->scale >= 0.0f) || std::isinf(d->scale)) return fail("ma_attn: scale must be finite and >= 0");
  return 0;
}

float scale_of(const ma_attn_desc* d) {
  if (d->scale > 0.0f) return d->scale;
  return 1.0f / std::sqrt(static_cast<float>(d->head_dim));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T>
int launch_rows(const ma_attn_desc* d, const void* q, const void* k, const void* v, void* o,
                hipStream_t st) {
  const int64_t rows = d->batch * d->seq_len * d->num_heads;
  const int64_t blocks = (rows + kRowsWaves - 1) / kRowsWaves;
  if (blocks > (int64_t)INT32_MAX) return fail("ma_attn: problem too large for one launch");
  const size_t shm = sizeof(float) * kRowsWaves * (size_t)d->head_dim;
  const ma::PatternParams pp = params_of(d, d->block_table);
  const float scale = scale_of(d);
  const int dpl = (int)((d->head_dim + 63) / 64);
  const T* tq = static_cast<const T*>(q);
  const T* tk = static_cast<const T*>(k);
  const T* tv = static_cast<const T*>(v);
  T* to = static_cast<T*>(o);
#define MA_ROWS(N_)                                                                            \
  launch(true, rows_kernel<T, N_>, dim3((unsigned)blocks), dim3(256), (uint32_t)shm, st, tq, tk, \
                     tv, to, d->batch, d->num_heads, d->head_dim, pp, scale, (const T*)nullptr, (RowStat*)nullptr)
  if (dpl <= 1)
    MA_ROWS(1);
  else if (dpl <= 2)
    MA_ROWS(2);
  else if (dpl <= 4)
    MA_ROWS(4);
  else if (dpl <= 8)
    MA_ROWS(8);
  else  // head_dim above 512: the query row from memory, output columns in passes of 512
    launch(true, rows_kernel<T, 8, false, true>, dim3((unsigned)blocks), dim3(256), 0u, st, tq, tk, tv, to, d->batch,
           d->num_heads, d->head_dim, pp, scale, (const T*)nullptr, (RowStat*)nullptr);
#undef MA_ROWS
  return 0;
}

// ------------------------------------------------------------------ gather_rows_kernel
//
// Head_dim 64, any key set (explicit index sets, and the patterns the tiled
// kernels do not take), with every gather a whole-row read.  A wave takes 4
// query rows (consecutive positions of one head), 16 lanes each: rows in
// flight hide the dependent offsets ->
// keys -> K -> V round trips, which bound this kernel.  Lane (r =
// (lane>>2)&3, c = lane&3) of a row holds head_dim 16c .. 16c+15 of the
// query.  A 32-key chunk is 8 passes of 4 keys, key 4*pass + r in pass
// `pass`: each pass reads 4 whole K rows per query row and sums the 4 partial
// dots of a key across its lanes; after the chunk's max the same keys' V rows
// go into the lane's 16 accumulators.  The 4 key slots' accumulators are added
// across lanes at the end and lanes with r = 0 write the row.
template <typename T>
__device__ __forceinline__ void unpack8(const T* p, float (&x)[8]) {
  if constexpr (sizeof(T) == 4) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = __uint_as_float(w[e]);
  } else {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = static_cast<float>(__builtin_bit_cast(T, (uint16_t)(w[e] & 0xffffu)));
      x[2 * e + 1] = static_cast<float>(__builtin_bit_cast(T, (uint16_t)(w[e] >> 16)));
    }
  }
}

// STATS (backward): the row's softmax statistics {lse, delta} instead of O,
// as rows_kernel<STATS>.
template <typename T, bool STATS = false>
__global__ __launch_bounds__(256) void gather_rows_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                          const T* __restrict__ v, T* __restrict__ o, int64_t B,
                                                          int64_t H, ma::PatternParams pp, float scale,
                                                          const T* __restrict__ dout = nullptr,
                                                          RowStat* __restrict__ stats = nullptr) {
  constexpr int D = 64;
  constexpr int QPW = 4;  // query rows per wave (16 lanes each)
  constexpr int NP = 8;   // passes per chunk, 4 keys per pass (16: 680 vs 575 us, fewer waves)
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int qs = lane >> 4;        // the lane's query row in the wave
  const int r4 = (lane >> 2) & 3;  // key slot in a pass
  const int c4 = lane & 3;         // head_dim 16*c4 .. 16*c4+15
  const int64_t N = pp.n;
  // A workgroup takes 16 consecutive positions of one (batch, head), so the
  // neighbouring queries' key rows meet in one L1; XCD x takes the x-th
  // eighth of the workgroups, so a head's key rows stay in one L2.
  const int64_t nblk = (N + 15) / 16;
  const int64_t g = xcd_row_order((int)blockIdx.x, (int)gridDim.x);
  const int64_t bh = g / nblk;
  const int64_t i0 = (g % nblk) * 16 + wv * QPW;  // the wave's first position
  if (i0 >= N) return;                             // uniform; no barrier in this kernel
  const int64_t b = bh / H;
  const int64_t h = bh % H;
  const int64_t ip = i0 + qs;
  const bool row_ok = ip < N;
  const int64_t i = row_ok ? ip : i0;
  const int64_t rr = (b * N + i) * H + h;
  const int64_t rs = H * D;  // elements between consecutive tokens

  float qv[16];
  {
    float x[8];
    unpack8(q + rr * D + 16 * c4, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[e] = x[e];
    unpack8(q + rr * D + 16 * c4 + 8, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[8 + e] = x[e];
  }
  const T* kb = k + (b * N * H + h) * D + 16 * c4;
  const T* vb = v + (b * N * H + h) * D + 16 * c4;
  const ma::RowKeys rk = ma::row_keys(pp, i);
  const int64_t cnt = row_ok ? rk.count : 0;
  int64_t cmax = cnt;  // the wave walks as many chunks as its longest row needs
#pragma unroll
  for (int sh = 16; sh <= 32; sh <<= 1) cmax = ma::imax64(cmax, (int64_t)__shfl_xor((long long)cmax, sh, 64));

  float m = -INFINITY, l = 0.0f;
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.0f;

  for (int64_t c0 = 0; c0 < cmax; c0 += 4 * NP) {
    float s[NP];
    int32_t j[NP];
    float mx = -INFINITY;
#pragma unroll
    for (int ps = 0; ps < NP; ++ps) {
      const int64_t t = c0 + 4 * ps + r4;
      const int64_t jk = t < cnt ? ma::key_at(pp, rk, i, t) : -1;
      const bool valid = jk >= 0 && jk < N;  // an index set's keys are checked here
      j[ps] = valid ? (int32_t)jk : -1;
      const T* kr = kb + (valid ? jk : 0) * rs;
      float x[8], dot = 0.0f;
      unpack8(kr, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) dot = fmaf(qv[e], x[e], dot);
      unpack8(kr + 8, x);
#pragma unroll
      for (int e = 0; e < 8; ++e) dot = fmaf(qv[8 + e], x[e], dot);
      dot += __shfl_xor(dot, 1, 64);
      dot += __shfl_xor(dot, 2, 64);
      s[ps] = valid ? dot * scale : -INFINITY;
      mx = fmaxf(mx, s[ps]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 4, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
    // mn is -inf only while every key so far was skipped
    const float mn = fmaxf(m, mx);
    const float mu = mn == -INFINITY ? 0.0f : mn;
    const float corr = expf(m - mu);
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] *= corr;
    float ls = 0.0f;
#pragma unroll
    for (int ps = 0; ps < NP; ++ps) {
      if (j[ps] >= 0) {
        const float p = expf(s[ps] - mu);
        ls += p;
        const T* vr = vb + (int64_t)j[ps] * rs;
        float x[8];
        unpack8(vr, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = fmaf(p, x[e], acc[e]);
        unpack8(vr + 8, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[8 + e] = fmaf(p, x[e], acc[8 + e]);
      }
    }
    ls += __shfl_xor(ls, 4, 64);
    ls += __shfl_xor(ls, 8, 64);
    l = l * corr + ls;
    m = mn;
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    acc[e] += __shfl_xor(acc[e], 4, 64);
    acc[e] += __shfl_xor(acc[e], 8, 64);
  }
  const float inv = cnt > 0 && l != 0.0f ? 1.0f / l : 0.0f;
  if constexpr (STATS) {
    float gv[16], part = 0.0f;
    unpack8(dout + rr * D + 16 * c4, *reinterpret_cast<float(*)[8]>(gv));
    unpack8(dout + rr * D + 16 * c4 + 8, *reinterpret_cast<float(*)[8]>(gv + 8));
#pragma unroll
    for (int e = 0; e < 16; ++e) part = fmaf(gv[e], acc[e] * inv, part);
    part += __shfl_xor(part, 1, 64);
    part += __shfl_xor(part, 2, 64);
    if (row_ok && lane % 16 == 0) stats[rr] = RowStat{cnt > 0 && l > 0.0f ? m + logf(l) : 0.0f, part};
  } else {
    if (row_ok && r4 == 0) {
      T* orow = o + rr * D + 16 * c4;
#pragma unroll
      for (int e = 0; e < 16; ++e) orow[e] = cvt_out<T>(acc[e] * inv);
    }
  }
}

// Backward at head_dim 64 over any key set, with the gather layout of
// gather_rows_kernel (4 rows per wave, 16 lanes per row, 4 partners per pass,
// whole-row reads), given the rows' {lse, delta}:
//   KV = false: row = query i over its keys t:   dq_i = scale * sum_t ds_it k_t
//   KV = true:  row = key j over its queries t:  dk_j = scale * sum_t ds_tj q_t,
//                                                dv_j = sum_t p_tj dO_t
// with p = exp(q.k * scale - lse_query), ds = p * (dO.v - delta_query).  The
// partner rows loaded for the two dot products are the ones accumulated, so
// each partner is read once.
template <typename T, bool KV>
__global__ __launch_bounds__(256) void gather_bwd_kernel(const T* __restrict__ q, const T* __restrict__ k,
                                                         const T* __restrict__ v, const T* __restrict__ dout,
                                                         const RowStat* __restrict__ stats, T* __restrict__ out1,
                                                         T* __restrict__ out2, int64_t B, int64_t H,
                                                         ma::PatternParams pp, float scale) {
  constexpr int D = 64;
  constexpr int QPW = 4;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int qs = lane >> 4;
  const int r4 = (lane >> 2) & 3;
  const int c4 = lane & 3;
  const int64_t N = pp.n;
  const int64_t nblk = (N + 15) / 16;
  const int64_t g = xcd_row_order((int)blockIdx.x, (int)gridDim.x);
  const int64_t bh = g / nblk;
  const int64_t i0 = (g % nblk) * 16 + wv * QPW;
  if (i0 >= N) return;  // uniform; no barrier in this kernel
  const int64_t b = bh / H;
  const int64_t h = bh % H;
  const int64_t ip = i0 + qs;
  const bool row_ok = ip < N;
  const int64_t i = row_ok ? ip : i0;
  const int64_t rr = (b * N + i) * H + h;
  const int64_t rs = H * D;
  const int64_t sbase = b * N * H + h;  // stats index of position 0 of this (batch, head)

  // own rows: (q_i, dO_i) for dq, (k_j, v_j) for dk/dv; partners the other pair
  float av[16], bv[16];
  {
    const T* A = (KV ? k : q) + rr * D + 16 * c4;
    const T* Bp = (KV ? v : dout) + rr * D + 16 * c4;
    unpack8(A, *reinterpret_cast<float(*)[8]>(av));
    unpack8(A + 8, *reinterpret_cast<float(*)[8]>(av + 8));
    unpack8(Bp, *reinterpret_cast<float(*)[8]>(bv));
    unpack8(Bp + 8, *reinterpret_cast<float(*)[8]>(bv + 8));
  }
  const T* xb = (KV ? q : k) + (b * N * H + h) * D + 16 * c4;
  const T* yb = (KV ? dout : v) + (b * N * H + h) * D + 16 * c4;
  RowStat own = RowStat{0.0f, 0.0f};
  if (!KV) own = stats[rr];
  const ma::RowKeys rk = ma::row_keys(pp, i);
  const int64_t cnt = row_ok ? rk.count : 0;
  int64_t cmax = cnt;
#pragma unroll
  for (int sh = 16; sh <= 32; sh <<= 1) cmax = ma::imax64(cmax, (int64_t)__shfl_xor((long long)cmax, sh, 64));

  float acc1[16], acc2[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc1[e] = acc2[e] = 0.0f;
  for (int64_t c0 = 0; c0 < cmax; c0 += 4) {
    const int64_t t = c0 + r4;
    const int64_t jk = t < cnt ? ma::key_at(pp, rk, i, t) : -1;
    const bool valid = jk >= 0 && jk < N;  // an index set's entries are checked here
    const int64_t pr = valid ? jk : 0;
    float x[16], y[16];
    unpack8(xb + pr * rs, *reinterpret_cast<float(*)[8]>(x));
    unpack8(xb + pr * rs + 8, *reinterpret_cast<float(*)[8]>(x + 8));
    unpack8(yb + pr * rs, *reinterpret_cast<float(*)[8]>(y));
    unpack8(yb + pr * rs + 8, *reinterpret_cast<float(*)[8]>(y + 8));
    float sd = 0.0f, pd = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      sd = fmaf(av[e], x[e], sd);
      pd = fmaf(bv[e], y[e], pd);
    }
    sd += __shfl_xor(sd, 1, 64);
    sd += __shfl_xor(sd, 2, 64);
    pd += __shfl_xor(pd, 1, 64);
    pd += __shfl_xor(pd, 2, 64);
    const RowStat st = KV ? stats[sbase + pr * H] : own;
    const float p = valid ? expf(sd * scale - st.lse) : 0.0f;
    const float ds = p * (pd - st.delta);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      acc1[e] = fmaf(ds, x[e], acc1[e]);
      if (KV) acc2[e] = fmaf(p, y[e], acc2[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    acc1[e] += __shfl_xor(acc1[e], 4, 64);
    acc1[e] += __shfl_xor(acc1[e], 8, 64);
    if (KV) {
      acc2[e] += __shfl_xor(acc2[e], 4, 64);
      acc2[e] += __shfl_xor(acc2[e], 8, 64);
    }
  }
  if (row_ok && r4 == 0) {
    T* o1 = out1 + rr * D + 16 * c4;
#pragma unroll
    for (int e = 0; e < 16; ++e) o1[e] = cvt_out<T>(acc1[e] * scale);
    if (KV) {
      T* o2 = out2 + rr * D + 16 * c4;
#pragma unroll
      for (int e = 0; e < 16; ++e) o2[e] = cvt_out<T>(acc2[e]);
    }
  }
}

bool gather_applies(const ma_attn_desc* d, const void* q, const void* k, const void* v, const void* o) {
  return d->head_dim == 64 && aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o);
}

template <typename T>
int launch_gather(const ma_attn_desc* d, const void* q, const void* k, const void* v, void* o, hipStream_t st) {
  // one workgroup per 16 positions of one (batch, head): 4 waves of 4 rows
  const int64_t blocks = d->batch * d->num_heads * ((d->seq_len + 15) / 16);
  if (blocks > (int64_t)INT32_MAX) return fail("ma_attn: problem too large for one launch");
  launch(true, gather_rows_kernel<T>, dim3((unsigned)blocks), dim3(256), 0u, st, static_cast<const T*>(q),
         static_cast<const T*>(k), static_cast<const T*>(v), static_cast<T*>(o), d->batch, d->num_heads,
         params_of(d, d->block_table), scale_of(d), (const T*)nullptr, (RowStat*)nullptr);
  return 0;
}

// Narrow heads on the one-query-per-lane kernel (band rows staged in LDS).
constexpr int64_t kNarrowLds = 64 * 1024;

int64_t narrow_lds(const ma_attn_desc* d) {
  const int64_t dp = d->head_dim <= 16 ? 16 : 32;
  const int64_t rows = ma::imin64(64 + d->left + d->right, d->seq_len);
  return (2 * rows * (dp + 4) + (kNarrowWaves - 1) * 64 * (dp + 2)) * 4;
}

bool narrow_applies(const ma_attn_desc* d) {
  if (d->pattern != MA_ATTN_SLIDING || d->dilation != 1 || d->left < 0 || d->right < 0) return false;
  if (d->head_dim < 1 || d->head_dim > 32 || d->left + d->right > (1 << 16)) return false;
  const int64_t tiles = (d->seq_len + 63) / 64;
  return narrow_lds(d) <= kNarrowLds && d->batch * d->num_heads * tiles <= (int64_t)INT32_MAX;
}

template <typename T>
int launch_narrow(const ma_attn_desc* d, const void* q, const void* k, const void* v, void* o, hipStream_t st) {
  const int64_t tiles = (d->seq_len + 63) / 64;
  const float scale = scale_of(d);
  const dim3 grid((unsigned)(d->batch * d->num_heads * tiles)), blk(64 * kNarrowWaves);
  const uint32_t shm = (uint32_t)narrow_lds(d);
  const T* tq = static_cast<const T*>(q);
  const T* tk = static_cast<const T*>(k);
  const T* tv = static_cast<const T*>(v);
  T* to = static_cast<T*>(o);
  const int D = (int)d->head_dim, L = (int)d->left, R = (int)d->right;
  if (D <= 16)
    launch(true, narrow_kernel<T, 16>, grid, blk, shm, st, tq, tk, tv, to, d->seq_len, d->num_heads, D, L, R, scale);
  else
    launch(true, narrow_kernel<T, 32>, grid, blk, shm, st, tq, tk, tv, to, d->seq_len, d->num_heads, D, L, R, scale);
  return 0;
}

bool band_applies(const ma_attn_desc* d, const void* q, const void* k, const void* v, const void* o) {
  return d->pattern == MA_ATTN_SLIDING && (d->dtype == MA_ATTN_BF16 || d->dtype == MA_ATTN_F16) &&
         d->head_dim == kBandD && d->left >= 0 && d->right >= 0 && aligned16(q) && aligned16(k) &&
         aligned16(v) && aligned16(o);
}

int launch_band(const ma_attn_desc* d, const void* q, const void* k, const void* v, void* o,
                hipStream_t st) {
  BandArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.B = d->batch;
  a.N = d->seq_len;
  a.H = d->num_heads;
  a.left = d->left;
  a.right = d->right;
  a.dil = d->dilation;
  const int64_t nr_max = (d->seq_len + d->dilation - 1) / d->dilation;
  a.tiles = (nr_max + kBandQ - 1) / kBandQ;
  a.scale_log2 = scale_of(d) * 1.4426950408889634f;
  const int64_t wgs = d->batch * a.tiles * d->num_heads * d->dilation;
  if (wgs > (int64_t)INT32_MAX) return fail("ma_attn: problem too large for one launch");
  if (d->dtype == MA_ATTN_BF16)
    launch(true, band_kernel<__bf16>, dim3((unsigned)wgs), dim3(256), 0, st, a);
  else
    launch(true, band_kernel<_Float16>, dim3((unsigned)wgs), dim3(256), 0, st, a);
  return 0;
}

// Ring blocks a tile touches: floor((63+R)/64) - floor(-L/64) + 1.
constexpr int kMaxSlots = 6;  // generic instantiations (16-bit: 108 KB, fp32: 102 KB of LDS)
constexpr int kStreamSG = 5;  // sub-tiles per softmax group (a causal-64 wave tile needs 5)

// The banded problem a descriptor maps to on the stream kernel: window
// [i-left, i+right] on residue classes of `dil`, plus G global tokens
// (Longformer, dilation 1).
struct StreamGeom {
  int64_t left, right, dil, G;
};

bool stream_geom(const ma_attn_desc* d, StreamGeom* g) {
  if (d->pattern == MA_ATTN_SLIDING) {
    *g = StreamGeom{d->left, d->right, d->dilation, 0};
    return true;
  }
  if (d->pattern == MA_ATTN_LONGFORMER) {
    *g = StreamGeom{d->left, d->right, 1, ma::imin64(d->num_global, d->seq_len)};
    return true;
  }
  return false;
}

// Work split of the stream kernel: `chunk` consecutive tiles per workgroup,
// enough workgroups to give every CU as many as its LDS holds.
struct StreamPlan {
  StreamGeom geom;
  int64_t rows, slot_bytes, max_per_cu, slots, lds, tiles, chunk, chunks, wgs, tok_bytes, partial_bytes;
};

StreamPlan stream_plan(const ma_attn_desc* d) {
  StreamPlan p;
  stream_geom(d, &p.geom);
  const bool f32 = d->dtype == MA_ATTN_F32;
  const bool lg = p.geom.G > 0;
  p.rows = f32 ? F32Path::kRows : HalfPath<__bf16>::kRows;
  p.slot_bytes = f32 ? F32Path::kSlot : HalfPath<__bf16>::kSlot;
  p.max_per_cu = f32 ? F32Path::kMinBlocks : HalfPath<__bf16>::kMinBlocks;
  p.slots = ma::floordiv64(63 + p.geom.right, p.rows) - ma::floordiv64(-p.geom.left, p.rows) + 1;
  p.lds = (p.slots + (lg ? 1 : 0)) * p.slot_bytes;
  const int64_t nr_max = (d->seq_len + p.geom.dil - 1) / p.geom.dil;
  p.tiles = (nr_max + 63) / 64;
  const int64_t streams = d->batch * d->num_heads * p.geom.dil;
  int64_t per_cu = ma::imax64(1, ma::imin64(p.max_per_cu, (160 * 1024) / p.lds));
  // A window with a right halo reads a halo block at both ends of a chunk.
  // For 16-bit tiles (light compute) one chunk twice as long per CU pays
  // that halo half as often and measured faster than two per CU (cfg2 bf16:
  // 35.0 -> 32.5 us); fp32 tiles need the second workgroup to hide their
  // MFMA latency (cfg2 fp32: 72 vs 82 us).
  if (!f32 && !lg && p.geom.right > 0) per_cu = 1;
  const int64_t slots = 256 * per_cu;  // resident workgroups
  // Workgroups per stream: as many as fit the resident slots in one wave
  // (rounded per stream, a grid that overflows the slots by a few
  // workgroups runs them alone afterwards: cfg4 with 24 streams took 2x).
  // Even where the paired chunk order applies.
  int64_t per_stream = ma::imax64(1, slots / streams);
  if ((p.geom.right > 0 || lg) && per_stream > 1) per_stream &= ~1LL;
  p.chunk = ma::imax64(1, (p.tiles + per_stream - 1) / per_stream);
  p.chunks = (p.tiles + p.chunk - 1) / p.chunk;
  p.wgs = streams * p.chunks;
  p.tok_bytes = p.geom.dil * d->num_heads * kHeadDim * (f32 ? 4 : 2);
  p.partial_bytes = lg ? streams * p.chunks * 16 * kPartial * (int64_t)sizeof(float) : 0;
  return p;
}

constexpr int kMaxGlobal = 16;  // Longformer global tokens handled by the stream kernel

bool stream_applies(const ma_attn_desc* d, const void* q, const void* k, const void* v, const void* o) {
  StreamGeom g;
  if (!stream_geom(d, &g) || d->head_dim != kHeadDim || g.left < 0 || g.right < 0) return false;
  if (g.G > kMaxGlobal) return false;
  if (!(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o))) return false;
  if (g.left > (1 << 20) || g.right > (1 << 20)) return false;
  const StreamPlan p = stream_plan(d);
  if (p.slots < 1 || p.slots > kMaxSlots || p.lds > 160 * 1024) return false;
  if (p.wgs > (int64_t)INT32_MAX || p.tiles > (1 << 24)) return false;
  // Every buffer offset a workgroup forms is below
  // (chunk*64 + left + right + 256 + rows*slots) rows past its first row
  // (Longformer: past row 0).
  const int64_t rows = (g.G > 0 ? d->seq_len : p.chunk * 64) + g.left + g.right + 256 + p.rows * p.slots;
  return p.tok_bytes < (1LL << 24) && rows * p.tok_bytes + 256 < (1LL << 31);
}

template <class P, int NSLOT, int FL, int FR, bool LG, bool DM>
int launch_stream_t(const StreamArgs& a, int64_t wgs, hipStream_t st) {
  const size_t shm = (size_t)(NSLOT + (LG ? 1 : 0)) * P::kSlot;
  auto kern = &stream_kernel<P, NSLOT, kStreamSG, FL, FR, LG, DM>;
  if (reserve_lds(reinterpret_cast<const void*>(kern), shm, st)) return 1;
  launch(!LG, kern, dim3((unsigned)wgs), dim3(256), (uint32_t)shm, st, a);  // Longformer: combine is last
  return 0;
}

// Fixed-window instantiations (the benchmark windows: causal 64, [i-32, i+31],
// Longformer causal 128); other windows run the
// generic kernel with `slots` ring slots.
template <class P, bool LG, bool DM>
int launch_stream_any(const StreamArgs& a, int64_t slots, int64_t wgs, hipStream_t st) {
  constexpr int RS = P::kRows;
  if (!g_opt.no_fixed) {
    if constexpr (!LG) {
      if (a.left == 63 && a.right == 0) return launch_stream_t<P, WinGeom<63, 0, RS>::NSLOT, 63, 0, LG, DM>(a, wgs, st);
      if (a.left == 32 && a.right == 31)
        return launch_stream_t<P, WinGeom<32, 31, RS>::NSLOT, 32, 31, LG, DM>(a, wgs, st);
    } else {
      if (a.left == 127 && a.right == 0)
        return launch_stream_t<P, WinGeom<127, 0, RS>::NSLOT, 127, 0, LG, DM>(a, wgs, st);
    }
  }
  switch (slots) {
    case 1: return launch_stream_t<P, 1, -1, -1, LG, DM>(a, wgs, st);
    case 2: return launch_stream_t<P, 2, -1, -1, LG, DM>(a, wgs, st);
    case 3: return launch_stream_t<P, 3, -1, -1, LG, DM>(a, wgs, st);
    case 4: return launch_stream_t<P, 4, -1, -1, LG, DM>(a, wgs, st);
    case 5: return launch_stream_t<P, 5, -1, -1, LG, DM>(a, wgs, st);
    default: return launch_stream_t<P, 6, -1, -1, LG, DM>(a, wgs, st);
  }
}

template <typename T>
int launch_stream_half(const ma_attn_desc* d, const StreamArgs& a, const StreamPlan& p, hipStream_t st) {
  using P = HalfPath<T>;
  if (p.geom.G == 0) return launch_stream_any<P, false, false>(a, p.slots, p.wgs, st);
  // delta mode is its own instantiation: as a runtime flag its dO loads and
  // sums cost the plain forward registers (177 -> 203 VGPRs, SGPR spills)
  // and ~3 % time
  const int rc = a.delta ? launch_stream_any<P, true, true>(a, p.slots, p.wgs, st)
                         : launch_stream_any<P, true, false>(a, p.slots, p.wgs, st);
  if (rc) return rc;
  launch(true, longformer_combine<T>, dim3((unsigned)(d->batch * d->num_heads * p.geom.G)), dim3(256), 0, st,
                     a.partials, static_cast<T*>(a.o), (int)p.chunks, (int)p.geom.G, (int)d->num_heads,
                     d->seq_len, a.lse, a.delta);
  return 0;
}

// fp32: the sliding windows, and Longformer (no delta mode: the one-pass
// backward is 16-bit) with its combine.
int launch_stream_f32(const ma_attn_desc* d, const StreamArgs& a, const StreamPlan& p, hipStream_t st) {
  if (p.geom.G == 0) return launch_stream_any<F32Path, false, false>(a, p.slots, p.wgs, st);
  if (a.delta) return fail("ma_attn: the Longformer delta-mode forward is 16-bit only");
  const int rc = launch_stream_any<F32Path, true, false>(a, p.slots, p.wgs, st);
  if (rc) return rc;
  launch(true, longformer_combine<float>, dim3((unsigned)(d->batch * d->num_heads * p.geom.G)), dim3(256), 0, st,
         a.partials, static_cast<float*>(a.o), (int)p.chunks, (int)p.geom.G, (int)d->num_heads, d->seq_len,
         a.lse, a.delta);
  return 0;
}

// dout, delta (Longformer only): delta mode, each row's
// delta = sum_j P_ij dP_ij (dP_ij = dO_i . V_j, fp32) into delta alongside
// lse, and O not written.
int launch_stream(const ma_attn_desc* d, const void* q, const void* k, const void* v, void* o, float* lse,
                  void* ws, size_t ws_bytes, hipStream_t st, const void* dout = nullptr, float* delta = nullptr) {
  const StreamPlan p = stream_plan(d);
  if ((int64_t)ws_bytes < p.partial_bytes || (p.partial_bytes > 0 && !ws))
    return fail("ma_attn: workspace of %lld bytes required (ma_attn_workspace_size), got %zu",
                (long long)p.partial_bytes, ws_bytes);
  StreamArgs a{};
  a.dout = dout;
  a.delta = delta;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.N = d->seq_len;
  a.H = d->num_heads;
  a.left = (int32_t)p.geom.left;
  a.right = (int32_t)p.geom.right;
  a.dil = (int32_t)p.geom.dil;
  a.tiles = (int32_t)p.tiles;
  a.chunk = (int32_t)p.chunk;
  a.chunks = (int32_t)p.chunks;
  a.tok_bytes = (int32_t)p.tok_bytes;
  a.scale_log2 = scale_of(d) * 1.4426950408889634f;
  a.num_global = (int32_t)p.geom.G;
  a.partials = static_cast<float*>(ws);
  a.lse = lse;  // Longformer only (forward_launch refuses it elsewhere)
  // Chunk pairs on one XCD (neighbours' shared halo block read at the same
  // moment into one L2): measured faster with a right halo (cfg2 bf16 37.5 ->
  // 36.8 us) and for Longformer (cfg4 184 -> 179 us); neutral on causal
  // windows (target fetch -3.6 %, time unchanged), which keep the plain order.
  const bool pairs_help = p.geom.right > 0 || p.geom.G > 0;
  a.pairs = pairs_help && p.wgs % 16 == 0 && p.chunks % 2 == 0 ? 1 : 0;
  switch (d->dtype) {
    case MA_ATTN_BF16: return launch_stream_half<__bf16>(d, a, p, st);
    case MA_ATTN_F16: return launch_stream_half<_Float16>(d, a, p, st);
    default: return launch_stream_f32(d, a, p, st);
  }
}

// Block-sparse on MFMA: block size 64, head_dim 64, 16-bit.  Dense (and
// causal) attention takes the same kernel with every block (blocks 0..r).
bool block_applies(const ma_attn_desc* d, const void* q, const void* k, const void* v, const void* o) {
  const bool blocks = d->pattern == MA_ATTN_BLOCK_SPARSE && d->block_size == 64;
  if (!(blocks || d->pattern == MA_ATTN_DENSE) || d->head_dim != kHeadDim) return false;
  if (!(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o))) return false;
  const int64_t tb = d->num_heads * kHeadDim * (d->dtype == MA_ATTN_F32 ? 4 : 2);
  const int64_t nbq = (d->seq_len + 63) / 64;
  return (d->seq_len + 128) * tb < (1LL << 31) && d->batch * d->num_heads * nbq <= (int64_t)INT32_MAX;
}

template <class P>
int launch_block_t(const BlockArgs& a, int64_t bh, hipStream_t st) {
  constexpr size_t shm = 2 * (size_t)P::kBlk;  // two block buffers (fp32: 68 KB)
  if (reserve_lds(reinterpret_cast<const void*>(&block_row_kernel<P>), shm, st)) return 1;
  launch(true, block_row_kernel<P>, dim3((unsigned)(bh * a.nbq)), dim3(256), (uint32_t)shm, st, a);
  return 0;
}

int launch_block(const ma_attn_desc* d, const void* q, const void* k, const void* v, void* o, float* lse,
                 hipStream_t st) {
  BlockArgs a;
  a.lse = lse;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  const bool dense = d->pattern == MA_ATTN_DENSE;
  a.table = dense ? nullptr : d->block_table;
  a.causal = dense && d->causal;
  a.N = (int32_t)d->seq_len;
  a.H = (int32_t)d->num_heads;
  a.bpr = dense ? 0 : (int32_t)d->blocks_per_row;
  a.nbq = (int32_t)((d->seq_len + 63) / 64);
  a.scale_log2 = scale_of(d) * 1.4426950408889634f;
  const int64_t bh = d->batch * d->num_heads;
  if (d->dtype == MA_ATTN_BF16) return launch_block_t<HalfPath<__bf16>>(a, bh, st);
  if (d->dtype == MA_ATTN_F16) return launch_block_t<HalfPath<_Float16>>(a, bh, st);
  return launch_block_t<F32Path>(a, bh, st);
}

// Backward: SLIDING and DENSE key sets (the reference's backward entry
// points), any dtype, head_dim <= 512.
bool backward_supported(const ma_attn_desc* d) {
  return d->pattern == MA_ATTN_SLIDING || d->pattern == MA_ATTN_DENSE || d->pattern == MA_ATTN_INDEX_SET ||
         d->pattern == MA_ATTN_LONGFORMER;
}

// The query sets T_j = {i : j in S_i}: a SLIDING pattern for the banded
// sets, the caller's transposed CSR for an index set.
ma::PatternParams transposed_params(const ma_attn_desc* d) {
  ma::PatternParams p = params_of(d, nullptr);
  if (d->pattern == MA_ATTN_INDEX_SET) {
    p.offsets = d->index_t_offsets;
    p.keys = d->index_t_queries;
    return p;
  }
  if (d->pattern == MA_ATTN_DENSE) {
    p.pattern = ma::kSliding;
    p.dilation = 1;
    p.left = d->causal ? 0 : d->seq_len - 1;  // i = j + t, t in [-left, right]
    p.right = d->seq_len - 1;
  } else {
    p.left = d->right;
    p.right = d->left;
  }
  p.causal = 0;
  return p;
}

// MFMA backward: 16-bit, head_dim 64, 16-byte aligned tensors, banded sets
// whose band holds the query's own key (SLIDING with left, right >= 0;
// DENSE as the band [i-(N-1), i] or [i-(N-1), i+(N-1)]).
bool bwd_band(const ma_attn_desc* d, int64_t* left, int64_t* right, int64_t* dil) {
  if (d->pattern == MA_ATTN_DENSE) {
    *left = d->seq_len - 1;
    *right = d->causal ? 0 : d->seq_len - 1;
    *dil = 1;
    return true;
  }
  if (d->pattern != MA_ATTN_SLIDING || d->left < 0 || d->right < 0) return false;
  *left = d->left;
  *right = d->right;
  *dil = d->dilation;
  return true;
}

bool bwd_mfma_applies(const ma_attn_desc* d, const void* const* ptrs) {
  if (d->head_dim != kHeadDim) return false;
  for (int i = 0; i < 7; ++i)
    if (!aligned16(ptrs[i])) return false;
  int64_t L, R, dil;
  if (!bwd_band(d, &L, &R, &dil)) return false;
  const int64_t tb = dil * d->num_heads * kHeadDim * (d->dtype == MA_ATTN_F32 ? 4 : 2);
  const int64_t nr = (d->seq_len + dil - 1) / dil;
  const int64_t tiles = (nr + 63) / 64;
  // byte offsets of rows (plus the out-of-range base) fit 32 bits; ids fit the grid
  return (nr + 128) * tb < (1LL << 31) && nr * dil * d->num_heads * 8 < (1LL << 31) && L + R < (1LL << 30) &&
         d->batch * d->num_heads * dil * tiles <= (int64_t)INT32_MAX;
}

// The fused backward's chunks of a stream's tiles, fitted to one round of the
// resident workgroups (two per CU).
void fused_chunks(BwdArgs& a, int64_t streams) {
  const int64_t per_stream = ma::imax64(1, 256 * 2 / streams);
  a.chunk = (int32_t)ma::imax64(1, (a.tiles + per_stream - 1) / per_stream);
  a.chunks = (int32_t)((a.tiles + a.chunk - 1) / a.chunk);
}

// fo, lse: the forward's O and statistics (ma_attn_backward_saved), or null.
// Only the one-tile-per-workgroup dQ kernel (bands wider than two blocks:
// dense, causal) takes them: the stream and fused kernels keep a tile's
// scores in registers between their statistics and their dQ.
template <class P>
int launch_backward_mfma(const ma_attn_desc* d, const void* const* ptrs, float* stats, hipStream_t st,
                         const void* fo = nullptr, const float* lse = nullptr) {
  int64_t L, R, dil;
  bwd_band(d, &L, &R, &dil);
  BwdArgs a;
  a.fo = fo;
  a.lse = lse;
  a.q = ptrs[0];
  a.k = ptrs[1];
  a.v = ptrs[2];
  a.dout = ptrs[3];
  a.dq = const_cast<void*>(ptrs[4]);
  a.dk = const_cast<void*>(ptrs[5]);
  a.dv = const_cast<void*>(ptrs[6]);
  a.stats = stats;
  a.N = d->seq_len;
  a.H = d->num_heads;
  a.left = (int32_t)L;
  a.right = (int32_t)R;
  a.dil = (int32_t)dil;
  const int64_t nr = (d->seq_len + dil - 1) / dil;
  a.tiles = (int32_t)((nr + 63) / 64);
  a.tok_bytes = (int32_t)(dil * d->num_heads * kHeadDim * sizeof(typename P::Elt));
  a.scale = scale_of(d);
  a.scale_log2 = a.scale * 1.4426950408889634f;
  const int64_t streams = d->batch * d->num_heads * dil;
  // two block buffers each: K, V for dQ; Q, dO + statistics for dK/dV (PairLds: rows only on
  // the 16-bit path, fp32 with the staged transposes)
  const size_t shm_q = 2 * (size_t)PairLds<P>::kBytes, shm_kv = 2 * ((size_t)PairLds<P>::kBytes + 512);
  // Bands that meet at most two 64-row blocks in both directions stream a
  // chunk of tiles per workgroup; wider bands take one workgroup per tile.
  // The stream kernels' blocks start at row -16*(ceil(L/16) & 3) (keys) and
  // -16*(ceil(R/16) & 3) (queries), which fits [i-32, i+31] in two.
  const int64_t obq = -16 * (((L + 15) / 16) & 3), obkv = -16 * (((R + 15) / 16) & 3);
  const bool chunked = ma::floordiv64(63 + R - obq, 64) - ma::floordiv64(-L - obq, 64) + 1 <= 2 &&
                       ma::floordiv64(63 + L - obkv, 64) - ma::floordiv64(-R - obkv, 64) + 1 <= 2;
  // fixed-window instantiations: causal 64 (also per residue class of a dilated window)
  // and [i-32, i+31] (cfg 2)
  const bool no_fixed = g_opt.bwd_no_fixed;
  const int fixed = !chunked || no_fixed ? 0 : L == 63 && R == 0 ? 1 : L == 32 && R == 31 ? 2 : 0;
  if constexpr (P::kSPB == 1) {
    if (fixed != 0 && !g_opt.bwd_unfused) {
      // the fixed windows in 16 bits: one fused launch (bwd_fused_kernel.h),
      // 80 KB of LDS, two workgroups per CU; chunks fitted to one round of
      // the resident workgroups (measured on the target: one round, chunk 16,
      // 10-15 % faster than two to six rounds)
      const size_t shm = (size_t)FusedLds::kBytes;
      fused_chunks(a, streams);
      auto kf = fixed == 1 ? &bwd_fused_kernel<P, 63, 0> : &bwd_fused_kernel<P, 32, 31>;
      if (reserve_lds(reinterpret_cast<const void*>(kf), shm, st)) return 1;
      launch(true, kf, dim3((unsigned)(streams * a.chunks)), dim3(256), (uint32_t)shm, st, a);
      return 0;
    }
  }
  auto kq = !chunked     ? (lse ? &bwd_q_kernel<P, true> : &bwd_q_kernel<P, false>)
            : fixed == 1 ? &bwd_q_stream_kernel<P, 63, 0>
            : fixed == 2 ? &bwd_q_stream_kernel<P, 32, 31>
                         : &bwd_q_stream_kernel<P, -1, -1>;
  auto kkv = !chunked     ? &bwd_kv_kernel<P>
             : fixed == 1 ? &bwd_kv_stream_kernel<P, 63, 0>
             : fixed == 2 ? &bwd_kv_stream_kernel<P, 32, 31>
                          : &bwd_kv_stream_kernel<P, -1, -1>;
  // chunks per stream fitted to two rounds of the resident workgroups (2 per
  // CU for 16-bit, 1 for fp32, whose block buffers are twice the size): the
  // second round fills the slots the first round's faster workgroups leave.
  // Measured on the target: 171 us at two rounds (chunk 8), 178 us at one
  // (chunk 16), 178-186 us at three or more.
  const int64_t per_cu = ma::imax64(1, ma::imin64(2, (int64_t)(160 * 1024) / (int64_t)ma::imax64(shm_q, shm_kv)));
  const int64_t per_stream = ma::imax64(1, 2 * 256 * per_cu / streams);
  a.chunk = (int32_t)ma::imax64(1, (a.tiles + per_stream - 1) / per_stream);
  a.chunks = (int32_t)((a.tiles + a.chunk - 1) / a.chunk);
  const int64_t wgs = chunked ? streams * a.chunks : streams * a.tiles;
  if (reserve_lds(reinterpret_cast<const void*>(kq), shm_q, st) ||
      reserve_lds(reinterpret_cast<const void*>(kkv), shm_kv, st))
    return 1;
  launch(false, kq, dim3((unsigned)wgs), dim3(256), (uint32_t)shm_q, st, a);
  launch(true, kkv, dim3((unsigned)wgs), dim3(256), (uint32_t)shm_kv, st, a);
  return 0;
}

template <typename T>
int launch_backward(const ma_attn_desc* d, const void* q, const void* k, const void* v, const void* dout,
                    void* dq, void* dk, void* dv, RowStat* stats, hipStream_t st) {
  const int64_t rows = d->batch * d->seq_len * d->num_heads;
  const int64_t blocks = (rows + kRowsWaves - 1) / kRowsWaves;
  if (blocks > (int64_t)INT32_MAX) return fail("ma_attn: problem too large for one launch");
  const ma::PatternParams pp = params_of(d, nullptr);
  const ma::PatternParams pt = transposed_params(d);
  const float scale = scale_of(d);
  const int dpl = (int)((d->head_dim + 63) / 64);
  const size_t shm1 = sizeof(float) * kRowsWaves * (size_t)d->head_dim;
  const size_t shm2 = 2 * shm1;
  const T* tq = static_cast<const T*>(q);
  const T* tk = static_cast<const T*>(k);
  const T* tv = static_cast<const T*>(v);
  const T* tg = static_cast<const T*>(dout);
  const dim3 grid((unsigned)blocks), blk(256);
  const int64_t B = d->batch, H = d->num_heads, D = d->head_dim;
  if (D == 64 && !g_opt.force_rows && aligned16(q) && aligned16(k) && aligned16(v) &&
      aligned16(dout) && aligned16(dq) && aligned16(dk) && aligned16(dv)) {
    // head_dim 64: the gather layout (whole-row reads, 4 rows per wave)
    const int64_t gblocks = B * H * ((d->seq_len + 15) / 16);
    if (gblocks > (int64_t)INT32_MAX) return fail("ma_attn: problem too large for one launch");
    const dim3 gg((unsigned)gblocks);
    launch(false, gather_rows_kernel<T, true>, gg, blk, 0u, st, tq, tk, tv, (T*)nullptr, B, H, pp, scale, tg,
           stats);
    launch(false, gather_bwd_kernel<T, false>, gg, blk, 0u, st, tq, tk, tv, tg, (const RowStat*)stats,
           static_cast<T*>(dq), (T*)nullptr, B, H, pp, scale);
    launch(true, gather_bwd_kernel<T, true>, gg, blk, 0u, st, tq, tk, tv, tg, (const RowStat*)stats,
           static_cast<T*>(dk), static_cast<T*>(dv), B, H, pt, scale);
    return 0;
  }
#define MA_BWD(N_)                                                                                          \
  do {                                                                                                      \
    launch(false, rows_kernel<T, N_, true>, grid, blk, (uint32_t)shm1, st, tq, tk, tv, (T*)nullptr, B, H, D, pp, \
                       scale, tg, stats);                                                                   \
    launch(false, bwd_dq_kernel<T, N_>, grid, blk, (uint32_t)shm2, st, tq, tk, tv, tg, (const RowStat*)stats,  \
                       static_cast<T*>(dq), B, H, D, pp, scale);                                            \
    launch(true, bwd_dkv_kernel<T, N_>, grid, blk, (uint32_t)shm2, st, tq, tk, tv, tg, (const RowStat*)stats, \
                       static_cast<T*>(dk), static_cast<T*>(dv), B, H, D, pt, scale);                       \
  } while (0)
  if (dpl <= 1)
    MA_BWD(1);
  else if (dpl <= 2)
    MA_BWD(2);
  else if (dpl <= 4)
    MA_BWD(4);
  else if (dpl <= 8)
    MA_BWD(8);
  else {  // head_dim above 512: rows from memory, columns in passes of 512
    launch(false, rows_kernel<T, 8, true, true>, grid, blk, 0u, st, tq, tk, tv, (T*)nullptr, B, H, D, pp, scale, tg,
           stats);
    launch(false, bwd_dq_kernel<T, 8, true>, grid, blk, 0u, st, tq, tk, tv, tg, (const RowStat*)stats,
           static_cast<T*>(dq), B, H, D, pp, scale);
    launch(true, bwd_dkv_kernel<T, 8, true>, grid, blk, 0u, st, tq, tk, tv, tg, (const RowStat*)stats,
           static_cast<T*>(dk), static_cast<T*>(dv), B, H, D, pt, scale);
  }
#undef MA_BWD
  return 0;
}

// Device address of `scratch` on the stream's device, looked up once per
// device with that device current.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the stream's device.  Only a successful
// lookup is kept: after a failure (hipSetDevice, hipGetSymbolAddress) the next
// call looks it up again.
int scratch_of_stream(hipStream_t st, void** out) {
  int dev = 0;
  if (stream_device(st, &dev)) return 1;
  if (dev < 0 || dev >= kMaxDevices) return fail("ma_attn: device %d out of range", dev);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      int cur = 0;
      hipError_t e = hipGetDevice(&cur);
      if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
      if (e == hipSuccess) e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (cur != dev) (void)hipSetDevice(cur);
      if (e != hipSuccess || !ptr)
        return fail("ma_attn: cannot locate the static scratch on device %d: %s", dev,
                    hipGetErrorString(e != hipSuccess ? e : hipErrorInvalidSymbol));
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return 0;
}

int forward_launch(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o, float* lse,
                   void* workspace, size_t workspace_bytes, hipStream_t st);

// ------------------------------------------------------------------ Longformer backward from saved statistics
//
// bwd_longformer_kernel.h: one pass over Q, K, V, dO and O for Longformer
// sets with a causal window of at most 128 keys ([i-L, i], L <= 127) and 1 to
// 16 global tokens, 16-bit, head_dim 64.  Workspace: per (batch, head), for
// each chunk and one more slot (block 0's sums of keys 0..G-1), the global
// rows' dQ and the global keys' dK, dV sums (3 x 16 x 64 floats).
struct LfPlan {
  int64_t per_wg, wgs, nslot, part_bytes;
};

LfPlan lf_plan(const ma_attn_desc* d) {
  LfPlan p;
  const int64_t nt = (d->seq_len + kLfRows - 1) / kLfRows;
  const int64_t streams = ma::imax64(d->batch * d->num_heads, 1);
  // one workgroup per CU (131 KB of LDS): the streams' tiles in equal runs
  // over one round of 256 workgroups, a run at most one stream long (so it
  // meets at most two streams); from 256 streams on, one stream per
  // workgroup
  const int64_t tiles = streams * nt;
  p.per_wg = streams >= 256 ? nt : ma::imax64(1, (tiles + 255) / 256);
  p.wgs = (tiles + p.per_wg - 1) / p.per_wg;
  p.nslot = (nt + p.per_wg - 1) / p.per_wg + 1;  // workgroups whose runs meet one stream, at most
  p.part_bytes = streams * (p.nslot + 1) * kLfPart * (int64_t)sizeof(float);
  return p;
}

bool lf_applies(const ma_attn_desc* d, const void* const* ptrs, int n) {
  if (d->pattern != MA_ATTN_LONGFORMER || d->dtype == MA_ATTN_F32 || d->head_dim != kHeadDim) return false;
  if (g_opt.force_rows || d->right != 0 || d->left < 0 || d->left >= kLfRows || d->num_global < 1 ||
      d->num_global > 16)
    return false;
  for (int i = 0; i < n; ++i)
    if (!aligned16(ptrs[i])) return false;
  const int64_t tb = d->num_heads * kHeadDim * 2;
  return (d->seq_len + 2 * kLfRows) * tb < (1LL << 31) &&
         lf_plan(d).wgs <= (int64_t)INT32_MAX && d->batch * d->num_heads <= (int64_t)INT32_MAX;
}

// ma_attn_backward on LONGFORMER (the one-pass domain): the forward in delta
// mode (lse and sum_j P_ij dP_ij per row; no O written), then the one-pass
// backward reading them.  Workspace: lse, delta, the forward's
// global-row partials, the backward's partials.
struct LfBwdWs {
  int64_t off_dlt, off_fp, fp_bytes, off_bp, bp_bytes, total;
};

LfBwdWs lf_bwd_ws(const ma_attn_desc* d) {
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t rows = d->batch * d->seq_len * d->num_heads;
  LfBwdWs w;
  w.off_dlt = up(rows * (int64_t)sizeof(float));
  w.off_fp = w.off_dlt + up(rows * (int64_t)sizeof(float));
  w.fp_bytes = stream_plan(d).partial_bytes;
  w.off_bp = w.off_fp + up(w.fp_bytes);
  w.bp_bytes = lf_plan(d).part_bytes;
  w.total = w.off_bp + w.bp_bytes;
  return w;
}

// delta (optional): each row's delta from a delta-mode forward; the DLT
// kernels read it and not o.
template <typename T>
int launch_lf_bwd(const ma_attn_desc* d, const void* const* ptrs, const void* o, const float* lse, void* ws,
                  hipStream_t st, const float* delta = nullptr) {
  const LfPlan p = lf_plan(d);
  LfArgs a;
  a.q = ptrs[0];
  a.k = ptrs[1];
  a.v = ptrs[2];
  a.dout = ptrs[3];
  a.dq = const_cast<void*>(ptrs[4]);
  a.dk = const_cast<void*>(ptrs[5]);
  a.dv = const_cast<void*>(ptrs[6]);
  a.o = o;
  a.lse = lse;
  a.delta = delta;
  a.part = static_cast<float*>(ws);
  a.N = (int32_t)d->seq_len;
  a.H = (int32_t)d->num_heads;
  a.L = (int32_t)d->left;
  a.G = (int32_t)ma::imin64(d->num_global, d->seq_len);
  a.streams = (int32_t)(d->batch * d->num_heads);
  a.per_wg = (int32_t)p.per_wg;
  a.nslot = (int32_t)p.nslot;
  a.tok_bytes = (int32_t)(d->num_heads * kHeadDim * sizeof(T));
  a.scale = scale_of(d);
  a.scale_log2 = a.scale * 1.4426950408889634f;
  const bool fixed = d->left == kLfRows - 1;
  auto kf = delta ? (fixed ? &bwd_lf_kernel<HalfPath<T>, true, true> : &bwd_lf_kernel<HalfPath<T>, false, true>)
                  : (fixed ? &bwd_lf_kernel<HalfPath<T>, true, false> : &bwd_lf_kernel<HalfPath<T>, false, false>);
  if (reserve_lds(reinterpret_cast<const void*>(kf), (size_t)LfLds::kBytes, st)) return 1;
  const int64_t streams = d->batch * d->num_heads;
  launch(false, kf, dim3((unsigned)p.wgs), dim3(kLfThreads), (uint32_t)LfLds::kBytes, st, a);
  launch(true, bwd_lf_combine<T>, dim3((unsigned)(streams * kLfCombineBlocks)), dim3(256), 0u, st, a);
  return 0;
}

// ------------------------------------------------------------------ tiled index sets
//
// INDEX_SET with a tile plan (ma_attn_tile_plan), head_dim 64, 16-byte
// aligned tensors: tile_kernel.h.  Workspace: the partial results of split
// work items, per (batch, head): forward [q partials][64][kTilePart] floats;
// backward the statistics, then one region the three passes reuse in turn
// ([q partials][64][kTilePart], [q partials][64][64], [k partials][64][128]).
bool tiles_apply(const ma_attn_desc* d, const void* const* ptrs, int n) {
  if (d->pattern != MA_ATTN_INDEX_SET || !d->tile_header || !d->tile_plan || d->head_dim != kHeadDim) return false;
  if (g_opt.force_rows) return false;
  for (int i = 0; i < n; ++i)
    if (!aligned16(ptrs[i])) return false;
  const ma_attn_tile_header& h = *d->tile_header;
  const int64_t tb = d->num_heads * kHeadDim * (d->dtype == MA_ATTN_F32 ? 4 : 2);
  const int64_t items = h.num_q_items > h.num_k_items ? h.num_q_items : h.num_k_items;
  return (d->seq_len + 64) * tb < (1LL << 31) && d->batch * d->num_heads * items <= (int64_t)INT32_MAX &&
         h.num_entries < (1LL << 30) && h.num_tiles < (1LL << 25) && (d->seq_len + 64) * d->num_heads * 8 < (1LL << 31);
}

int64_t tiles_fwd_part_bytes(const ma_attn_desc* d) {
  return d->batch * d->num_heads * d->tile_header->num_q_partials * 64 * kTilePart * (int64_t)sizeof(float);
}

int64_t tiles_bwd_part_bytes(const ma_attn_desc* d) {
  const ma_attn_tile_header& h = *d->tile_header;
  const int64_t q = h.num_q_partials * 64 * kTilePart, k = h.num_k_partials * 64 * 128;
  return d->batch * d->num_heads * (q > k ? q : k) * (int64_t)sizeof(float);
}

int64_t stats_bytes(const ma_attn_desc* d) {
  return (d->batch * d->seq_len * d->num_heads * (int64_t)sizeof(RowStat) + 255) / 256 * 256;
}

TileArgs tile_args(const ma_attn_desc* d, bool kside) {
  const ma_attn_tile_header& h = *d->tile_header;
  const uint8_t* base = static_cast<const uint8_t*>(d->tile_plan);
  TileArgs a;
  memset(&a, 0, sizeof(a));
  a.blk = reinterpret_cast<const int32_t*>(base + h.off_blk);
  a.mask = reinterpret_cast<const uint64_t*>(base + h.off_mask);
  a.kmask = reinterpret_cast<const uint64_t*>(base + h.off_kmask);
  a.etile = reinterpret_cast<const int32_t*>(base + h.off_tile);
  a.kentry = reinterpret_cast<const int32_t*>(base + h.off_kentry);
  a.items = reinterpret_cast<const int32_t*>(base + (kside ? h.off_k_items : h.off_q_items));
  a.split = reinterpret_cast<const int32_t*>(base + (kside ? h.off_k_split : h.off_q_split));
  a.nitems = (int32_t)(kside ? h.num_k_items : h.num_q_items);
  a.nsplit = (int32_t)(kside ? h.num_k_split : h.num_q_split);
  a.npart = (int32_t)(kside ? h.num_k_partials : h.num_q_partials);
  a.nent = (int32_t)h.num_entries;
  a.ntiles = (int32_t)h.num_tiles;
  a.N = (int32_t)d->seq_len;
  a.H = (int32_t)d->num_heads;
  a.scale = scale_of(d);
  a.scale_log2 = a.scale * 1.4426950408889634f;
  return a;
}

template <class P>
int launch_tiles_fwd(const ma_attn_desc* d, const void* q, const void* k, const void* v, void* o, float* lse,
                     void* ws, size_t ws_bytes, hipStream_t st) {
  const int64_t need = tiles_fwd_part_bytes(d);
  if ((int64_t)ws_bytes < need || (need > 0 && !ws))
    return fail("ma_attn: workspace of %lld bytes required (ma_attn_workspace_size), got %zu", (long long)need,
                ws_bytes);
  TileArgs a = tile_args(d, false);
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.part = static_cast<float*>(ws);
  const int64_t bh = d->batch * d->num_heads;
  const size_t shm = 2 * (size_t)P::kBlk;
  // a plan of full entries only (block tables) takes the kernels with no mask work
  auto kf = d->tile_header->num_masked != 0 ? &tile_fwd_kernel<P, false, true>
                                            : &tile_fwd_kernel<P, false, false>;
  if (reserve_lds(reinterpret_cast<const void*>(kf), shm, st)) return 1;
  launch(a.nsplit == 0, kf, dim3((unsigned)(bh * a.nitems)), dim3(256), (uint32_t)shm, st, a);
  if (a.nsplit > 0)
    launch(true, tile_combine_kernel<typename P::Elt, false>, dim3((unsigned)(bh * a.nsplit * (64 / kMergeRows))),
           dim3(256), 0u, st, a);
  return 0;
}

// fo, lse: the forward's O and statistics (ma_attn_backward_saved), or null:
// then the statistics are recomputed.
template <class P>
int launch_tiles_bwd(const ma_attn_desc* d, const void* const* ptrs, void* ws, hipStream_t st, const void* fo,
                     const float* lse) {
  TileArgs a = tile_args(d, false);
  a.fo = fo;
  a.lse = const_cast<float*>(lse);
  a.q = ptrs[0];
  a.k = ptrs[1];
  a.v = ptrs[2];
  a.dout = ptrs[3];
  a.o = const_cast<void*>(ptrs[4]);  // dQ
  a.dk = const_cast<void*>(ptrs[5]);
  a.dv = const_cast<void*>(ptrs[6]);
  a.stats = static_cast<float*>(ws);
  a.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + stats_bytes(d));
  const int64_t bh = d->batch * d->num_heads;
  using Elt = typename P::Elt;
  const bool masked = d->tile_header->num_masked != 0;
  auto kf = masked ? &tile_fwd_kernel<P, true, true> : &tile_fwd_kernel<P, true, false>;
  const bool saved = lse != nullptr;
  auto kq = saved ? (masked ? &tile_dq_kernel<P, true, true> : &tile_dq_kernel<P, false, true>)
                  : (masked ? &tile_dq_kernel<P, true, false> : &tile_dq_kernel<P, false, false>);
  auto kkv = masked ? &tile_dkv_kernel<P, true> : &tile_dkv_kernel<P, false>;
  const size_t shm_f = 2 * (size_t)P::kBlk, shm_q = 2 * (size_t)PairLds<P>::kBytes,
               shm_kv = 2 * ((size_t)PairLds<P>::kBytes + 512);
  if (reserve_lds(reinterpret_cast<const void*>(kf), shm_f, st) ||
      reserve_lds(reinterpret_cast<const void*>(kq), shm_q, st) ||
      reserve_lds(reinterpret_cast<const void*>(kkv), shm_kv, st))
    return 1;
  // split tiles: statistics from partials and their merge; then dQ (unsplit
  // tiles compute their own statistics there).  From saved statistics every
  // tile takes them in the dQ pass.
  if (a.nsplit > 0 && !saved) {
    launch(false, kf, dim3((unsigned)(bh * a.nitems)), dim3(256), (uint32_t)shm_f, st, a);
    launch(false, tile_combine_kernel<Elt, true>, dim3((unsigned)(bh * a.nsplit * (64 / kMergeRows))), dim3(256), 0u,
           st, a);
  }
  launch(false, kq, dim3((unsigned)(bh * a.nitems)), dim3(256), (uint32_t)shm_q, st, a);
  if (a.nsplit > 0)
    launch(false, tile_sum_kernel<Elt, 64>, dim3((unsigned)(bh * a.nsplit * (64 / kMergeRows))), dim3(256), 0u, st, a);
  // dK, dV (key side)
  TileArgs b = tile_args(d, true);
  b.q = a.q;
  b.k = a.k;
  b.v = a.v;
  b.dout = a.dout;
  b.dk = a.dk;
  b.dv = a.dv;
  b.stats = a.stats;
  b.part = a.part;
  launch(b.nsplit == 0, kkv, dim3((unsigned)(bh * b.nitems)), dim3(256), (uint32_t)shm_kv, st, b);
  if (b.nsplit > 0)
    launch(true, tile_sum_kernel<Elt, 128>, dim3((unsigned)(bh * b.nsplit * (64 / kMergeRows))), dim3(256), 0u, st, b);
  return 0;
}

uint64_t splitmix64(uint64_t* s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

}  // namespace

extern "C" {

int ma_attn_abi_version(void) { return MA_ATTN_ABI_VERSION; }

const char* ma_attn_last_error(void) { return g_last_error.c_str(); }

int ma_attn_validate(const ma_attn_desc* desc) {
  g_last_error.clear();
  return validate(desc);
}

size_t ma_attn_workspace_size(const ma_attn_desc* desc) {
  g_last_error.clear();
  if (validate(desc)) return 0;
  if (desc->batch * desc->seq_len * desc->num_heads == 0 || desc->head_dim != kHeadDim) return 0;
  // the size the kernels need whenever they may take this descriptor
  // (pointer alignment is not known here; 16-byte-aligned tensors are assumed)
  static const char dummy[16] __attribute__((aligned(16))) = {0};
  const void* const ptrs[4] = {dummy, dummy, dummy, dummy};
  if (tiles_apply(desc, ptrs, 4)) return (size_t)tiles_fwd_part_bytes(desc);
  if (desc->pattern != MA_ATTN_LONGFORMER) return 0;
  if (!stream_applies(desc, dummy, dummy, dummy, dummy)) return 0;
  return (size_t)stream_plan(desc).partial_bytes;
}

int ma_attn_forward(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o,
                    void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (validate(desc)) return 1;
  const int64_t rows = desc->batch * desc->seq_len * desc->num_heads;
  if (rows == 0 || desc->head_dim == 0) return 0;
  if (!q || !k || !v || !o) return fail("ma_attn: null tensor pointer");
  return forward_launch(desc, q, k, v, o, nullptr, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int ma_attn_forward_lse(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o,
                        float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (validate(desc)) return 1;
  const int64_t rows = desc->batch * desc->seq_len * desc->num_heads;
  if (rows == 0 || desc->head_dim == 0) return 0;
  if (!q || !k || !v || !o || !lse) return fail("ma_attn_forward_lse: null tensor pointer");
  return forward_launch(desc, q, k, v, o, lse, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int ma_attn_forward_noalloc(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o,
                            void* stream) {
  g_last_error.clear();
  if (validate(desc)) return 1;
  const int64_t rows = desc->batch * desc->seq_len * desc->num_heads;
  if (rows == 0 || desc->head_dim == 0) return 0;
  if (!q || !k || !v || !o) return fail("ma_attn: null tensor pointer");
  // the scratch the kernels that take this call would need (the Longformer
  // stream kernel's per-chunk partials, a tiled index set's split partials;
  // nothing for every other kernel)
  const void* const qkvo[4] = {q, k, v, o};
  const size_t need = stream_applies(desc, q, k, v, o) ? (size_t)stream_plan(desc).partial_bytes
                      : tiles_apply(desc, qkvo, 4)     ? (size_t)tiles_fwd_part_bytes(desc)
                                                       : 0;
  if (need > (size_t)MA_ATTN_NOALLOC_SCRATCH_BYTES)
    return fail("ma_attn_forward_noalloc: this call needs %zu bytes of scratch, above the %zu bytes of the "
                "library's static scratch; use ma_attn_forward with a workspace",
                need, (size_t)MA_ATTN_NOALLOC_SCRATCH_BYTES);
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if (need > 0 && scratch_of_stream(st, &ws)) return 1;
  return forward_launch(desc, q, k, v, o, nullptr, ws, need, st);
}

}  // extern "C"

namespace {

// lse: optional per-row softmax statistics (ma_attn_forward_lse), written by
// the block-row, tiled and Longformer stream kernels; other kernels refuse
// it.
int forward_launch(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o, float* lse,
                   void* workspace, size_t workspace_bytes, hipStream_t st) {
  (void)hipGetLastError();  // launch errors below must be ours
  const void* const qkvo[4] = {q, k, v, o};
  int rc;
  const bool want_rows = g_opt.force_rows;
  const bool want_band = g_opt.force_band;
  const bool stream = !want_rows && !want_band && stream_applies(desc, q, k, v, o);
  const bool block = !stream && !want_rows && block_applies(desc, q, k, v, o);
  if (lse && !block && !tiles_apply(desc, qkvo, 4) &&
      !(stream && desc->pattern == MA_ATTN_LONGFORMER && desc->num_global > 0))
    return fail("ma_attn_forward_lse: these kernels write no statistics (block-sparse, dense, Longformer "
                "with 1 to 16 global tokens and index sets with a tile plan do, at head_dim 64)");
  if (stream) {
    rc = launch_stream(desc, q, k, v, o, lse, workspace, workspace_bytes, st);
  } else if (block) {
    rc = launch_block(desc, q, k, v, o, lse, st);
  } else if (!want_rows && band_applies(desc, q, k, v, o)) {
    rc = launch_band(desc, q, k, v, o, st);
  } else if (tiles_apply(desc, qkvo, 4)) {
    switch (desc->dtype) {
      case MA_ATTN_F32:
        rc = launch_tiles_fwd<F32Path>(desc, q, k, v, o, lse, workspace, workspace_bytes, st);
        break;
      case MA_ATTN_BF16:
        rc = launch_tiles_fwd<HalfPath<__bf16>>(desc, q, k, v, o, lse, workspace, workspace_bytes, st);
        break;
      default:
        rc = launch_tiles_fwd<HalfPath<_Float16>>(desc, q, k, v, o, lse, workspace, workspace_bytes, st);
        break;
    }
  } else if (!want_rows && gather_applies(desc, q, k, v, o)) {
    switch (desc->dtype) {
      case MA_ATTN_F32:
        rc = launch_gather<float>(desc, q, k, v, o, st);
        break;
      case MA_ATTN_BF16:
        rc = launch_gather<__bf16>(desc, q, k, v, o, st);
        break;
      default:
        rc = launch_gather<_Float16>(desc, q, k, v, o, st);
        break;
    }
  } else if (!want_rows && narrow_applies(desc)) {
    switch (desc->dtype) {
      case MA_ATTN_F32:
        rc = launch_narrow<float>(desc, q, k, v, o, st);
        break;
      case MA_ATTN_BF16:
        rc = launch_narrow<__bf16>(desc, q, k, v, o, st);
        break;
      default:
        rc = launch_narrow<_Float16>(desc, q, k, v, o, st);
        break;
    }
  } else {
    switch (desc->dtype) {
      case MA_ATTN_F32:
        rc = launch_rows<float>(desc, q, k, v, o, st);
        break;
      case MA_ATTN_BF16:
        rc = launch_rows<__bf16>(desc, q, k, v, o, st);
        break;
      default:
        rc = launch_rows<_Float16>(desc, q, k, v, o, st);
        break;
    }
  }
  if (rc) return rc;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("ma_attn: kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

}  // namespace

extern "C" {

size_t ma_attn_backward_workspace_size(const ma_attn_desc* desc) {
  g_last_error.clear();
  if (validate(desc)) return 0;
  static const char dummy[16] __attribute__((aligned(16))) = {0};
  const void* const ptrs[7] = {dummy, dummy, dummy, dummy, dummy, dummy, dummy};
  if (desc->batch * desc->seq_len * desc->num_heads > 0 && tiles_apply(desc, ptrs, 7))
    return (size_t)(stats_bytes(desc) + tiles_bwd_part_bytes(desc));
  if (desc->batch * desc->seq_len * desc->num_heads > 0 && lf_applies(desc, ptrs, 7))
    return (size_t)lf_bwd_ws(desc).total;  // ma_attn_backward's (ma_attn_backward_saved needs part of it)
  return (size_t)(desc->batch * desc->seq_len * desc->num_heads) * sizeof(RowStat);
}

int ma_attn_backward(const ma_attn_desc* desc, const void* q, const void* k, const void* v, const void* dout,
                     void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (validate(desc)) return 1;
  if (!backward_supported(desc))
    return fail("ma_attn_backward: pattern %d has no backward (SLIDING, DENSE, INDEX_SET and LONGFORMER only)",
                desc->pattern);
  if (desc->pattern == MA_ATTN_INDEX_SET && desc->seq_len > 0 &&
      (!desc->index_t_offsets || (desc->num_indices > 0 && !desc->index_t_queries)))
    return fail("ma_attn_backward: an index set needs its transposed set (index_t_offsets, index_t_queries)");
  const int64_t rows = desc->batch * desc->seq_len * desc->num_heads;
  if (rows == 0 || desc->head_dim == 0) return 0;
  if (!q || !k || !v || !dout || !dq || !dk || !dv) return fail("ma_attn_backward: null tensor pointer");
  if (desc->pattern == MA_ATTN_LONGFORMER) {
    const void* ptrs[7] = {q, k, v, dout, dq, dk, dv};
    if (!lf_applies(desc, ptrs, 7) || !stream_applies(desc, q, k, v, dout))
      return fail("ma_attn_backward: LONGFORMER takes 16-bit tensors, head_dim 64, right = 0, left < 128, 1 to 16 "
                  "global tokens, 16-byte aligned tensors (index_set_backward over the pattern's key sets "
                  "serves the rest)");
    const LfBwdWs w = lf_bwd_ws(desc);
    if (!workspace || workspace_bytes < (size_t)w.total)
      return fail("ma_attn_backward: workspace of %lld bytes needed, %zu given", (long long)w.total,
                  workspace_bytes);
    hipStream_t st = static_cast<hipStream_t>(stream);
    (void)hipGetLastError();
    uint8_t* wb = static_cast<uint8_t*>(workspace);
    float* lse = reinterpret_cast<float*>(wb);
    float* dlt = reinterpret_cast<float*>(wb + w.off_dlt);
    // The forward's kernels leave a timed call's stop event to the backward's last.
    hipEvent_t stop = g_ev_stop;
    g_ev_stop = nullptr;
    int rc = launch_stream(desc, q, k, v, nullptr, lse, wb + w.off_fp, (size_t)w.fp_bytes, st, dout, dlt);
    g_ev_stop = stop;
    if (!rc)
      rc = desc->dtype == MA_ATTN_BF16
               ? launch_lf_bwd<__bf16>(desc, ptrs, nullptr, lse, wb + w.off_bp, st, dlt)
               : launch_lf_bwd<_Float16>(desc, ptrs, nullptr, lse, wb + w.off_bp, st, dlt);
    if (rc) return rc;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("ma_attn_backward: kernel launch failed: %s", hipGetErrorString(e));
    return 0;
  }
  const size_t need = (size_t)rows * sizeof(RowStat);
  if (!workspace || workspace_bytes < need)
    return fail("ma_attn_backward: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  RowStat* stats = static_cast<RowStat*>(workspace);
  const void* ptrs[7] = {q, k, v, dout, dq, dk, dv};
  int rc;
  if (tiles_apply(desc, ptrs, 7)) {
    const size_t need_t = (size_t)(stats_bytes(desc) + tiles_bwd_part_bytes(desc));
    if (workspace_bytes < need_t)
      return fail("ma_attn_backward: workspace of %zu bytes needed, %zu given", need_t, workspace_bytes);
    rc = desc->dtype == MA_ATTN_BF16 ? launch_tiles_bwd<HalfPath<__bf16>>(desc, ptrs, workspace, st, nullptr, nullptr)
         : desc->dtype == MA_ATTN_F16
             ? launch_tiles_bwd<HalfPath<_Float16>>(desc, ptrs, workspace, st, nullptr, nullptr)
             : launch_tiles_bwd<F32BwdPath>(desc, ptrs, workspace, st, nullptr, nullptr);
    if (rc) return rc;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("ma_attn_backward: kernel launch failed: %s", hipGetErrorString(e));
    return 0;
  }
  if (!g_opt.force_rows && bwd_mfma_applies(desc, ptrs)) {
    float* sf = reinterpret_cast<float*>(stats);
    rc = desc->dtype == MA_ATTN_BF16  ? launch_backward_mfma<HalfPath<__bf16>>(desc, ptrs, sf, st)
         : desc->dtype == MA_ATTN_F16 ? launch_backward_mfma<HalfPath<_Float16>>(desc, ptrs, sf, st)
                                      : launch_backward_mfma<F32BwdPath>(desc, ptrs, sf, st);
    if (rc) return rc;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("ma_attn_backward: kernel launch failed: %s", hipGetErrorString(e));
    return 0;
  }
  switch (desc->dtype) {
    case MA_ATTN_F32:
      rc = launch_backward<float>(desc, q, k, v, dout, dq, dk, dv, stats, st);
      break;
    case MA_ATTN_BF16:
      rc = launch_backward<__bf16>(desc, q, k, v, dout, dq, dk, dv, stats, st);
      break;
    default:
      rc = launch_backward<_Float16>(desc, q, k, v, dout, dq, dk, dv, stats, st);
      break;
  }
  if (rc) return rc;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("ma_attn_backward: kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

int ma_attn_forward_timed(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o,
                          void* workspace, size_t workspace_bytes, void* stream, void* start_event,
                          void* stop_event) {
  g_ev_start = static_cast<hipEvent_t>(start_event);
  g_ev_stop = static_cast<hipEvent_t>(stop_event);
  const int rc = ma_attn_forward(desc, q, k, v, o, workspace, workspace_bytes, stream);
  g_ev_start = g_ev_stop = nullptr;
  return rc;
}

int ma_attn_forward_lse_timed(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o,
                              float* lse, void* workspace, size_t workspace_bytes, void* stream, void* start_event,
                              void* stop_event) {
  g_ev_start = static_cast<hipEvent_t>(start_event);
  g_ev_stop = static_cast<hipEvent_t>(stop_event);
  const int rc = ma_attn_forward_lse(desc, q, k, v, o, lse, workspace, workspace_bytes, stream);
  g_ev_start = g_ev_stop = nullptr;
  return rc;
}

int ma_attn_backward_saved(const ma_attn_desc* desc, const void* q, const void* k, const void* v, const void* o,
                           const float* lse, const void* dout, void* dq, void* dk, void* dv, void* workspace,
                           size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (validate(desc)) return 1;
  const int64_t rows = desc->batch * desc->seq_len * desc->num_heads;
  if (rows == 0 || desc->head_dim == 0) return 0;
  if (!q || !k || !v || !o || !lse || !dout || !dq || !dk || !dv)
    return fail("ma_attn_backward_saved: null tensor pointer");
  const void* ptrs[8] = {q, k, v, dout, dq, dk, dv, o};
  const bool tiles = tiles_apply(desc, ptrs, 8);
  const bool dense =
      desc->pattern == MA_ATTN_DENSE && !g_opt.force_rows && aligned16(o) && bwd_mfma_applies(desc, ptrs);
  const bool lf = lf_applies(desc, ptrs, 8);
  if (!tiles && !dense && !lf)
    return fail("ma_attn_backward_saved: takes an INDEX_SET with a tile plan, DENSE, or LONGFORMER (16-bit, "
                "window [i-L, i] with L <= 127, 1 to 16 global tokens), head_dim 64, 16-byte aligned tensors");
  const size_t need = tiles ? (size_t)(stats_bytes(desc) + tiles_bwd_part_bytes(desc))
                      : lf  ? (size_t)lf_plan(desc).part_bytes
                            : (size_t)rows * sizeof(RowStat);
  if (!workspace || workspace_bytes < need)
    return fail("ma_attn_backward_saved: workspace of %zu bytes needed, %zu given", need, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  float* sf = static_cast<float*>(workspace);
  const int rc =
      lf ? (desc->dtype == MA_ATTN_BF16 ? launch_lf_bwd<__bf16>(desc, ptrs, o, lse, workspace, st)
                                        : launch_lf_bwd<_Float16>(desc, ptrs, o, lse, workspace, st))
      : tiles ? (desc->dtype == MA_ATTN_BF16 ? launch_tiles_bwd<HalfPath<__bf16>>(desc, ptrs, workspace, st, o, lse)
               : desc->dtype == MA_ATTN_F16
                   ? launch_tiles_bwd<HalfPath<_Float16>>(desc, ptrs, workspace, st, o, lse)
                   : launch_tiles_bwd<F32BwdPath>(desc, ptrs, workspace, st, o, lse))
            : (desc->dtype == MA_ATTN_BF16 ? launch_backward_mfma<HalfPath<__bf16>>(desc, ptrs, sf, st, o, lse)
               : desc->dtype == MA_ATTN_F16
                   ? launch_backward_mfma<HalfPath<_Float16>>(desc, ptrs, sf, st, o, lse)
                   : launch_backward_mfma<F32BwdPath>(desc, ptrs, sf, st, o, lse));
  if (rc) return rc;
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("ma_attn_backward_saved: kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

int ma_attn_backward_saved_timed(const ma_attn_desc* desc, const void* q, const void* k, const void* v,
                                 const void* o, const float* lse, const void* dout, void* dq, void* dk, void* dv,
                                 void* workspace, size_t workspace_bytes, void* stream, void* start_event,
                                 void* stop_event) {
  g_ev_start = static_cast<hipEvent_t>(start_event);
  g_ev_stop = static_cast<hipEvent_t>(stop_event);
  const int rc =
      ma_attn_backward_saved(desc, q, k, v, o, lse, dout, dq, dk, dv, workspace, workspace_bytes, stream);
  g_ev_start = g_ev_stop = nullptr;
  return rc;
}

int ma_attn_backward_timed(const ma_attn_desc* desc, const void* q, const void* k, const void* v,
                           const void* dout, void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                           void* stream, void* start_event, void* stop_event) {
  g_ev_start = static_cast<hipEvent_t>(start_event);
  g_ev_stop = static_cast<hipEvent_t>(stop_event);
  const int rc = ma_attn_backward(desc, q, k, v, dout, dq, dk, dv, workspace, workspace_bytes, stream);
  g_ev_start = g_ev_stop = nullptr;
  return rc;
}

size_t ma_tick_features_workspace_size(int64_t n) {
  (void)n;
  return (size_t)ma_feat::kStatBlocks * ma_feat::kFeatures * 3 * sizeof(double);
}

int ma_tick_features(const double* timestamp, const double* price, const double* bid_price,
                     const double* ask_price, const double* bid_volume, const double* ask_volume, int64_t n,
                     float* out, double* stats, void* workspace, size_t workspace_bytes, void* stream) {
  g_last_error.clear();
  if (n < 0) return fail("ma_tick_features: negative tick count");
  if (n == 0) return 0;
  if (!timestamp || !price || !bid_price || !ask_price || !bid_volume || !ask_volume || !out || !stats)
    return fail("ma_tick_features: null pointer");
  if (!workspace || workspace_bytes < ma_tick_features_workspace_size(n))
    return fail("ma_tick_features: workspace of %zu bytes needed, %zu given", ma_tick_features_workspace_size(n),
                workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const ma_feat::TickCols c{timestamp, price, bid_price, ask_price, bid_volume, ask_volume};
  const int blocks = (int)ma::imax64(1, ma::imin64(ma_feat::kStatBlocks, (n + 4095) / 4096));
  double* partial = static_cast<double*>(workspace);
  launch(false, ma_feat::features_stats, dim3((unsigned)blocks), dim3(ma_feat::kStatThreads), 0, st, c, n, partial);
  launch(false, ma_feat::features_finish, dim3(1), dim3(ma_feat::kFinishThreads), 0, st, (const double*)partial, blocks, stats);
  const int wblocks = (int)ma::imax64(1, ma::imin64(8192, (n + 1023) / 1024));
  launch(true, ma_feat::features_write, dim3((unsigned)wblocks), dim3(256), 0, st, c, n, (const double*)stats, out);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("ma_tick_features: kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

int ma_tick_features_timed(const double* timestamp, const double* price, const double* bid_price,
                           const double* ask_price, const double* bid_volume, const double* ask_volume, int64_t n,
                           float* out, double* stats, void* workspace, size_t workspace_bytes, void* stream,
                           void* start_event, void* stop_event) {
  g_ev_start = static_cast<hipEvent_t>(start_event);
  g_ev_stop = static_cast<hipEvent_t>(stop_event);
  const int rc = ma_tick_features(timestamp, price, bid_price, ask_price, bid_volume, ask_volume, n, out, stats,
                                  workspace, workspace_bytes, stream);
  g_ev_start = g_ev_stop = nullptr;
  return rc;
}

int ma_attn_block_table(uint64_t seed, int64_t num_blocks, int64_t random_per_row, int32_t* out) {
  g_last_error.clear();
  if (num_blocks < 0 || random_per_row < 0 || random_per_row > 62 || (!out && num_blocks > 0))
    return fail("ma_attn_block_table: bad arguments");
  const int64_t w = 2 + random_per_row;
  const uint64_t nb = (uint64_t)num_blocks;
  const uint64_t limit = nb ? (UINT64_MAX / nb) * nb : 0;
  for (int64_t r = 0; r < num_blocks; ++r) {
    int32_t row[64];
    int64_t cnt = 0;
    row[cnt++] = (int32_t)r;
    if (r >= 1) row[cnt++] = (int32_t)(r - 1);
    const int64_t want = ma::imin64(random_per_row, num_blocks - cnt);
    uint64_t s = seed ^ (0x9E3779B97F4A7C15ull * (uint64_t)(r + 1));
    int64_t got = 0;
    while (got < want) {
      const uint64_t z = splitmix64(&s);
      if (z >= limit) continue;
      const int32_t cand = (int32_t)(z % nb);
      bool dup = false;
      for (int64_t e = 0; e < cnt; ++e) dup = dup || row[e] == cand;
      if (dup) continue;
      row[cnt++] = cand;
      ++got;
    }
    for (int64_t x = 1; x < cnt; ++x) {  // insertion sort, ascending
      const int32_t key = row[x];
      int64_t y = x - 1;
      while (y >= 0 && row[y] > key) {
        row[y + 1] = row[y];
        --y;
      }
      row[y + 1] = key;
    }
    for (int64_t e = 0; e < w; ++e) out[r * w + e] = e < cnt ? row[e] : -1;
  }
  return 0;
}

int64_t ma_attn_row_keys(const ma_attn_desc* desc, const int32_t* host_block_table, int64_t i,
                         int64_t* keys_out, int64_t cap) {
  g_last_error.clear();
  if (validate(desc)) return -1;
  if (desc->pattern == MA_ATTN_BLOCK_SPARSE && !host_block_table) {
    fail("ma_attn_row_keys: block table required");
    return -1;
  }
  if (desc->pattern == MA_ATTN_INDEX_SET) {
    fail("ma_attn_row_keys: an index set's keys are the caller's own input");
    return -1;
  }
  const ma::PatternParams pp = params_of(desc, host_block_table);
  const ma::RowKeys rk = ma::row_keys(pp, i);
  for (int64_t t = 0; t < rk.count && t < cap; ++t) keys_out[t] = ma::key_at(pp, rk, i, t);
  return rk.count;
}

int64_t ma_attn_pattern_csr(const ma_attn_desc* desc, const int32_t* host_block_table, int64_t* offsets_out,
                            int32_t* keys_out, int64_t keys_cap) {
  g_last_error.clear();
  if (validate(desc)) return -1;
  if (desc->pattern == MA_ATTN_BLOCK_SPARSE && !host_block_table && desc->seq_len > 0) {
    fail("ma_attn_pattern_csr: block table required");
    return -1;
  }
  if (desc->pattern == MA_ATTN_INDEX_SET) {
    fail("ma_attn_pattern_csr: an index set's keys are the caller's own input");
    return -1;
  }
  const ma::PatternParams pp = params_of(desc, host_block_table);
  const int64_t N = desc->seq_len;
  int64_t nnz = 0;
  for (int64_t i = 0; i < N; ++i) {
    if (offsets_out) offsets_out[i] = nnz;
    nnz += ma::row_keys(pp, i).count;
  }
  if (offsets_out) offsets_out[N] = nnz;
  if (!keys_out) return nnz;
  if (keys_cap < nnz) {
    fail("ma_attn_pattern_csr: %lld keys do not fit a buffer of %lld", (long long)nnz, (long long)keys_cap);
    return -1;
  }
  int64_t at = 0;
  for (int64_t i = 0; i < N; ++i) {
    const ma::RowKeys rk = ma::row_keys(pp, i);
    if (pp.pattern == ma::kBlockSparse) {
      // the row's table entries in order: whole blocks, clipped at N
      const int64_t bs = pp.block_size, row = i / bs;
      for (int64_t e = 0; e < pp.bpr; ++e) {
        const int32_t c = pp.table[row * pp.bpr + e];
        if (c < 0) continue;
        const int64_t end = ma::imin64((int64_t)c * bs + bs, N);
        for (int64_t j = (int64_t)c * bs; j < end; ++j) keys_out[at++] = (int32_t)j;
      }
    } else {
      for (int64_t t = 0; t < rk.count; ++t) keys_out[at++] = (int32_t)ma::key_at(pp, rk, i, t);
    }
  }
  return nnz;
}

int ma_attn_copy_probe(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o,
                       void* stream) {
  g_last_error.clear();
  if (validate(desc)) return 1;
  if (desc->pattern != MA_ATTN_SLIDING && desc->pattern != MA_ATTN_BLOCK_SPARSE)
    return fail("ma_attn_copy_probe: SLIDING and BLOCK_SPARSE descriptors only");
  if (desc->batch * desc->seq_len * desc->num_heads == 0) return 0;
  if (!q || !k || !v || !o) return fail("ma_attn: null tensor pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (desc->pattern == MA_ATTN_BLOCK_SPARSE) {
    if (!block_applies(desc, q, k, v, o) || desc->blocks_per_row > 4)
      return fail("ma_attn_copy_probe: the block-row kernel does not take this descriptor (block_size 64, "
                  "head_dim 64, at most 4 blocks per row, 16-byte aligned tensors)");
    BlockArgs a;
    memset(&a, 0, sizeof(a));
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.table = desc->block_table;
    a.N = (int32_t)desc->seq_len;
    a.H = (int32_t)desc->num_heads;
    a.bpr = (int32_t)desc->blocks_per_row;
    a.nbq = (int32_t)((desc->seq_len + 63) / 64);
    const unsigned grid = (unsigned)(desc->batch * desc->num_heads * a.nbq);
    (void)hipGetLastError();
    if (desc->dtype == MA_ATTN_F32)
      launch(true, block_probe_kernel<256>, dim3(grid), dim3(256), 0u, st, a);
    else
      launch(true, block_probe_kernel<128>, dim3(grid), dim3(256), 0u, st, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail("ma_attn_copy_probe: kernel launch failed: %s", hipGetErrorString(e));
    return 0;
  }
  if (!stream_applies(desc, q, k, v, o))
    return fail("ma_attn_copy_probe: the stream kernel does not take this descriptor (head_dim 64, "
                "left, right >= 0, 16-byte aligned tensors)");
  const StreamPlan p = stream_plan(desc);
  StreamArgs a;
  memset(&a, 0, sizeof(a));
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.N = desc->seq_len;
  a.H = desc->num_heads;
  a.left = (int32_t)p.geom.left;
  a.right = (int32_t)p.geom.right;
  a.dil = (int32_t)p.geom.dil;
  a.tiles = (int32_t)p.tiles;
  a.chunk = (int32_t)p.chunk;
  a.chunks = (int32_t)p.chunks;
  a.tok_bytes = (int32_t)p.tok_bytes;
  a.pairs = p.geom.right > 0 && p.wgs % 16 == 0 && p.chunks % 2 == 0 ? 1 : 0;  // as launch_stream
  (void)hipGetLastError();
  if (desc->dtype == MA_ATTN_F32)
    launch(true, copy_probe_kernel<256>, dim3((unsigned)p.wgs), dim3(256), 0u, st, a);
  else
    launch(true, copy_probe_kernel<128>, dim3((unsigned)p.wgs), dim3(256), 0u, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("ma_attn_copy_probe: kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

int ma_attn_copy_probe_timed(const ma_attn_desc* desc, const void* q, const void* k, const void* v, void* o,
                             void* stream, void* start_event, void* stop_event) {
  g_ev_start = static_cast<hipEvent_t>(start_event);
  g_ev_stop = static_cast<hipEvent_t>(stop_event);
  const int rc = ma_attn_copy_probe(desc, q, k, v, o, stream);
  g_ev_start = g_ev_stop = nullptr;
  return rc;
}

int ma_attn_backward_copy_probe(const ma_attn_desc* desc, const void* q, const void* k, const void* v,
                                const void* dout, void* dq, void* dk, void* dv, void* stream) {
  g_last_error.clear();
  if (validate(desc)) return 1;
  if (desc->batch * desc->seq_len * desc->num_heads == 0) return 0;
  if (!q || !k || !v || !dout || !dq || !dk || !dv) return fail("ma_attn: null tensor pointer");
  const void* ptrs[7] = {q, k, v, dout, dq, dk, dv};
  const int fixed = desc->pattern != MA_ATTN_SLIDING || desc->dtype == MA_ATTN_F32 || !bwd_mfma_applies(desc, ptrs)
                        ? 0
                    : desc->left == 63 && desc->right == 0  ? 1
                    : desc->left == 32 && desc->right == 31 ? 2
                                                            : 0;
  if (fixed == 0)
    return fail("ma_attn_backward_copy_probe: the fused backward does not take this descriptor (SLIDING, "
                "16-bit, head_dim 64, windows [i-63, i] or [i-32, i+31] of any dilation, 16-byte aligned "
                "tensors)");
  BwdArgs a;
  memset(&a, 0, sizeof(a));
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.N = desc->seq_len;
  a.H = desc->num_heads;
  a.left = (int32_t)desc->left;
  a.right = (int32_t)desc->right;
  a.dil = (int32_t)desc->dilation;
  const int64_t nr = (desc->seq_len + desc->dilation - 1) / desc->dilation;
  a.tiles = (int32_t)((nr + 63) / 64);
  a.tok_bytes = (int32_t)(desc->dilation * desc->num_heads * kHeadDim * 2);
  const int64_t streams = desc->batch * desc->num_heads * desc->dilation;
  fused_chunks(a, streams);
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  launch(true, fixed == 1 ? bwd_probe_kernel<63, 0> : bwd_probe_kernel<32, 31>, dim3((unsigned)(streams * a.chunks)),
         dim3(256), 0u, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail("ma_attn_backward_copy_probe: kernel launch failed: %s", hipGetErrorString(e));
  return 0;
}

int ma_attn_backward_copy_probe_timed(const ma_attn_desc* desc, const void* q, const void* k, const void* v,
                                      const void* dout, void* dq, void* dk, void* dv, void* stream,
                                      void* start_event, void* stop_event) {
  g_ev_start = static_cast<hipEvent_t>(start_event);
  g_ev_stop = static_cast<hipEvent_t>(stop_event);
  const int rc = ma_attn_backward_copy_probe(desc, q, k, v, dout, dq, dk, dv, stream);
  g_ev_start = g_ev_stop = nullptr;
  return rc;
}

int ma_attn_tile_plan(int64_t N, const int64_t* off, const int32_t* keys, int64_t seg, ma_attn_tile_header* hdr,
                      void* plan, size_t plan_bytes) {
  g_last_error.clear();
  if (!hdr) return fail("ma_attn_tile_plan: null header"), -1;
  if (N < 0 || N > (int64_t)INT32_MAX - 64) return fail("ma_attn_tile_plan: seq_len out of range"), -1;
  if (N > 0 && !off) return fail("ma_attn_tile_plan: null offsets"), -1;
  if (seg <= 0) seg = kTileSeg;
  const int64_t nnz = N > 0 ? off[N] : 0;
  if (N > 0 && off[0] != 0) return fail("ma_attn_tile_plan: offsets[0] must be 0"), -1;
  if (nnz > 0 && !keys) return fail("ma_attn_tile_plan: null keys"), -1;
  for (int64_t i = 0; i < N; ++i) {
    if (off[i + 1] < off[i] || off[i + 1] > nnz) return fail("ma_attn_tile_plan: offsets not non-decreasing"), -1;
    for (int64_t x = off[i]; x < off[i + 1]; ++x)
      if (keys[x] < 0 || keys[x] >= N || (x > off[i] && keys[x] <= keys[x - 1]))
        return fail("ma_attn_tile_plan: keys must be in [0, N) and strictly ascending per row"), -1;
  }
  const int64_t nt = (N + 63) / 64;
  // distinct key blocks of each query tile, ascending
  std::vector<int32_t> mark((size_t)nt, -1), tile_first((size_t)nt + 1, 0), ent_blk;
  std::vector<int32_t> list;
  for (int64_t t = 0; t < nt; ++t) {
    list.clear();
    const int64_t r1 = std::min<int64_t>(N, 64 * t + 64);
    for (int64_t i = 64 * t; i < r1; ++i)
      for (int64_t x = off[i]; x < off[i + 1]; ++x) {
        const int32_t c = keys[x] >> 6;
        if (mark[c] != (int32_t)t) {
          mark[c] = (int32_t)t;
          list.push_back(c);
        }
      }
    std::sort(list.begin(), list.end());
    ent_blk.insert(ent_blk.end(), list.begin(), list.end());
    tile_first[t + 1] = (int32_t)ent_blk.size();
  }
  const int64_t ne = (int64_t)ent_blk.size();
  // work items: every tile / key block gets at least one (an empty one writes zeros)
  std::vector<int32_t> kcount((size_t)nt, 0);
  for (int32_t c : ent_blk) ++kcount[c];
  auto items_of = [&](int64_t n) { return n <= seg ? (int64_t)1 : (n + seg - 1) / seg; };
  int64_t qi = 0, qs = 0, qp = 0, ki = 0, ks = 0, kp = 0;
  for (int64_t t = 0; t < nt; ++t) {
    const int64_t n = tile_first[t + 1] - tile_first[t], m = items_of(n);
    qi += m;
    if (m > 1) ++qs, qp += m;
    const int64_t mk = items_of(kcount[t]);
    ki += mk;
    if (mk > 1) ++ks, kp += mk;
  }
  ma_attn_tile_header h;
  memset(&h, 0, sizeof(h));
  h.seq_len = N;
  h.num_tiles = nt;
  h.num_entries = ne;
  h.seg = seg;
  h.num_q_items = qi;
  h.num_q_split = qs;
  h.num_q_partials = qp;
  h.num_k_items = ki;
  h.num_k_split = ks;
  h.num_k_partials = kp;
  int64_t at = 256;  // the header's copy comes first
  auto take = [&](int64_t bytes) {
    const int64_t o = at;
    at += (bytes + 255) / 256 * 256;
    return o;
  };
  h.off_blk = take(4 * ne);
  h.off_mask = take(8 * 64 * ne);
  h.off_kmask = take(8 * 64 * ne);
  h.off_tile = take(4 * ne);
  h.off_kentry = take(4 * ne);
  h.off_q_items = take(16 * qi);
  h.off_q_split = take(16 * qs);
  h.off_k_items = take(16 * ki);
  h.off_k_split = take(16 * ks);
  h.total_bytes = at;
  h.num_masked = -1;  // known once the masks are built
  *hdr = h;
  if (!plan) return 0;
  if (plan_bytes < (size_t)h.total_bytes) return fail("ma_attn_tile_plan: plan buffer too small"), -1;
  uint8_t* base = static_cast<uint8_t*>(plan);
  memset(base, 0, (size_t)h.total_bytes);
  memcpy(base, &h, sizeof(h));
  int32_t* blk = reinterpret_cast<int32_t*>(base + h.off_blk);
  uint64_t* mask = reinterpret_cast<uint64_t*>(base + h.off_mask);
  int32_t* etile = reinterpret_cast<int32_t*>(base + h.off_tile);
  int32_t* kentry = reinterpret_cast<int32_t*>(base + h.off_kentry);
  std::vector<int32_t> pos((size_t)nt, 0);
  for (int64_t t = 0; t < nt; ++t) {
    const int32_t e0 = tile_first[t], e1 = tile_first[t + 1];
    for (int32_t e = e0; e < e1; ++e) {
      pos[ent_blk[e]] = e;
      blk[e] = ent_blk[e];
      etile[e] = (int32_t)t;
    }
    const int64_t r1 = std::min<int64_t>(N, 64 * t + 64);
    for (int64_t i = 64 * t; i < r1; ++i)
      for (int64_t x = off[i]; x < off[i + 1]; ++x)
        mask[(int64_t)pos[keys[x] >> 6] * 64 + (i - 64 * t)] |= 1ull << (keys[x] & 63);
    // full entries: every row and key of the block exists and every pair is in the set
    if (64 * t + 63 < N)
      for (int32_t e = e0; e < e1; ++e) {
        bool full = 64 * (int64_t)ent_blk[e] + 63 < N;
        for (int r = 0; r < 64 && full; ++r) full = mask[(int64_t)e * 64 + r] == ~0ull;
        if (full) blk[e] |= 1 << 30;
      }
  }
  int64_t masked = 0;
  for (int64_t e = 0; e < ne; ++e) masked += (blk[e] & (1 << 30)) == 0;
  hdr->num_masked = masked;
  reinterpret_cast<ma_attn_tile_header*>(base)->num_masked = masked;
  // the transposed masks: bit r of word k
  uint64_t* kmask = reinterpret_cast<uint64_t*>(base + h.off_kmask);
  for (int64_t e = 0; e < ne; ++e)
    for (int r = 0; r < 64; ++r) {
      uint64_t w = mask[e * 64 + r];
      while (w) {
        const int k = __builtin_ctzll(w);
        kmask[e * 64 + k] |= 1ull << r;
        w &= w - 1;
      }
    }
  // entries by key block, then tile (stable: entries are in tile order)
  std::vector<int32_t> kfirst((size_t)nt + 1, 0);
  for (int64_t c = 0; c < nt; ++c) kfirst[c + 1] = kfirst[c] + kcount[c];
  {
    std::vector<int32_t> fill(kfirst.begin(), kfirst.end() - 1);
    for (int64_t e = 0; e < ne; ++e) kentry[fill[ent_blk[e]]++] = (int32_t)e;
  }
  int32_t* q_items = reinterpret_cast<int32_t*>(base + h.off_q_items);
  int32_t* q_split = reinterpret_cast<int32_t*>(base + h.off_q_split);
  int32_t* k_items = reinterpret_cast<int32_t*>(base + h.off_k_items);
  int32_t* k_split = reinterpret_cast<int32_t*>(base + h.off_k_split);
  auto emit = [&](int32_t* items, int32_t* split, int64_t& ni, int64_t& ns, int64_t& np, int32_t id, int32_t a,
                  int32_t b) {
    const int64_t n = b - a, m = items_of(n);
    if (m == 1) {
      int32_t* it = items + 4 * ni++;
      it[0] = id, it[1] = a, it[2] = b, it[3] = -1;
      return;
    }
    int32_t* sp = split + 4 * ns++;
    sp[0] = id, sp[1] = (int32_t)np, sp[2] = (int32_t)m, sp[3] = 0;
    for (int64_t j = 0; j < m; ++j) {
      int32_t* it = items + 4 * ni++;
      it[0] = id, it[1] = a + (int32_t)(j * seg), it[2] = (int32_t)std::min<int64_t>(b, a + (j + 1) * seg);
      it[3] = (int32_t)np++;
    }
  };
  int64_t ni = 0, ns = 0, np = 0;
  for (int64_t t = 0; t < nt; ++t) emit(q_items, q_split, ni, ns, np, (int32_t)t, tile_first[t], tile_first[t + 1]);
  ni = ns = np = 0;
  for (int64_t c = 0; c < nt; ++c) emit(k_items, k_split, ni, ns, np, (int32_t)c, kfirst[c], kfirst[c + 1]);
  return 0;
}

void ma_attn_reload_options(void) { g_opt = read_options(); }

}  // extern "C"
