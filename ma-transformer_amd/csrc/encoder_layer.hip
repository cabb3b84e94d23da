// encoder_layer.hip -- the reference encoder layer's eval-mode forward in one
// kernel (C-ABI in include/ma_encoder.h).
//
// Reference: CustomTransformerEncoderLayer.forward (src/model.py:42-53) with
// its SparseAttention (src/layers/sparse_attention.py:49-86: one head over
// [B, S, d_model], window w, keys [i-w, i+w]) and torch's LayerNorm / Linear.
//
// One workgroup (4 waves) per 16 consecutive tokens of [B*S, d_model]:
//   1. attention (16 lanes per token, d_model/16 values per lane): the row's
//      keys are its sequence's rows [i-w, i+w] (K = V = src), an online
//      softmax in registers; h = src + attn; LayerNorm1 -> LDS.
//   2. linear1 + bias + ReLU on fp32 MFMA (16x16x4): wave v computes hidden
//      units [v*d, (v+1)*d) of the 16 tokens -> LDS.
//   3. linear2 on fp32 MFMA: wave v contracts hidden units [v*d, (v+1)*d)
//      for every output column; the four partial sums meet in LDS and are
//      added in a fixed order.
//   4. residual, bias, LayerNorm2; each token's row stored once.
// MFMA operands: for 4 consecutive 16x16x4 steps, lane group g (lane/16)
// feeds contraction indices 16t + 4g + {0..3}, so each lane fetches its four
// A values (LDS) and four B values (the weight row, from L2) as one 16-byte
// read each.  The contraction order therefore differs from torch's; the
// arithmetic is float32 throughout.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>

#include "../../include/ma_encoder.h"
#include "device_common.h"

namespace ma_host {
void clear_error();
int set_error(const char* msg);
}  // namespace ma_host

namespace {

using ma_dev::f32x4;
using ma_dev::mfma_f32;

constexpr int kTokens = 16;  // tokens per workgroup

struct EncArgs {
  const float* src;
  const float* attn;  // null: computed here
  float* out;
  const float *g1, *be1, *w1, *bi1, *w2, *bi2, *g2, *be2;
  int64_t rows;  // batch * seq_len
  int32_t seq_len;
  int32_t window;  // clipped to [-1, seq_len]
  float scale;
  float eps;
};

template <int D>
struct EncGeom {
  static constexpr int F = 4 * D;       // hidden units
  static constexpr int EPT = D / 16;    // values per lane in the row passes (16 lanes per token)
  static constexpr int XS = D + 4;      // LDS row stride (floats) of LayerNorm1's output
  static constexpr int ZS = F + 4;      // of relu(linear1)
  static constexpr int PS = D + 4;      // of linear2's per-wave partial sums
  static constexpr int ZBUF = 16 * ZS > 64 * PS ? 16 * ZS : 64 * PS;
};

template <int N>
__device__ __forceinline__ void load_row(const float* p, float (&x)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int e = 0; e < N; e += 4) {
      const float4 v = *reinterpret_cast<const float4*>(p + e);
      x[e] = v.x;
      x[e + 1] = v.y;
      x[e + 2] = v.z;
      x[e + 3] = v.w;
    }
  } else if constexpr (N == 2) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    x[0] = v.x;
    x[1] = v.y;
  } else {
    x[0] = p[0];
  }
}

template <int N>
__device__ __forceinline__ void store_row(float* p, const float (&x)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int e = 0; e < N; e += 4) *reinterpret_cast<float4*>(p + e) = make_float4(x[e], x[e + 1], x[e + 2], x[e + 3]);
  } else if constexpr (N == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
  } else {
    p[0] = x[0];
  }
}

// Sum over the 16 lanes of a token (lanes 16k .. 16k+15 of a wave).
__device__ __forceinline__ float sum16(float x) {
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

// LayerNorm of a 16-lane-distributed row: (x - mean) / sqrt(var + eps) * g + b,
// biased variance, as torch.nn.LayerNorm.
template <int N, int D>
__device__ __forceinline__ void layer_norm(float (&x)[N], const float (&gw)[N], const float (&bw)[N], float eps) {
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < N; ++e) s += x[e];
  const float mean = sum16(s) / (float)D;
  float q = 0.0f;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float c = x[e] - mean;
    q = fmaf(c, c, q);
  }
  const float rstd = 1.0f / sqrtf(sum16(q) / (float)D + eps);
#pragma unroll
  for (int e = 0; e < N; ++e) x[e] = (x[e] - mean) * rstd * gw[e] + bw[e];
}

template <int D>
__global__ __launch_bounds__(256) void encoder_layer_kernel(EncArgs a) {
  using G = EncGeom<D>;
  constexpr int F = G::F, EPT = G::EPT, NT = D / 16;  // NT: 16-wide column tiles (and 16-deep k groups) per wave
  __shared__ __attribute__((aligned(16))) float xs[kTokens * G::XS];
  __shared__ __attribute__((aligned(16))) float zs[G::ZBUF];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const int r = tid >> 4, u = tid & 15;  // token of the tile, lane within the token
  const int d0 = u * EPT;
  const int64_t m = (int64_t)blockIdx.x * kTokens + r;
  const bool live = m < a.rows;

  // ---- 1. attention, residual, LayerNorm1
  float x[EPT], h[EPT];
#pragma unroll
  for (int e = 0; e < EPT; ++e) x[e] = 0.0f;
  if (live) load_row<EPT>(a.src + m * D + d0, x);
  // the lane's slices of both norms' affine parameters and linear2's bias,
  // loaded up front so their round trip overlaps the attention
  float g1[EPT], be1[EPT], g2[EPT], be2[EPT], b2[EPT];
  load_row<EPT>(a.g1 + d0, g1);
  load_row<EPT>(a.be1 + d0, be1);
  load_row<EPT>(a.g2 + d0, g2);
  load_row<EPT>(a.be2 + d0, be2);
  load_row<EPT>(a.bi2 + d0, b2);
  if (a.attn) {
    float at[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) at[e] = 0.0f;
    if (live) load_row<EPT>(a.attn + m * D + d0, at);
#pragma unroll
    for (int e = 0; e < EPT; ++e) h[e] = x[e] + at[e];
  } else {
    const int64_t i = live ? m % a.seq_len : 0;
    const int64_t base = m - i;  // the sequence's first token
    const int64_t jlo = live ? (i - a.window > 0 ? i - a.window : 0) : 1;
    const int64_t jhi = live ? (i + a.window < a.seq_len - 1 ? i + a.window : a.seq_len - 1) : 0;
    float mx = -INFINITY, l = 0.0f, acc[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) acc[e] = 0.0f;
    // keys in batches of kKB: the batch's rows are loaded together (one
    // round trip), rows past the window's end re-read its last row and get
    // no weight; the loop bounds are uniform across the token's 16 lanes
    constexpr int kKB = 8;  // the reference window (w = 3, 7 keys) in one batch
    for (int64_t j = jlo; j <= jhi; j += kKB) {
      float kv[kKB][EPT], s[kKB];
#pragma unroll
      for (int c = 0; c < kKB; ++c) {
        const int64_t jj = j + c <= jhi ? j + c : jhi;
        load_row<EPT>(a.src + (base + jj) * D + d0, kv[c]);
      }
#pragma unroll
      for (int c = 0; c < kKB; ++c) {
        float t = 0.0f;
#pragma unroll
        for (int e = 0; e < EPT; ++e) t = fmaf(x[e], kv[c][e], t);
        s[c] = t;
      }
      float mn = mx;
#pragma unroll
      for (int c = 0; c < kKB; ++c) {
        const float t = sum16(s[c]) * a.scale;
        s[c] = j + c <= jhi ? t : -INFINITY;
        mn = fmaxf(mn, s[c]);
      }
      const float cf = expf(mx - mn);
      l *= cf;
#pragma unroll
      for (int e = 0; e < EPT; ++e) acc[e] *= cf;
#pragma unroll
      for (int c = 0; c < kKB; ++c) {
        const float p = expf(s[c] - mn);  // 0 for the batch's padding
        l += p;
#pragma unroll
        for (int e = 0; e < EPT; ++e) acc[e] = fmaf(p, kv[c][e], acc[e]);
      }
      mx = mn;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; ++e) h[e] = x[e] + acc[e] * inv;
  }
  layer_norm<EPT, D>(h, g1, be1, a.eps);
  store_row<EPT>(xs + r * G::XS + d0, h);
  __syncthreads();

  const int lr = lane & 15, lg = lane >> 4;

  // ---- 2. linear1 + bias + ReLU: wave wv, hidden units [wv*D, (wv+1)*D)
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const int col = wv * D + ct * 16 + lr;
    const float* wrow = a.w1 + (int64_t)col * D;
    float4 bv[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) bv[t] = *reinterpret_cast<const float4*>(wrow + 16 * t + 4 * lg);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float4 av = *reinterpret_cast<const float4*>(xs + lr * G::XS + 16 * t + 4 * lg);
      acc = mfma_f32(av.x, bv[t].x, acc);
      acc = mfma_f32(av.y, bv[t].y, acc);
      acc = mfma_f32(av.z, bv[t].z, acc);
      acc = mfma_f32(av.w, bv[t].w, acc);
    }
    const float bias = a.bi1[col];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) zs[(4 * lg + jj) * G::ZS + col] = fmaxf(acc[jj] + bias, 0.0f);
  }
  __syncthreads();

  // ---- 3. linear2: wave wv contracts hidden units [wv*D, (wv+1)*D) for every column
  f32x4 part[NT];
#pragma unroll
  for (int ct = 0; ct < NT; ++ct) {
    const int col = ct * 16 + lr;
    const float* wrow = a.w2 + (int64_t)col * F + wv * D;
    float4 bv[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) bv[t] = *reinterpret_cast<const float4*>(wrow + 16 * t + 4 * lg);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float4 av = *reinterpret_cast<const float4*>(zs + lr * G::ZS + wv * D + 16 * t + 4 * lg);
      acc = mfma_f32(av.x, bv[t].x, acc);
      acc = mfma_f32(av.y, bv[t].y, acc);
      acc = mfma_f32(av.z, bv[t].z, acc);
      acc = mfma_f32(av.w, bv[t].w, acc);
    }
    part[ct] = acc;
  }
  __syncthreads();  // every wave is done reading zs: its space takes the partial sums
  float* ps = zs;
#pragma unroll
  for (int ct = 0; ct < NT; ++ct)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) ps[(wv * 16 + 4 * lg + jj) * G::PS + ct * 16 + lr] = part[ct][jj];
  __syncthreads();

  // ---- 4. residual + bias, LayerNorm2, store
  float y[EPT], p0[EPT], p1[EPT], p2[EPT], p3[EPT];
  load_row<EPT>(ps + (0 * 16 + r) * G::PS + d0, p0);
  load_row<EPT>(ps + (1 * 16 + r) * G::PS + d0, p1);
  load_row<EPT>(ps + (2 * 16 + r) * G::PS + d0, p2);
  load_row<EPT>(ps + (3 * 16 + r) * G::PS + d0, p3);
#pragma unroll
  for (int e = 0; e < EPT; ++e) y[e] = h[e] + ((((p0[e] + p1[e]) + p2[e]) + p3[e]) + b2[e]);
  layer_norm<EPT, D>(y, g2, be2, a.eps);
  if (live) store_row<EPT>(a.out + m * D + d0, y);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool overlaps(const void* a, const void* b, size_t bytes) {
  const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
  return x < y + bytes && y < x + bytes;
}

int fail(const char* fmt, long long v = 0) {
  char buf[256];
  snprintf(buf, sizeof(buf), fmt, v);
  return ma_host::set_error(buf);
}

}  // namespace

extern "C" int ma_encoder_layer_forward(const ma_encoder_layer* L, const float* src, const float* attn, float* out,
                                        void* stream) {
  ma_host::clear_error();
  if (!L) return fail("ma_encoder_layer_forward: null layer");
  const int64_t D = L->d_model;
  if (D != 16 && D != 32 && D != 64 && D != 128)
    return fail("ma_encoder_layer_forward: d_model %lld unsupported (16, 32, 64 or 128)", (long long)D);
  if (L->d_ff != 4 * D) return fail("ma_encoder_layer_forward: d_ff must be 4 * d_model (got %lld)", (long long)L->d_ff);
  if (L->batch < 0 || L->seq_len < 0) return fail("ma_encoder_layer_forward: negative batch or seq_len");
  if (L->seq_len > (int64_t)INT32_MAX) return fail("ma_encoder_layer_forward: seq_len exceeds int32 range");
  if (!(L->ln_eps > 0.0f) || std::isinf(L->ln_eps)) return fail("ma_encoder_layer_forward: ln_eps must be finite and > 0");
  const int64_t rows = L->batch * L->seq_len;
  if (rows == 0) return 0;
  const int64_t wgs = (rows + kTokens - 1) / kTokens;
  if (wgs > (int64_t)INT32_MAX) return fail("ma_encoder_layer_forward: too many tokens for one launch");
  const void* ptrs[] = {src, out, L->norm1_weight, L->norm1_bias, L->linear1_weight, L->linear1_bias,
                        L->linear2_weight, L->linear2_bias, L->norm2_weight, L->norm2_bias};
  for (const void* p : ptrs)
    if (!p || !aligned16(p)) return fail("ma_encoder_layer_forward: null or non-16-byte-aligned pointer");
  if (attn && !aligned16(attn)) return fail("ma_encoder_layer_forward: attn is not 16-byte aligned");
  const size_t bytes = (size_t)rows * (size_t)D * sizeof(float);
  if (overlaps(out, src, bytes) || (attn && overlaps(out, attn, bytes)))
    return fail("ma_encoder_layer_forward: out overlaps src or attn");
  EncArgs a;
  a.src = src;
  a.attn = attn;
  a.out = out;
  a.g1 = L->norm1_weight;
  a.be1 = L->norm1_bias;
  a.w1 = L->linear1_weight;
  a.bi1 = L->linear1_bias;
  a.w2 = L->linear2_weight;
  a.bi2 = L->linear2_bias;
  a.g2 = L->norm2_weight;
  a.be2 = L->norm2_bias;
  a.rows = rows;
  a.seq_len = (int32_t)L->seq_len;
  a.window = (int32_t)(L->window < 0 ? -1 : (L->window > L->seq_len ? L->seq_len : L->window));
  a.scale = 1.0f / std::sqrt(static_cast<float>(D));  // as src/csrc/ma_core.cpp:188 for head_dim = d_model
  a.eps = L->ln_eps;
  hipStream_t st = static_cast<hipStream_t>(stream);
  (void)hipGetLastError();
  const dim3 grid((unsigned)wgs), block(256);
  switch (D) {
    case 16: hipLaunchKernelGGL(encoder_layer_kernel<16>, grid, block, 0, st, a); break;
    case 32: hipLaunchKernelGGL(encoder_layer_kernel<32>, grid, block, 0, st, a); break;
    case 64: hipLaunchKernelGGL(encoder_layer_kernel<64>, grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL(encoder_layer_kernel<128>, grid, block, 0, st, a); break;
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ma_host::set_error(hipGetErrorString(e));
  return 0;
}
