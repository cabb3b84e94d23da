// backward_kernel.h -- MFMA backward of banded attention (SLIDING with any
// dilation, DENSE and causal as the band [i-(N-1), i+R]), head_dim 64,
// bf16/fp16.
//
// With s_ij = q_i.k_j (raw), p_ij = exp2(s_ij*scale*log2e - lse2_i),
// dp_ij = dout_i.v_j and ds_ij = p_ij (dp_ij - delta_i):
//   dq_i = scale * sum_j ds_ij k_j,   dk_j = scale * sum_i ds_ij q_i,
//   dv_j = sum_i p_ij dout_i,         delta_i = sum_j p_ij dp_ij
// (the reference's backward kernel, src/cuda/sparse_attention_kernel.cu:
// 265-346, with its s_dot = delta).  Two launches, both one workgroup (4
// waves x 16 rows) per 64-row tile of one (batch, head, residue class), the
// band's 64-row blocks of the other operand streaming through a two-buffer
// LDS ring with the next block in flight into registers:
//
// bwd_q_kernel   query tile.  Each key block is staged as (K rows, K^T) and
//   (V rows, V^T) -- the 16-bit stream layout with K or V in both parts.
//   Pass 1 over the band: S^T = K Q^T and dP^T = V dO^T on 16x16x32 MFMA,
//   online max / sum / sum(e * dp), giving lse2 and delta with no O.  Pass 2
//   over the same blocks: dS^T from registers, dQ^T += K^T dS^T (pv2).
//   Writes dq and the per-row {lse2, delta}.
// bwd_kv_kernel  key tile, after bwd_q_kernel.  Each query block is staged
//   as (Q rows, Q^T), (dO rows, dO^T) and its 64 {lse2, delta}.  S = Q K^T
//   and dP = dO V^T with the tile's K, V rows as the register operand (the
//   MFMA output lands as lane (key c, group g) holding queries 4g..4g+3,
//   which is the B operand of the next products); dV^T += dO^T P and
//   dK^T += Q^T dS (pv2).  No atomics: each output row has one writer.
//
// Every load and store is a range-checked buffer operation on the residue
// class, unconditional (out-of-range rows read zero, stores are dropped).
#pragma once

#include "stream_kernel.h"

namespace ma_dev {

struct BwdArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  float* stats;  // [B*N*H][2] {lse2, delta} per token row (lse2: log2 units of the scaled scores)
  int64_t N, H;
  int32_t left, right, dil;  // band [m-left, m+right] on a residue class; left, right >= 0
  int32_t tiles;             // 64-row tiles of the longest residue class
  int32_t tok_bytes;         // bytes between consecutive rows of a residue class
  float scale, scale_log2;
};

// Workgroup -> (b, h, rho, tile) and the residue class's resources.
struct BwdTile {
  int b, h, rho, t, Nr, nblk;
  uint32_t tb;
  int64_t base;  // element offset of class row 0
  uint32_t nrec;
};

template <class P>
__device__ __forceinline__ bool bwd_tile(const BwdArgs& a, BwdTile& w) {
  int lin = blockIdx.x;
  w.t = lin % a.tiles;
  lin /= a.tiles;
  w.rho = lin % a.dil;
  lin /= a.dil;
  w.h = lin % (int)a.H;
  w.b = lin / (int)a.H;
  w.Nr = (int)((a.N - w.rho + a.dil - 1) / a.dil);
  w.nblk = (w.Nr + 63) >> 6;
  w.tb = (uint32_t)a.tok_bytes;
  w.base = (((int64_t)w.b * a.N + w.rho) * a.H + w.h) * kHeadDim;
  w.nrec = (uint32_t)((int64_t)(w.Nr - 1) * w.tb + kHeadDim * sizeof(typename P::Elt));
  return 64 * w.t < w.Nr;
}

// Mask of one 16x16 product: element r of lane (c, g) pairs rows whose
// key - query offset plus left is x + SGN*r (x per lane, see the callers),
// and whose streamed row (key in bwd_q_kernel, query in bwd_kv_kernel) is
// idx0 + r; kept iff the offset lies in [-left, right] and that row is below
// lim.
template <int SGN>
__device__ __forceinline__ void bwd_mask(f32x4& z, int x, int span, int idx0, int lim) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
    z[r] = (uint32_t)(x + SGN * r) <= (uint32_t)span && idx0 + r < lim ? z[r] : -INFINITY;
}

template <class P>
__global__ __launch_bounds__(256, 2) void bwd_q_kernel(BwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // 2 buffers x (K slot, V slot)
  using Elt = typename P::Elt;
  constexpr int kBuf = 2 * P::kSlot;
  BwdTile w;
  if (!bwd_tile<P>(a, w)) return;  // uniform, before any barrier
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  const int L = a.left, R = a.right;
  const uint32_t tb = w.tb;

  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const Elt*>(a.dout) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t DQr = make_rsrc(static_cast<Elt*>(a.dq) + w.base, w.nrec);

  const int q0 = 64 * w.t + 16 * wv;  // this wave's first query row
  const uint32_t qrow = (uint32_t)(q0 + c) * tb;
  typename P::Q qr, gr;
  P::load_q(qr, Qr, qrow, g);
  P::load_q(gr, Gr, qrow, g);
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);

  // key blocks of the band of this tile's queries
  const int kb_lo = max(floordiv32(64 * w.t - L, 64), 0);
  const int kb_hi = min(floordiv32(64 * w.t + 63 + R, 64), w.nblk - 1);
  const int nb = kb_hi - kb_lo + 1;
  const int items = 2 * nb;  // pass 1, then pass 2 over the same blocks
  auto blk_of = [&](int e) { return kb_lo + (e < nb ? e : e - nb); };
  auto off_of = [&](int e) { return e < items ? (uint32_t)(64 * blk_of(e)) * tb : kOob; };

  typename P::Slot xk, xv;
  P::load_slot(xk, Kr, Kr, off_of(0), tid, tb);
  P::load_slot(xv, Vr, Vr, off_of(0), tid, tb);
  P::store_slot(xk, ring, tid);
  P::store_slot(xv, ring + P::kSlot, tid);
  __syncthreads();

  const float sl2 = a.scale_log2;
  const int span = L + R;
  const int dl = 4 * g - c + L;  // key - query + L of element 0, minus the sub-tile base
  float m_run = -INFINITY, l_run = 0.0f, a_run = 0.0f, lse2 = 0.0f, dlt = 0.0f;
  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int e = 0; e < items; ++e) {
    P::load_slot(xk, Kr, Kr, off_of(e + 1), tid, tb);
    P::load_slot(xv, Vr, Vr, off_of(e + 1), tid, tb);
    const uint8_t* sk = ring + (e & 1) * kBuf;
    const uint8_t* sv = sk + P::kSlot;
    const int key0 = 64 * blk_of(e);
    f32x4 s[4], dp[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      s[u] = P::qk(sk + P::k_sub(u) + kl, qr);
      dp[u] = P::qk(sv + P::k_sub(u) + kl, gr);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int rel = key0 + 16 * u - q0;  // key - query offsets span [rel-15, rel+15]
      if (rel - 15 < -L || rel + 15 > R || key0 + 16 * u + 15 >= w.Nr)
        bwd_mask<1>(s[u], dl + rel, span, key0 + 16 * u + 4 * g, w.Nr);
    }
    if (e < nb) {  // pass 1: online max, sum of e and of e * dp
      float mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < 4; ++u) mx = fmaxf(mx, fmaxf(fmaxf(s[u][0], s[u][1]), fmaxf(s[u][2], s[u][3])));
      const float m_new = fmaxf(m_run, col_max(mx));
      const float m_use = m_new == -INFINITY ? 0.0f : m_new * sl2;
      const float corr = __builtin_amdgcn_exp2f(m_run * sl2 - m_use);
      l_run *= corr;
      a_run *= corr;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float ex = __builtin_amdgcn_exp2f(fmaf(s[u][r], sl2, -m_use));
          l_run += ex;
          a_run = fmaf(ex, dp[u][r], a_run);
        }
      m_run = m_new;
      if (e == nb - 1) {  // every query sees its own key (left, right >= 0): l_tot > 0
        const float l_tot = col_sum(l_run);
        lse2 = m_use + __log2f(l_tot);
        dlt = col_sum(a_run) / l_tot;
      }
    } else {  // pass 2: dS^T in registers, dQ^T += K^T dS^T
#pragma unroll
      for (int u = 0; u < 4; u += 2) {
        float d0[4], d1[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          d0[r] = __builtin_amdgcn_exp2f(fmaf(s[u][r], sl2, -lse2)) * (dp[u][r] - dlt);
          d1[r] = __builtin_amdgcn_exp2f(fmaf(s[u + 1][r], sl2, -lse2)) * (dp[u + 1][r] - dlt);
        }
        P::pv2(sk + P::v_sub(u) + vl, sk + P::v_sub(u + 1) + vl, d0, d1, acc);
      }
    }
    // the next item goes into the buffer item e-1 used (every wave passed the
    // barrier that ended item e-1)
    P::store_slot(xk, ring + ((e + 1) & 1) * kBuf, tid);
    P::store_slot(xv, ring + ((e + 1) & 1) * kBuf + P::kSlot, tid);
    __syncthreads();
  }
  P::store_o(acc, a.scale, DQr, qrow, g);
  // {lse2, delta} of query q0 + c, one lane per query
  const int64_t srow = (((int64_t)w.b * a.N + w.rho + (int64_t)a.dil * (q0 + c)) * a.H + w.h);
  if (g == 0 && q0 + c < w.Nr) *reinterpret_cast<float2*>(a.stats + 2 * srow) = make_float2(lse2, dlt);
}

template <class P>
__global__ __launch_bounds__(256, 2) void bwd_kv_kernel(BwdArgs a) {
  // 2 buffers x (Q slot, dO slot, 64 lse2, 64 delta)
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
  using Elt = typename P::Elt;
  constexpr int kBuf = 2 * P::kSlot + 512;
  BwdTile w;
  if (!bwd_tile<P>(a, w)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;
  const int L = a.left, R = a.right;
  const uint32_t tb = w.tb;

  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const Elt*>(a.dout) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t DKr = make_rsrc(static_cast<Elt*>(a.dk) + w.base, w.nrec);
  const __amdgpu_buffer_rsrc_t DVr = make_rsrc(static_cast<Elt*>(a.dv) + w.base, w.nrec);
  // statistics of the class: row m at float2 index m * dil * H
  const int64_t sbase = ((int64_t)w.b * a.N + w.rho) * a.H + w.h;
  const uint32_t sstride = (uint32_t)(a.dil * a.H) * 8u;
  const __amdgpu_buffer_rsrc_t Sr = make_rsrc(a.stats + 2 * sbase, (uint32_t)(w.Nr - 1) * sstride + 8u);

  const int k0 = 64 * w.t + 16 * wv;  // this wave's first key row
  const uint32_t krow = (uint32_t)(k0 + c) * tb;
  typename P::Q kr, vr;
  P::load_q(kr, Kr, krow, g);
  P::load_q(vr, Vr, krow, g);
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);

  // query blocks whose band reaches this tile's keys: queries [key-R, key+L]
  const int qb_lo = max(floordiv32(64 * w.t - R, 64), 0);
  const int qb_hi = min(floordiv32(64 * w.t + 63 + L, 64), w.nblk - 1);
  const int nb = qb_hi - qb_lo + 1;
  auto off_of = [&](int e) { return e < nb ? (uint32_t)(64 * (qb_lo + e)) * tb : kOob; };
  // thread tid < 64 carries the statistics of query row tid of the block
  auto stat_off = [&](int e) { return e < nb && tid < 64 ? (uint32_t)(64 * (qb_lo + e) + tid) * sstride : kOob; };

  typename P::Slot xq, xg;
  uint2 xs;
  P::load_slot(xq, Qr, Qr, off_of(0), tid, tb);
  P::load_slot(xg, Gr, Gr, off_of(0), tid, tb);
  xs = bload8(Sr, stat_off(0));
  auto stage = [&](uint8_t* buf) {
    P::store_slot(xq, buf, tid);
    P::store_slot(xg, buf + P::kSlot, tid);
    if (tid < 64) {
      float* st = reinterpret_cast<float*>(buf + 2 * P::kSlot);
      st[tid] = __uint_as_float(xs.x);       // lse2
      st[64 + tid] = __uint_as_float(xs.y);  // delta
    }
  };
  stage(ring);
  __syncthreads();

  const float sl2 = a.scale_log2;
  const int span = L + R;
  const int dl = c - 4 * g + L;  // key - query + L of element 0, minus the sub-tile base
  f32x4 acc_k[4], acc_v[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc_k[dt] = acc_v[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int e = 0; e < nb; ++e) {
    P::load_slot(xq, Qr, Qr, off_of(e + 1), tid, tb);
    P::load_slot(xg, Gr, Gr, off_of(e + 1), tid, tb);
    xs = bload8(Sr, stat_off(e + 1));
    const uint8_t* sq = ring + (e & 1) * kBuf;
    const uint8_t* sg = sq + P::kSlot;
    const float* st = reinterpret_cast<const float*>(sq + 2 * P::kSlot);
    const int qbase = 64 * (qb_lo + e);
    f32x4 s[4], dp[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      s[u] = P::qk(sq + P::k_sub(u) + kl, kr);   // S[query 16u+4g+r][key c]
      dp[u] = P::qk(sg + P::k_sub(u) + kl, vr);  // dP[query][key c]
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int rel = k0 - (qbase + 16 * u);  // key - query offsets span [rel-15, rel+15]
      if (rel - 15 < -L || rel + 15 > R || qbase + 16 * u + 15 >= w.Nr)
        bwd_mask<-1>(s[u], dl + rel, span, qbase + 16 * u + 4 * g, w.Nr);
    }
#pragma unroll
    for (int u = 0; u < 4; u += 2) {
      const f32x4 lse0 = *reinterpret_cast<const f32x4*>(st + 16 * u + 4 * g);
      const f32x4 dl0 = *reinterpret_cast<const f32x4*>(st + 64 + 16 * u + 4 * g);
      const f32x4 lse1 = *reinterpret_cast<const f32x4*>(st + 16 * (u + 1) + 4 * g);
      const f32x4 dl1 = *reinterpret_cast<const f32x4*>(st + 64 + 16 * (u + 1) + 4 * g);
      float p0[4], p1[4], d0[4], d1[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p0[r] = __builtin_amdgcn_exp2f(fmaf(s[u][r], sl2, -lse0[r]));
        p1[r] = __builtin_amdgcn_exp2f(fmaf(s[u + 1][r], sl2, -lse1[r]));
        d0[r] = p0[r] * (dp[u][r] - dl0[r]);
        d1[r] = p1[r] * (dp[u + 1][r] - dl1[r]);
      }
      P::pv2(sg + P::v_sub(u) + vl, sg + P::v_sub(u + 1) + vl, p0, p1, acc_v);  // dV^T += dO^T P
      P::pv2(sq + P::v_sub(u) + vl, sq + P::v_sub(u + 1) + vl, d0, d1, acc_k);  // dK^T += Q^T dS
    }
    stage(ring + ((e + 1) & 1) * kBuf);
    __syncthreads();
  }
  P::store_o(acc_v, 1.0f, DVr, krow, g);
  P::store_o(acc_k, a.scale, DKr, krow, g);
}

}  // namespace ma_dev
