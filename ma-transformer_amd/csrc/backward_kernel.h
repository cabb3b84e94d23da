// backward_kernel.h -- MFMA backward of banded attention (SLIDING with any
// dilation, DENSE and causal as the band [i-(N-1), i+R]), head_dim 64,
// bf16/fp16 (16x16x32 MFMA) and fp32 (16x16x4 MFMA; 64-row blocks of two
// 32-row fp32 slots).
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
// bwd_q_kernel   query tile.  Each key block is staged as K and V rows in one
//   slot; K^T comes from the K rows (16-bit: the LDS transpose read; fp32:
//   16-byte reads of the column-permuted rows).
//   Pass 1 over the band: S^T = K Q^T and dP^T = V dO^T on 16x16x32 MFMA,
//   online max / sum / sum(e * dp), giving lse2 and delta with no O.  Pass 2
//   over the same blocks: dS^T from registers, dQ^T += K^T dS^T (pv2).
//   Writes dq and the per-row {lse2, delta}.
// bwd_kv_kernel  key tile, after bwd_q_kernel.  Each query block is staged
//   as Q and dO rows in one slot (Q^T, dO^T read from them) and its 64
//   {lse2, delta}.  S = Q K^T
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
  int32_t chunk, chunks;     // stream kernels: tiles per workgroup, workgroups per residue class
  const float* lse;          // bwd_q_kernel<SAVED>: the forward's row statistics (store_lse), [B*N*H]
  const void* fo;            // bwd_q_kernel<SAVED>: the forward's O (delta = dO . O)
};

// LDS of one streamed block in the backward passes: two matrices (K and V
// for dQ, Q and dO for dK/dV) in one block buffer, the first in the slots'
// first halves, the second in their second halves; a matrix read transposed
// is read from the same rows (16-bit: tr_read; fp32: permuted columns).
// kRows2: the second matrix's rows relative to the first's; kT1 / kT2: the
// transposed operand of the first / second matrix, relative to buffer +
// blk_v(u) + v_lane.
template <class P>
struct PairLds {
  static constexpr int kBytes = P::kBlk;
  static constexpr int kRows2 = P::kSlotK;
  static constexpr int kT1 = -P::kSlotK;
  static constexpr int kT2 = 0;
};

// A block's two matrices in flight into registers, and their store into a
// PairLds buffer: dQ pass (K read as rows and transposed, V as rows) and
// dK/dV pass (Q and dO, each read as rows and transposed).
template <class P>
struct KvRegs {
  BlkSlots<P> k;
};
template <class P>
__device__ __forceinline__ void kv_load(KvRegs<P>& x, __amdgpu_buffer_rsrc_t Kr, __amdgpu_buffer_rsrc_t Vr,
                                        uint32_t off, int tid, uint32_t tb) {
  load_blk<P>(x.k, Kr, Vr, off, tid, tb);
}
template <class P>
__device__ __forceinline__ void kv_store(const KvRegs<P>& x, uint8_t* buf, int tid) {
  store_blk<P>(x.k, buf, tid);
}
template <class P>
using QgRegs = KvRegs<P>;
template <class P>
__device__ __forceinline__ void qg_load(QgRegs<P>& x, __amdgpu_buffer_rsrc_t Qr, __amdgpu_buffer_rsrc_t Gr,
                                        uint32_t off, int tid, uint32_t tb) {
  load_blk<P>(x.k, Qr, Gr, off, tid, tb);
}
template <class P>
__device__ __forceinline__ void qg_store(const QgRegs<P>& x, uint8_t* buf, int tid) {
  store_blk<P>(x.k, buf, tid);
}

// Workgroup -> (b, h, rho, tile) and the residue class's resources.
struct BwdTile {
  int b, h, rho, t, Nr, nblk;
  uint32_t tb;
  int64_t base;  // element offset of class row 0
  uint32_t nrec;
};

// Ids are XCD-contiguous (xcd_row_order): an XCD runs whole heads' tiles,
// so the head's streamed rows, which every tile of the head reads, meet in
// its L2.  rev: tiles in descending order, for passes whose work grows with
// the tile (dQ of a band with a long left side: the longest tiles start
// first instead of forming the launch's tail).
template <class P>
__device__ __forceinline__ bool bwd_tile(const BwdArgs& a, BwdTile& w, bool rev = false) {
  int lin = xcd_row_order((int)blockIdx.x, (int)gridDim.x);
  w.t = rev ? a.tiles - 1 - lin % a.tiles : lin % a.tiles;
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
// idx0 + r; kept iff the offset lies in [-left, right] and that row lies in
// [0, lim) (stream kernels' first block may start before row 0).
template <int SGN>
__device__ __forceinline__ void bwd_mask(f32x4& z, int x, int span, int idx0, int lim) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
    z[r] = (uint32_t)(x + SGN * r) <= (uint32_t)span && (uint32_t)(idx0 + r) < (uint32_t)lim ? z[r] : -INFINITY;
}

// ---------------------------------------------------------------- per-block work
//
// One 64-row block of the streamed operand against this wave's 16 rows.

// Scores S^T = K Q^T and dP^T = V dO^T of one key block (sk: (K, K^T) slot,
// sv: V rows) for this wave's queries q0..q0+15, masked to the band.
// Returns the wave-uniform mask of live sub-tiles: a sub-tile with no key in
// any of the 16 queries' bands (or past the end) is not computed (scores
// -inf, dP 0), and the passes below skip it.
template <class P>
__device__ __forceinline__ int bwdq_scores(const uint8_t* sk, const uint8_t* sv, uint32_t kl, const typename P::Q& qr,
                                           const typename P::Q& gr, int key0, int q0, int L, int R, int dl, int g,
                                           int Nr, f32x4 (&s)[4], f32x4 (&dp)[4]) {
  int live = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int rel = key0 + 16 * u - q0;  // key - query offsets span [rel-15, rel+15]
    if (rel + 15 < -L || rel - 15 > R || key0 + 16 * u >= Nr || key0 + 16 * u + 15 < 0) {
      s[u] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      dp[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      continue;
    }
    live |= 1 << u;
    s[u] = P::qk(sk + P::blk_k(u) + kl, qr);
    dp[u] = P::qk(sv + P::blk_k(u) + kl, gr);
    if (rel - 15 < -L || rel + 15 > R || key0 + 16 * u + 15 >= Nr || key0 + 16 * u < 0)
      bwd_mask<1>(s[u], dl + rel, L + R, key0 + 16 * u + 4 * g, Nr);
  }
  return live;
}

// Pass 1: online max (m_run, raw scores), sum of e = exp2(s*sl2 - m) and of
// e*dp over the live sub-tiles.
__device__ __forceinline__ void bwdq_pass1(const f32x4 (&s)[4], const f32x4 (&dp)[4], int live, float sl2,
                                           float& m_run, float& l_run, float& a_run) {
  if (!live) return;  // uniform
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < 4; ++u) mx = fmaxf(mx, fmaxf(fmaxf(s[u][0], s[u][1]), fmaxf(s[u][2], s[u][3])));
  const float m_new = fmaxf(m_run, col_max(mx));
  const float m_use = m_new == -INFINITY ? 0.0f : m_new * sl2;
  const float corr = __builtin_amdgcn_exp2f(m_run * sl2 - m_use);
  l_run *= corr;
  a_run *= corr;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (!(live >> u & 1)) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float ex = __builtin_amdgcn_exp2f(fmaf(s[u][r], sl2, -m_use));
      l_run += ex;
      a_run = fmaf(ex, dp[u][r], a_run);
    }
  }
  m_run = m_new;
}

// lse2 and delta of the wave's queries once pass 1 has seen the whole band
// (every query sees its own key: left, right >= 0, so the sum is positive).
__device__ __forceinline__ void bwdq_stats(float m_run, float l_run, float a_run, float sl2, float& lse2,
                                           float& dlt) {
  const float l_tot = col_sum(l_run);
  lse2 = (m_run == -INFINITY ? 0.0f : m_run * sl2) + __log2f(l_tot);
  dlt = col_sum(a_run) / l_tot;
}

// Pass 2: dS^T in registers, dQ^T += K^T dS^T (sk's K^T part), pairs of
// sub-tiles with a live one.
template <class P>
__device__ __forceinline__ void bwdq_pass2(const uint8_t* sk, uint32_t vl, const f32x4 (&s)[4], const f32x4 (&dp)[4],
                                           int live, float sl2, float lse2, float dlt, f32x4 (&acc)[4]) {
#pragma unroll
  for (int u = 0; u < 4; u += 2) {
    if (!(live >> u & 3)) continue;  // uniform
    float d0[4], d1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      d0[r] = __builtin_amdgcn_exp2f(fmaf(s[u][r], sl2, -lse2)) * (dp[u][r] - dlt);
      d1[r] = __builtin_amdgcn_exp2f(fmaf(s[u + 1][r], sl2, -lse2)) * (dp[u + 1][r] - dlt);
    }
    P::pv2(sk + P::blk_v(u) + vl, sk + P::blk_v(u + 1) + vl, d0, d1, acc);
  }
}

// One query block (PairLds buffer sq: Q, dO; sg: the dO rows; st: 64 lse2
// then 64 delta) against this wave's keys k0..k0+15 (kr, vr: their K and V
// rows): dV^T += dO^T P and dK^T += Q^T dS (Q^T, dO^T reads at lane offsets
// vq, vg from sq + blk_v(u)).
template <class P>
__device__ __forceinline__ void bwdkv_block(const uint8_t* sq, const uint8_t* sg, const float* st, uint32_t kl,
                                            uint32_t vq, uint32_t vg, const typename P::Q& kr, const typename P::Q& vr,
                                            int qbase,
                                            int k0, int L, int R, int dl, int g, int Nr, float sl2,
                                            f32x4 (&acc_k)[4], f32x4 (&acc_v)[4]) {
  // sub-tiles whose 16 queries have no band overlap with the wave's 16 keys
  // (or lie past the end) are not computed; pairs with no live sub-tile are
  // skipped (wave-uniform tests)
  f32x4 s[4], dp[4];
  int live = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int rel = k0 - (qbase + 16 * u);  // key - query offsets span [rel-15, rel+15]
    if (rel + 15 < -L || rel - 15 > R || qbase + 16 * u >= Nr || qbase + 16 * u + 15 < 0) {
      s[u] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      dp[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      continue;
    }
    live |= 1 << u;
    s[u] = P::qk(sq + P::blk_k(u) + kl, kr);   // S[query 16u+4g+r][key c]
    dp[u] = P::qk(sg + P::blk_k(u) + kl, vr);  // dP[query][key c]
    if (rel - 15 < -L || rel + 15 > R || qbase + 16 * u + 15 >= Nr || qbase + 16 * u < 0)
      bwd_mask<-1>(s[u], dl + rel, L + R, qbase + 16 * u + 4 * g, Nr);
  }
#pragma unroll
  for (int u = 0; u < 4; u += 2) {
    if (!(live >> u & 3)) continue;
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
    P::pv2(sq + P::blk_v(u) + vg, sq + P::blk_v(u + 1) + vg, p0, p1, acc_v);  // dV^T += dO^T P
    P::pv2(sq + P::blk_v(u) + vq, sq + P::blk_v(u + 1) + vq, d0, d1, acc_k);  // dK^T += Q^T dS
  }
}

// Query block's statistics staged by threads 0..63 (row tid of the block).
__device__ __forceinline__ void bwd_stage_stats(uint8_t* st, uint2 xs, int tid) {
  if (tid < 64) {
    float* f = reinterpret_cast<float*>(st);
    f[tid] = __uint_as_float(xs.x);       // lse2
    f[64 + tid] = __uint_as_float(xs.y);  // delta
  }
}

// Statistics of a residue class: row m at float2 index m * dil * H.
struct BwdStats {
  __amdgpu_buffer_rsrc_t r;
  uint32_t stride;
};

__device__ __forceinline__ BwdStats bwd_stats_rsrc(const BwdArgs& a, int b, int h, int rho, int Nr) {
  const int64_t sbase = ((int64_t)b * a.N + rho) * a.H + h;
  BwdStats st;
  st.stride = (uint32_t)(a.dil * a.H) * 8u;
  st.r = make_rsrc(a.stats + 2 * sbase, (uint32_t)(Nr - 1) * st.stride + 8u);
  return st;
}

// dot(x, y) of one row over the head_dim values this lane holds, both in the
// Q register layout of P (their sum over the row's four lane groups is the
// row's dot product).
template <class P>
__device__ __forceinline__ float bwd_row_dot(const typename P::Q& x, const typename P::Q& y) {
  float d = 0.0f;
  if constexpr (P::kSPB == 1) {
    using T = typename P::Elt;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t wx[4] = {x.r[h].x, x.r[h].y, x.r[h].z, x.r[h].w};
      const uint32_t wy[4] = {y.r[h].x, y.r[h].y, y.r[h].z, y.r[h].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        d = fmaf(static_cast<float>(__builtin_bit_cast(T, (uint16_t)(wx[j] & 0xffffu))),
                 static_cast<float>(__builtin_bit_cast(T, (uint16_t)(wy[j] & 0xffffu))), d);
        d = fmaf(static_cast<float>(__builtin_bit_cast(T, (uint16_t)(wx[j] >> 16))),
                 static_cast<float>(__builtin_bit_cast(T, (uint16_t)(wy[j] >> 16))), d);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 xv = __builtin_bit_cast(f32x4, x.r[j]), yv = __builtin_bit_cast(f32x4, y.r[j]);
#pragma unroll
      for (int r = 0; r < 4; ++r) d = fmaf(xv[r], yv[r], d);
    }
  }
  return d;
}

// ---------------------------------------------------------------- one tile per workgroup

// SAVED: from the forward's statistics (lse, and delta = dO . O of the row):
// pass 2 only.
template <class P, bool SAVED>
__global__ __launch_bounds__(256, 2) void bwd_q_kernel(BwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // 2 buffers x PairLds (K, V)
  using Elt = typename P::Elt;
  using PL = PairLds<P>;
  constexpr int kBuf = PL::kBytes;
  BwdTile w;
  if (!bwd_tile<P>(a, w, a.left > a.right)) return;  // uniform, before any barrier
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

  // 64-row groups of keys from the band's first row, not from block
  // boundaries: the tile's keys [64t-L, 64t+63+R] take ceil((64+L+R)/64)
  // groups (2 for [i-32, i+31], which straddles 3 aligned blocks)
  const int key_lo = max(64 * w.t - L, 0);
  const int key_hi = min(64 * w.t + 63 + R, w.Nr - 1);
  const int nb = (key_hi - key_lo) / 64 + 1;
  const int items = SAVED ? nb : 2 * nb;  // pass 1, then pass 2 over the same blocks
  // A band of at most two blocks stays resident in the two buffers for pass
  // 2 (block j in buffer j); wider bands stream through them twice.
  const bool resident = nb <= 2;
  auto row_of = [&](int e) { return key_lo + 64 * (e < nb ? e : e - nb); };  // first key of item e's group
  auto buf_of = [&](int e) { return resident ? (e < nb ? e : e - nb) : (e & 1); };
  auto off_of = [&](int e) { return e < (resident ? nb : items) ? (uint32_t)row_of(e) * tb : kOob; };

  const int64_t srow = (((int64_t)w.b * a.N + w.rho + (int64_t)a.dil * (q0 + c)) * a.H + w.h);
  typename P::Q fo_row;
  float lse2 = 0.0f, dlt = 0.0f;
  if constexpr (SAVED) {
    P::load_q(fo_row, make_rsrc(static_cast<const Elt*>(a.fo) + w.base, w.nrec), qrow, g);
    if (q0 + c < w.Nr) lse2 = a.lse[srow];
  }
  KvRegs<P> xk;  // V is read only as rows (dP^T = V dO^T)
  kv_load<P>(xk, Kr, Vr, off_of(0), tid, tb);
  if constexpr (SAVED) dlt = col_sum(bwd_row_dot<P>(gr, fo_row));  // after the first block's loads are issued
  kv_store<P>(xk, ring, tid);
  __syncthreads();

  const float sl2 = a.scale_log2;
  const int dl = 4 * g - c + L;  // key - query + L of element 0, minus the sub-tile base
  float m_run = -INFINITY, l_run = 0.0f, a_run = 0.0f;
  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int e = 0; e < items; ++e) {
    kv_load<P>(xk, Kr, Vr, off_of(e + 1), tid, tb);
    const uint8_t* sk = ring + buf_of(e) * kBuf;
    f32x4 s[4], dp[4];
    const int live = bwdq_scores<P>(sk, sk + PL::kRows2, kl, qr, gr, row_of(e), q0, L, R, dl, g, w.Nr, s, dp);
    if (!SAVED && e < nb) {  // pass 1
      bwdq_pass1(s, dp, live, sl2, m_run, l_run, a_run);
      if (e == nb - 1) bwdq_stats(m_run, l_run, a_run, sl2, lse2, dlt);
    } else {  // pass 2
      bwdq_pass2<P>(sk, vl + PL::kT1, s, dp, live, sl2, lse2, dlt, acc);
    }
    // the next item goes into the buffer item e-1 used (every wave passed the
    // barrier that ended item e-1); resident bands load nothing after pass 1
    if (!resident || e + 1 < nb) kv_store<P>(xk, ring + buf_of(e + 1) * kBuf, tid);
    __syncthreads();
  }
  P::store_o(acc, a.scale, DQr, qrow, g);
  // {lse2, delta} of query q0 + c, one lane per query
  if (g == 0 && q0 + c < w.Nr) *reinterpret_cast<float2*>(a.stats + 2 * srow) = make_float2(lse2, dlt);
}

template <class P>
__global__ __launch_bounds__(256, 2) void bwd_kv_kernel(BwdArgs a) {
  // 2 buffers x (PairLds (Q, dO), 64 lse2, 64 delta)
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
  using Elt = typename P::Elt;
  using PL = PairLds<P>;
  constexpr int kBuf = PL::kBytes + 512;
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
  const BwdStats S = bwd_stats_rsrc(a, w.b, w.h, w.rho, w.Nr);

  const int k0 = 64 * w.t + 16 * wv;  // this wave's first key row
  const uint32_t krow = (uint32_t)(k0 + c) * tb;
  typename P::Q kr, vr;
  P::load_q(kr, Kr, krow, g);
  P::load_q(vr, Vr, krow, g);
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);

  // 64-row groups of queries from the first query that sees the tile's keys
  // ([64t-R, 64t+63+L]), as the key groups of bwd_q_kernel
  const int q_lo = max(64 * w.t - R, 0);
  const int q_hi = min(64 * w.t + 63 + L, w.Nr - 1);
  const int nb = (q_hi - q_lo) / 64 + 1;
  auto off_of = [&](int e) { return e < nb ? (uint32_t)(q_lo + 64 * e) * tb : kOob; };
  // thread tid < 64 carries the statistics of query row tid of the block
  auto stat_off = [&](int e) { return e < nb && tid < 64 ? (uint32_t)(q_lo + 64 * e + tid) * S.stride : kOob; };

  QgRegs<P> xq;
  qg_load<P>(xq, Qr, Gr, off_of(0), tid, tb);
  uint2 xs = bload8(S.r, stat_off(0));
  qg_store<P>(xq, ring, tid);
  bwd_stage_stats(ring + PL::kBytes, xs, tid);
  __syncthreads();

  const int dl = c - 4 * g + L;  // key - query + L of element 0, minus the sub-tile base
  f32x4 acc_k[4], acc_v[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc_k[dt] = acc_v[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int e = 0; e < nb; ++e) {
    qg_load<P>(xq, Qr, Gr, off_of(e + 1), tid, tb);
    xs = bload8(S.r, stat_off(e + 1));
    const uint8_t* sq = ring + (e & 1) * kBuf;
    bwdkv_block<P>(sq, sq + PL::kRows2, reinterpret_cast<const float*>(sq + PL::kBytes), kl, vl + PL::kT1,
                   vl + PL::kT2, kr, vr, q_lo + 64 * e, k0, L, R, dl, g, w.Nr, a.scale_log2, acc_k, acc_v);
    uint8_t* nx = ring + ((e + 1) & 1) * kBuf;
    qg_store<P>(xq, nx, tid);
    bwd_stage_stats(nx + PL::kBytes, xs, tid);
    __syncthreads();
  }
  P::store_o(acc_v, 1.0f, DVr, krow, g);
  P::store_o(acc_k, a.scale, DKr, krow, g);
}

// ---------------------------------------------------------------- fixed-window interior tiles
//
// For a fixed band [m-L, m+R] (the causal 64 window: L = 63, R = 0) an interior
// tile's geometry is compile-time, as in the forward's window_tile: a wave's
// 16 rows touch NSUB sub-tiles of 16 streamed rows at fixed offsets from its
// own (5 for causal 64, against 8 for whole 64-row blocks), and only the
// first and last need a mask.  The scores of all of them stay in registers,
// so the statistics need no online rescaling, and pass 2 reuses pass 1's
// exponentials (p = e / l) instead of recomputing exp2.

// bwd_q_stream_kernel, interior tile t: the wave's queries qa = 64t + 16wv
// against key sub-tiles s = 4t + wv - CL + j.  The kernel's blocks start at
// row 64j - 16*(CL & 3), so sub-tile s lies in block (s + (CL & 3)) >> 2, in
// ring buffer parity of that.  Gives lse2 and delta of query qa + c and dQ^T
// (unscaled).
template <class P, int L, int R>
__device__ __forceinline__ void bwdq_window_tile(const uint8_t* ring, uint32_t kl, uint32_t vl, const typename P::Q& qr,
                                                 const typename P::Q& gr, int t, int wv, int dl, float sl2,
                                                 float& lse2, float& dlt, f32x4 (&acc)[4]) {
  using G = WinGeom<L, R, 64>;
  using PL = PairLds<P>;
  constexpr int kBuf = PL::kBytes;
  constexpr int kSh = G::CL & 3;
  f32x4 e[G::NSUB], dp[G::NSUB];
  uint32_t kt[G::NSUB];  // K^T of sub-tile j (the K buffer's transposed part)
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < G::NSUB; ++j) {
    const int s = 4 * t + wv - G::CL + j + kSh;  // shifted-grid sub-tile index
    const uint32_t bb = (uint32_t)(((s >> 2) & 1) * kBuf);
    const int u = s & 3;
    kt[j] = bb + P::blk_v(u) + vl + PL::kT1;
    f32x4 z = P::qk(ring + bb + P::blk_k(u) + kl, qr);
    dp[j] = P::qk(ring + bb + PL::kRows2 + P::blk_k(u) + kl, gr);
    const int rel = 16 * (j - G::CL);     // key - query offsets span [rel-15, rel+15]
    if (rel - 15 < -L || rel + 15 > R) {  // resolved at compile time
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(dl + rel + r) <= (uint32_t)(L + R) ? z[r] : -INFINITY;
    }
    e[j] = z;
    mx = fmaxf(mx, fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3])));
  }
  const float m_use = col_max(mx) * sl2;  // finite: every query sees its own key
  float l_run = 0.0f, a_run = 0.0f;
#pragma unroll
  for (int j = 0; j < G::NSUB; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float x = __builtin_amdgcn_exp2f(fmaf(e[j][r], sl2, -m_use));
      e[j][r] = x;
      l_run += x;
      a_run = fmaf(x, dp[j][r], a_run);
    }
  const float l_tot = col_sum(l_run);
  const float inv = __builtin_amdgcn_rcpf(l_tot);
  lse2 = m_use + __log2f(l_tot);
  dlt = col_sum(a_run) * inv;
#pragma unroll
  for (int j = 0; j < G::NSUB; j += 2) {
    float d0[4], d1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) d0[r] = e[j][r] * inv * (dp[j][r] - dlt);
    if (j + 1 < G::NSUB) {  // resolved at compile time
#pragma unroll
      for (int r = 0; r < 4; ++r) d1[r] = e[j + 1][r] * inv * (dp[j + 1][r] - dlt);
      P::pv2(ring + kt[j], ring + kt[j + 1], d0, d1, acc);
    } else {
      P::pv(ring + kt[j], d0, acc);
    }
  }
}

// bwd_kv_stream_kernel, interior tile t: the wave's keys ka = 64t + 16wv
// against query sub-tiles s = 4t + wv - CR + j (the mirrored band: queries of
// key k are [k-R, k+L]).  Blocks start at row 64j - 16*(CR & 3); sub-tile s
// lies in block (s + (CR & 3)) >> 2 with its staged statistics.  dV^T and
// dK^T (unscaled) accumulate in acc_v, acc_k.
template <class P, int L, int R>
__device__ __forceinline__ void bwdkv_window_tile(const uint8_t* ring, uint32_t kl, uint32_t vl, const typename P::Q& kr,
                                                  const typename P::Q& vr, int t, int wv, int g, int dl, float sl2,
                                                  f32x4 (&acc_k)[4], f32x4 (&acc_v)[4]) {
  using G = WinGeom<R, L, 64>;
  using PL = PairLds<P>;
  constexpr int kBuf = PL::kBytes + 512;
  constexpr int kSh = G::CL & 3;
  float p[G::NSUB][4], d[G::NSUB][4];
  uint32_t qt[G::NSUB];  // Q^T of sub-tile j (dO^T at + kBlk)
#pragma unroll
  for (int j = 0; j < G::NSUB; ++j) {
    const int s = 4 * t + wv - G::CL + j + kSh;  // shifted-grid sub-tile index
    const uint32_t bb = (uint32_t)(((s >> 2) & 1) * kBuf);
    const int u = s & 3;
    qt[j] = bb + P::blk_v(u) + vl;  // + kT1: Q^T, + kT2: dO^T
    f32x4 z = P::qk(ring + bb + P::blk_k(u) + kl, kr);                  // S[query 4g+r][key c]
    const f32x4 dz = P::qk(ring + bb + PL::kRows2 + P::blk_k(u) + kl, vr);  // dP[query][key c]
    const int rel = 16 * (G::CL - j);     // key - query offsets span [rel-15, rel+15]
    if (rel - 15 < -L || rel + 15 > R) {  // resolved at compile time
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(dl + rel - r) <= (uint32_t)(L + R) ? z[r] : -INFINITY;
    }
    const float* st = reinterpret_cast<const float*>(ring + bb + PL::kBytes);
    const f32x4 lse = *reinterpret_cast<const f32x4*>(st + 16 * u + 4 * g);
    const f32x4 del = *reinterpret_cast<const f32x4*>(st + 64 + 16 * u + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[j][r] = __builtin_amdgcn_exp2f(fmaf(z[r], sl2, -lse[r]));
      d[j][r] = p[j][r] * (dz[r] - del[r]);
    }
  }
#pragma unroll
  for (int j = 0; j < G::NSUB; j += 2) {
    if (j + 1 < G::NSUB) {  // resolved at compile time
      P::pv2(ring + (qt[j] + PL::kT2), ring + (qt[j + 1] + PL::kT2), p[j], p[j + 1], acc_v);  // dV^T += dO^T P
      P::pv2(ring + (qt[j] + PL::kT1), ring + (qt[j + 1] + PL::kT1), d[j], d[j + 1], acc_k);  // dK^T += Q^T dS
    } else {
      P::pv(ring + (qt[j] + PL::kT2), p[j], acc_v);
      P::pv(ring + (qt[j] + PL::kT1), d[j], acc_k);
    }
  }
}

// ---------------------------------------------------------------- chunks of tiles per workgroup
//
// For bands of at most two 64-row blocks (windows like the causal
// 64): one workgroup streams a chunk of consecutive tiles of a residue class.
// The band's two blocks sit in two LDS slots (block j in slot j & 1); moving
// to tile t+1 adds at most one block, prefetched into registers while tile t
// computes and written over the block tile t+1 no longer reads.  The next
// tile's register rows are prefetched the same way.  Each block and row
// crosses HBM once per chunk.

struct BwdChunk {
  int b, h, rho, t0, t1, Nr, nblk;
  uint32_t tb;
  int64_t base;
  uint32_t nrec;
};

template <class P>
__device__ __forceinline__ bool bwd_chunk(const BwdArgs& a, BwdChunk& w) {
  // Dilation 1: XCD-contiguous ids, so neighbouring chunks (which share a
  // halo block) run on one L2 (cfg2 fp32 backward 232.6 -> 220.4 us).  The
  // residue classes of a dilated window interleave row by row in memory and
  // run best side by side on different XCDs, as dispatched (cfg5 fp32: 412
  // against 434 us contiguous).
  int lin = a.dil == 1 ? xcd_row_order((int)blockIdx.x, (int)gridDim.x) : (int)blockIdx.x;
  const int chunk_id = lin % a.chunks;
  lin /= a.chunks;
  w.rho = lin % a.dil;
  lin /= a.dil;
  w.h = lin % (int)a.H;
  w.b = lin / (int)a.H;
  w.Nr = (int)((a.N - w.rho + a.dil - 1) / a.dil);
  w.nblk = (w.Nr + 63) >> 6;
  w.t0 = chunk_id * a.chunk;
  w.t1 = min(w.t0 + a.chunk, w.nblk);
  w.tb = (uint32_t)a.tok_bytes;
  w.base = (((int64_t)w.b * a.N + w.rho) * a.H + w.h) * kHeadDim;
  w.nrec = (uint32_t)((int64_t)(w.Nr - 1) * w.tb + kHeadDim * sizeof(typename P::Elt));
  return w.t0 < w.t1;
}

// FL >= 0: specialised for the band [m-FL, m+FR] (interior tiles take the
// fixed-window tiles above); FL < 0: any band of at most two blocks.
template <class P, int FL, int FR>
__global__ __launch_bounds__(256, 2) void bwd_q_stream_kernel(BwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // 2 slots x (K slot, V slot)
  using Elt = typename P::Elt;
  using PL = PairLds<P>;
  constexpr int kBuf = PL::kBytes;
  BwdChunk w;
  if (!bwd_chunk<P>(a, w)) return;  // uniform, before any barrier
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

  // Key blocks are 64 rows from row ob = -16*(ceil(L/16) & 3), so that a
  // band whose 64 + L + R keys fit two blocks meets exactly two ([i-32, i+31]
  // straddles 3 aligned blocks, 2 shifted ones; causal 64 has ob = 0).  Rows
  // of block 0 before row 0 get offsets that wrap past the buffer range and
  // read zero, and their keys are masked.
  const int ob = -16 * (((L + 15) >> 4) & 3);
  const int nbs = floordiv32(w.Nr - 1 - ob, 64) + 1;
  auto lo_of = [&](int t) { return max(floordiv32(64 * t - L - ob, 64), 0); };
  auto hi_of = [&](int t) { return min(floordiv32(64 * t + 63 + R - ob, 64), nbs - 1); };
  auto boff = [&](int j) { return (uint32_t)(64 * j + ob) * tb; };
  const uint32_t lrow = (uint32_t)(16 * wv + c) * tb;  // this lane's row within a tile
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);

  // prologue: the first tile's rows and band
  typename P::Q qr, gr, qn, gn;
  P::load_q(qr, Qr, (uint32_t)(64 * w.t0) * tb + lrow, g);
  P::load_q(gr, Gr, (uint32_t)(64 * w.t0) * tb + lrow, g);
  KvRegs<P> xk;  // V is read only as rows
  for (int j = lo_of(w.t0); j <= hi_of(w.t0); ++j) {
    kv_load<P>(xk, Kr, Vr, boff(j), tid, tb);
    kv_store<P>(xk, ring + (j & 1) * kBuf, tid);
  }
  __syncthreads();

  const float sl2 = a.scale_log2;
  const int dl = 4 * g - c + L;
  for (int t = w.t0; t < w.t1; ++t) {
    // prefetch: tile t+1's new block and rows
    const bool more = t + 1 < w.t1;
    const int nblk_new = more && hi_of(t + 1) > hi_of(t) ? hi_of(t + 1) : -1;
    const uint32_t noff = nblk_new >= 0 ? boff(nblk_new) : kOob;
    kv_load<P>(xk, Kr, Vr, noff, tid, tb);
    const uint32_t nrow = more ? (uint32_t)(64 * (t + 1)) * tb + lrow : kOob;
    P::load_q(qn, Qr, nrow, g);
    P::load_q(gn, Gr, nrow, g);

    const int q0 = 64 * t + 16 * wv;
    float lse2, dlt;
    f32x4 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bool done = false;
    if constexpr (FL >= 0) {
      // interior: every key sub-tile of every wave lies in [0, Nr)
      using G = WinGeom<FL, FR, 64>;
      if (4 * t - G::CL >= 0 && 16 * (4 * t + 3 - G::CL + G::NSUB) <= w.Nr) {
        bwdq_window_tile<P, FL, FR>(ring, kl, vl, qr, gr, t, wv, dl, sl2, lse2, dlt, acc);
        done = true;
      }
    }
    if (!done) {
      const int lo = lo_of(t), hi = hi_of(t);  // hi - lo is 0 or 1
      // Both blocks' scores stay in registers from pass 1 to pass 2.
      float m_run = -INFINITY, l_run = 0.0f, a_run = 0.0f;
      const uint8_t* sk0 = ring + (lo & 1) * kBuf;
      const uint8_t* sk1 = ring + (hi & 1) * kBuf;
      f32x4 s0[4], dp0[4], s1[4], dp1[4];
      const int live0 = bwdq_scores<P>(sk0, sk0 + PL::kRows2, kl, qr, gr, 64 * lo + ob, q0, L, R, dl, g, w.Nr, s0,
                                       dp0);
      bwdq_pass1(s0, dp0, live0, sl2, m_run, l_run, a_run);
      int live1 = 0;
      if (hi > lo) {
        live1 = bwdq_scores<P>(sk1, sk1 + PL::kRows2, kl, qr, gr, 64 * hi + ob, q0, L, R, dl, g, w.Nr, s1, dp1);
        bwdq_pass1(s1, dp1, live1, sl2, m_run, l_run, a_run);
      }
      bwdq_stats(m_run, l_run, a_run, sl2, lse2, dlt);
      bwdq_pass2<P>(sk0, vl + PL::kT1, s0, dp0, live0, sl2, lse2, dlt, acc);
      if (hi > lo) bwdq_pass2<P>(sk1, vl + PL::kT1, s1, dp1, live1, sl2, lse2, dlt, acc);
    }
    P::store_o(acc, a.scale, DQr, (uint32_t)(64 * t) * tb + lrow, g);
    const int64_t srow = (((int64_t)w.b * a.N + w.rho + (int64_t)a.dil * (q0 + c)) * a.H + w.h);
    if (g == 0 && q0 + c < w.Nr) *reinterpret_cast<float2*>(a.stats + 2 * srow) = make_float2(lse2, dlt);

    // the new block replaces block hi(t+1) - 2, which tile t may still read
    __syncthreads();
    if (nblk_new >= 0) {
      kv_store<P>(xk, ring + (nblk_new & 1) * kBuf, tid);
    }
    __syncthreads();
    qr = qn;
    gr = gn;
  }
}

template <class P, int FL, int FR>
__global__ __launch_bounds__(256, 2) void bwd_kv_stream_kernel(BwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // 2 slots x (Q slot, dO slot, stats)
  using Elt = typename P::Elt;
  using PL = PairLds<P>;
  constexpr int kBuf = PL::kBytes + 512;
  BwdChunk w;
  if (!bwd_chunk<P>(a, w)) return;
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
  const BwdStats S = bwd_stats_rsrc(a, w.b, w.h, w.rho, w.Nr);

  // Query blocks are 64 rows from row ob = -16*(ceil(R/16) & 3) (as the key
  // blocks of bwd_q_stream_kernel, mirrored)
  const int ob = -16 * (((R + 15) >> 4) & 3);
  const int nbs = floordiv32(w.Nr - 1 - ob, 64) + 1;
  auto lo_of = [&](int t) { return max(floordiv32(64 * t - R - ob, 64), 0); };
  auto hi_of = [&](int t) { return min(floordiv32(64 * t + 63 + L - ob, 64), nbs - 1); };
  auto boff = [&](int j) { return (uint32_t)(64 * j + ob) * tb; };
  auto stat_off = [&](int j) { return j >= 0 && tid < 64 ? (uint32_t)(64 * j + ob + tid) * S.stride : kOob; };
  const uint32_t lrow = (uint32_t)(16 * wv + c) * tb;
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);

  typename P::Q kr, vr, kn, vn;
  P::load_q(kr, Kr, (uint32_t)(64 * w.t0) * tb + lrow, g);
  P::load_q(vr, Vr, (uint32_t)(64 * w.t0) * tb + lrow, g);
  QgRegs<P> xq;
  uint2 xs;
  for (int j = lo_of(w.t0); j <= hi_of(w.t0); ++j) {
    qg_load<P>(xq, Qr, Gr, boff(j), tid, tb);
    xs = bload8(S.r, stat_off(j));
    uint8_t* sb = ring + (j & 1) * kBuf;
    qg_store<P>(xq, sb, tid);
    bwd_stage_stats(sb + PL::kBytes, xs, tid);
  }
  __syncthreads();

  const int dl = c - 4 * g + L;
  for (int t = w.t0; t < w.t1; ++t) {
    const bool more = t + 1 < w.t1;
    const int nblk_new = more && hi_of(t + 1) > hi_of(t) ? hi_of(t + 1) : -1;
    const uint32_t noff = nblk_new >= 0 ? boff(nblk_new) : kOob;
    qg_load<P>(xq, Qr, Gr, noff, tid, tb);
    xs = bload8(S.r, stat_off(nblk_new));
    const uint32_t nrow = more ? (uint32_t)(64 * (t + 1)) * tb + lrow : kOob;
    P::load_q(kn, Kr, nrow, g);
    P::load_q(vn, Vr, nrow, g);

    const int k0 = 64 * t + 16 * wv;
    f32x4 acc_k[4], acc_v[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc_k[dt] = acc_v[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    bool done = false;
    if constexpr (FL >= 0) {
      // interior: every query sub-tile of every wave lies in [0, Nr)
      using G = WinGeom<FR, FL, 64>;
      if (4 * t - G::CL >= 0 && 16 * (4 * t + 3 - G::CL + G::NSUB) <= w.Nr) {
        bwdkv_window_tile<P, FL, FR>(ring, kl, vl, kr, vr, t, wv, g, dl, a.scale_log2, acc_k, acc_v);
        done = true;
      }
    }
    if (!done)
      for (int j = lo_of(t); j <= hi_of(t); ++j) {
        const uint8_t* sq = ring + (j & 1) * kBuf;
        bwdkv_block<P>(sq, sq + PL::kRows2, reinterpret_cast<const float*>(sq + PL::kBytes), kl, vl + PL::kT1,
                       vl + PL::kT2, kr, vr, 64 * j + ob,
                       k0, L, R, dl, g, w.Nr, a.scale_log2, acc_k, acc_v);
      }
    const uint32_t orow = (uint32_t)(64 * t) * tb + lrow;
    P::store_o(acc_v, 1.0f, DVr, orow, g);
    P::store_o(acc_k, a.scale, DKr, orow, g);

    __syncthreads();
    if (nblk_new >= 0) {
      uint8_t* sb = ring + (nblk_new & 1) * kBuf;
      qg_store<P>(xq, sb, tid);
      bwd_stage_stats(sb + PL::kBytes, xs, tid);
    }
    __syncthreads();
    kr = kn;
    vr = vn;
  }
}

}  // namespace ma_dev
