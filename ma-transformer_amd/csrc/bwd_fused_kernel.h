// bwd_fused_kernel.h -- one-launch backward of the causal 64-key window
// (keys [m-63, m] on a residue class m of any dilation), bf16/fp16, head_dim
// 64.  Same arithmetic as bwd_q_stream_kernel + bwd_kv_stream_kernel
// (backward_kernel.h), in one pass over the inputs.
//
// One workgroup (4 waves) streams a chunk [t0, t1) of the 64-row tiles of one
// (batch, head, residue class).  Step t holds tiles t-1 and t in a two-slot
// LDS ring; a slot is the tile's K, V, Q and dO rows (row-major, 144 B rows)
// and its 64 {lse2, delta}:
//   query pass, tile t: S^T = K Q^T and dP^T = V dO^T over the 5 key
//     sub-tiles of each wave's 16 queries (in tiles t-1 and t), lse2 and
//     delta of the queries in registers (two-pass softmax, every score
//     resident), dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T.  dQ is stored,
//     {lse2, delta} go to the slot.
//   key pass, tile t-1 (complete now: the queries of its keys lie in tiles
//     t-1 and t, both with statistics): S = Q K^T and dP = dO V^T over the 5
//     query sub-tiles of each wave's 16 keys, P and dS from the slots'
//     statistics, dV^T += dO^T P and dK^T += Q^T dS.
// The transposed operands (K^T, Q^T, dO^T) are read from the row-major slots
// with gfx950's LDS transpose read (ds_read_b64_tr_b16), so no slot carries a
// transposed copy: two slots of 36.5 KB, two workgroups per CU.  While step t
// computes, tile t+1's four row blocks are in flight into registers.
//
// Each chunk also runs the query pass of tile t1 (statistics only: its dQ
// belongs to the next chunk) to complete key tile t1-1, and reads tile
// t0-1's K, V for the query pass of tile t0.  Chunks are dealt to XCDs in
// contiguous runs, so those re-reads of a neighbour's rows meet in one L2.
// Every other Q, K, V, dO row crosses HBM once; dQ, dK, dV are written once,
// with one writer per row.  No statistics reach HBM.
//
// Rows before row 0 (tile -1) read as zero and their keys are masked; rows
// at or past the class end read as zero (their dO is zero, so they add
// nothing to dK, dV) and their stores are dropped by the buffer range check.
#pragma once

#include "backward_kernel.h"
#include "block_kernel.h"

namespace ma_dev {

struct FusedSlot {
  static constexpr int kRow = 144;          // bytes per row (128 + 16 pad)
  static constexpr int kMat = 64 * kRow;    // one 64-row matrix
  static constexpr int kK = 0, kV = kMat, kQ = 2 * kMat, kG = 3 * kMat, kSt = 4 * kMat;
  static constexpr int kBytes = 4 * kMat + 512;  // + 64 lse2, 64 delta
};

// A operand words of M^T for the MFMA head_dim tile dt from a row-major
// 16-row sub-tile of M: lane (c, g) receives M[4g + e][d(dt, c)], e = 0..3,
// with d(dt, m) = 32(dt>>1) + 8(m>>2) + 4(dt&1) + (m&3), the head_dim order
// of the 16-bit path's O^T tiles.  The transpose read gives lane i of a
// 16-lane group element i%4 of the 8-byte chunk addressed by lane 4e + i/4,
// so lane l addresses row l>>2 at head_dim 32(dt>>1) + 8(l&3) + 4(dt&1):
// `p` = sub-tile base + tr_lane(lane) + tr_dt(dt).
__device__ __forceinline__ uint32_t tr_lane(int lane) { return (lane >> 2) * FusedSlot::kRow + 16 * (lane & 3); }
__device__ __forceinline__ constexpr uint32_t tr_dt(int dt) { return 64 * (dt >> 1) + 8 * (dt & 1); }

__device__ __forceinline__ uint2 tr_read(const uint8_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p));
  return __builtin_bit_cast(uint2, r);
}

// acc += M^T X^T over two 16-row sub-tiles m0, m1 of M (rows = the
// contraction), x0/x1 the lane's 4 values of each (rows 4g..4g+3, column c):
// one 16x16x32 MFMA per head_dim tile, as HalfPath::pv2.
template <typename T>
__device__ __forceinline__ void pv2_tr(const uint8_t* m0, const uint8_t* m1, const float (&x0)[4],
                                       const float (&x1)[4], f32x4 (&acc)[4]) {
  uint4 b;
  b.x = Mma<T>::pack2(x0[0], x0[1]);
  b.y = Mma<T>::pack2(x0[2], x0[3]);
  b.z = Mma<T>::pack2(x1[0], x1[1]);
  b.w = Mma<T>::pack2(x1[2], x1[3]);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const uint2 a0 = tr_read(m0 + tr_dt(dt));
    const uint2 a1 = tr_read(m1 + tr_dt(dt));
    acc[dt] = Mma<T>::x32(make_uint4(a0.x, a0.y, a1.x, a1.y), b, acc[dt]);
  }
}

// The same over one sub-tile (16x16x16 MFMA).
template <typename T>
__device__ __forceinline__ void pv_tr(const uint8_t* m0, const float (&x0)[4], f32x4 (&acc)[4]) {
  uint2 b;
  b.x = Mma<T>::pack2(x0[0], x0[1]);
  b.y = Mma<T>::pack2(x0[2], x0[3]);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = Mma<T>::x16(tr_read(m0 + tr_dt(dt)), b, acc[dt]);
}

// The register operand of row r of a slot matrix (lane (c, g): head_dim
// 8g..8g+7 and 32+8g..32+8g+7), as HalfPath::load_q from global memory.
template <class P>
__device__ __forceinline__ void lds_q(typename P::Q& x, const uint8_t* mat, int r, int g) {
  x.r[0] = *reinterpret_cast<const uint4*>(mat + r * FusedSlot::kRow + 16 * g);
  x.r[1] = *reinterpret_cast<const uint4*>(mat + r * FusedSlot::kRow + 16 * g + 64);
}

// Query pass of tile t for wave wv: queries 64t + 16wv + c against key
// sub-tiles s = 4t + wv - 4 + j, j = 0..4 (sub-tile s in slot (s >> 2) & 1).
// EDGE (t = 0): keys below row 0 are masked too.  Gives lse2, delta of the
// lane's query and dQ^T (unscaled) in acc.
template <class P, bool EDGE>
__device__ __forceinline__ void fused_qpass(const uint8_t* ring, int t, int wv, int c, int g, int lane, float sl2,
                                            float& lse2, float& dlt, f32x4 (&acc)[4]) {
  using T = typename P::Elt;
  constexpr int NS = 5, CL = 4;
  const uint8_t* st = ring + (t & 1) * FusedSlot::kBytes;
  typename P::Q qb, gb;
  lds_q<P>(qb, st + FusedSlot::kQ, 16 * wv + c, g);
  lds_q<P>(gb, st + FusedSlot::kG, 16 * wv + c, g);
  const uint32_t kl = c * FusedSlot::kRow + 16 * g;
  const uint32_t trl = tr_lane(lane);
  const int dl = 4 * g - c + 63;  // key - query + 63 of element 0, minus the sub-tile offset
  f32x4 e[NS], dp[NS];
  uint32_t kt[NS];  // sub-tile j's K rows (transpose-read base)
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int s = 4 * t + wv - CL + j;
    const uint32_t sub = (uint32_t)(((s >> 2) & 1) * FusedSlot::kBytes + 16 * (s & 3) * FusedSlot::kRow);
    kt[j] = sub + FusedSlot::kK + trl;
    f32x4 z = P::qk(ring + sub + FusedSlot::kK + kl, qb);
    dp[j] = P::qk(ring + sub + FusedSlot::kV + kl, gb);
    const int rel = 16 * (j - CL);
    if (j == 0 || j == NS - 1) {  // resolved at compile time: the band's two edge sub-tiles
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(dl + rel + r) <= 63u ? z[r] : -INFINITY;
    }
    if constexpr (EDGE) {
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = 16 * s + 4 * g + r >= 0 ? z[r] : -INFINITY;
    }
    e[j] = z;
    mx = fmaxf(mx, fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3])));
  }
  const float m_use = col_max(mx) * sl2;  // finite: every query sees its own key
  float l_run = 0.0f, a_run = 0.0f;
#pragma unroll
  for (int j = 0; j < NS; ++j)
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
  for (int j = 0; j < NS; j += 2) {
    float d0[4], d1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) d0[r] = e[j][r] * inv * (dp[j][r] - dlt);
    if (j + 1 < NS) {  // resolved at compile time
#pragma unroll
      for (int r = 0; r < 4; ++r) d1[r] = e[j + 1][r] * inv * (dp[j + 1][r] - dlt);
      pv2_tr<T>(ring + kt[j], ring + kt[j + 1], d0, d1, acc);
    } else {
      pv_tr<T>(ring + kt[j], d0, acc);
    }
  }
}

// Key pass of key tile kt for wave wv: keys 64kt + 16wv + c against query
// sub-tiles s = 4kt + wv + j, j = 0..4 (in tiles kt and kt+1).  dV^T and
// dK^T (unscaled) accumulate in acc_v, acc_k.
template <class P>
__device__ __forceinline__ void fused_kpass(const uint8_t* ring, int kt, int wv, int c, int g, int lane, float sl2,
                                            f32x4 (&acc_k)[4], f32x4 (&acc_v)[4]) {
  using T = typename P::Elt;
  constexpr int NS = 5;
  const uint8_t* sk = ring + (kt & 1) * FusedSlot::kBytes;
  typename P::Q kb, vb;
  lds_q<P>(kb, sk + FusedSlot::kK, 16 * wv + c, g);
  lds_q<P>(vb, sk + FusedSlot::kV, 16 * wv + c, g);
  const uint32_t kl = c * FusedSlot::kRow + 16 * g;
  const uint32_t trl = tr_lane(lane);
  const int dl = c - 4 * g + 63;  // key - query + 63 of element 0, plus the sub-tile offset
  float p[NS][4], d[NS][4];
  uint32_t qt[NS];  // sub-tile j's Q rows (transpose-read base); dO rows at + (kG - kQ)
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int s = 4 * kt + wv + j;
    const uint32_t slot = (uint32_t)(((s >> 2) & 1) * FusedSlot::kBytes);
    const uint32_t sub = slot + 16 * (s & 3) * FusedSlot::kRow;
    qt[j] = sub + FusedSlot::kQ + trl;
    f32x4 z = P::qk(ring + sub + FusedSlot::kQ + kl, kb);         // S[query 16s+4g+r][key c]
    const f32x4 dz = P::qk(ring + sub + FusedSlot::kG + kl, vb);  // dP[query][key c]
    if (j == 0 || j == NS - 1) {  // resolved at compile time
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(dl - 16 * j - r) <= 63u ? z[r] : -INFINITY;
    }
    const float* sts = reinterpret_cast<const float*>(ring + slot + FusedSlot::kSt);
    const f32x4 lse = *reinterpret_cast<const f32x4*>(sts + 16 * (s & 3) + 4 * g);
    const f32x4 del = *reinterpret_cast<const f32x4*>(sts + 64 + 16 * (s & 3) + 4 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[j][r] = __builtin_amdgcn_exp2f(fmaf(z[r], sl2, -lse[r]));
      d[j][r] = p[j][r] * (dz[r] - del[r]);
    }
  }
  constexpr uint32_t kGQ = FusedSlot::kG - FusedSlot::kQ;
#pragma unroll
  for (int j = 0; j < NS; j += 2) {
    if (j + 1 < NS) {  // resolved at compile time
      pv2_tr<T>(ring + qt[j] + kGQ, ring + qt[j + 1] + kGQ, p[j], p[j + 1], acc_v);  // dV^T += dO^T P
      pv2_tr<T>(ring + qt[j], ring + qt[j + 1], d[j], d[j + 1], acc_k);              // dK^T += Q^T dS
    } else {
      pv_tr<T>(ring + qt[j] + kGQ, p[j], acc_v);
      pv_tr<T>(ring + qt[j], d[j], acc_k);
    }
  }
}

// Tile x's four row blocks in flight: thread tid carries rows tid>>3 and
// (tid>>3)+32 at 16-byte column tid&7 of K, V, Q and dO.
template <class P>
struct FusedRows {
  typename P::Rows k, v, q, g;
};

template <class P>
__device__ __forceinline__ void fused_load(FusedRows<P>& x, __amdgpu_buffer_rsrc_t Kr, __amdgpu_buffer_rsrc_t Vr,
                                           __amdgpu_buffer_rsrc_t Qr, __amdgpu_buffer_rsrc_t Gr, uint32_t off_kv,
                                           uint32_t off_qg, int tid, uint32_t tb) {
  P::load_rows(x.k, Kr, off_kv, tid, tb);
  P::load_rows(x.v, Vr, off_kv, tid, tb);
  P::load_rows(x.q, Qr, off_qg, tid, tb);
  P::load_rows(x.g, Gr, off_qg, tid, tb);
}

template <class P>
__device__ __forceinline__ void fused_store(const FusedRows<P>& x, uint8_t* slot, int tid) {
  P::store_rows(x.k, slot + FusedSlot::kK, tid);
  P::store_rows(x.v, slot + FusedSlot::kV, tid);
  P::store_rows(x.q, slot + FusedSlot::kQ, tid);
  P::store_rows(x.g, slot + FusedSlot::kG, tid);
}

template <class P>
__global__ __launch_bounds__(256, 2) void bwd_fused_kernel(BwdArgs a) {
  static_assert(P::kKRow == FusedSlot::kRow, "slot rows are the 16-bit path's");
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // 2 x FusedSlot
  using Elt = typename P::Elt;
  // chunks dealt to XCDs in contiguous runs (neighbouring chunks share an L2)
  int lin = xcd_row_order(blockIdx.x, gridDim.x);
  const int chunk_id = lin % a.chunks;
  lin /= a.chunks;
  const int rho = lin % a.dil;
  lin /= a.dil;
  const int h = lin % (int)a.H;
  const int b = lin / (int)a.H;
  const int Nr = (int)((a.N - rho + a.dil - 1) / a.dil);
  const int nblk = (Nr + 63) >> 6;
  const int t0 = chunk_id * a.chunk;
  const int t1 = min(t0 + a.chunk, nblk);
  if (t0 >= t1) return;  // uniform, before any barrier
  const uint32_t tb = (uint32_t)a.tok_bytes;
  const int64_t base = (((int64_t)b * a.N + rho) * a.H + h) * kHeadDim;
  const uint32_t nrec = (uint32_t)((int64_t)(Nr - 1) * tb + kHeadDim * sizeof(Elt));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + base, nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + base, nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + base, nrec);
  const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const Elt*>(a.dout) + base, nrec);
  const __amdgpu_buffer_rsrc_t DQr = make_rsrc(static_cast<Elt*>(a.dq) + base, nrec);
  const __amdgpu_buffer_rsrc_t DKr = make_rsrc(static_cast<Elt*>(a.dk) + base, nrec);
  const __amdgpu_buffer_rsrc_t DVr = make_rsrc(static_cast<Elt*>(a.dv) + base, nrec);
  auto toff = [&](int x) { return (uint32_t)(64 * x) * tb; };  // x >= 0
  const uint32_t lrow = (uint32_t)(16 * wv + c) * tb;

  // prologue: tile t0-1's K, V (zero before row 0) and tile t0's rows
  FusedRows<P> x;
  fused_load<P>(x, Kr, Vr, Qr, Gr, t0 > 0 ? toff(t0 - 1) : kOob, kOob, tid, tb);
  fused_store<P>(x, ring + ((t0 - 1) & 1) * FusedSlot::kBytes, tid);
  fused_load<P>(x, Kr, Vr, Qr, Gr, toff(t0), toff(t0), tid, tb);
  fused_store<P>(x, ring + (t0 & 1) * FusedSlot::kBytes, tid);
  __syncthreads();

  const float sl2 = a.scale_log2;
  for (int t = t0; t <= t1; ++t) {
    // tile t+1's rows in flight (past the class end they read as zero)
    const bool more = t < t1;
    if (more) fused_load<P>(x, Kr, Vr, Qr, Gr, toff(t + 1), toff(t + 1), tid, tb);

    // query pass of tile t: dQ (owned for t < t1) and the statistics
    {
      float lse2, dlt;
      f32x4 acc[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (t == 0)
        fused_qpass<P, true>(ring, t, wv, c, g, lane, sl2, lse2, dlt, acc);
      else
        fused_qpass<P, false>(ring, t, wv, c, g, lane, sl2, lse2, dlt, acc);
      if (t < t1) P::store_o(acc, a.scale, DQr, toff(t) + lrow, g);
      float* sts = reinterpret_cast<float*>(ring + (t & 1) * FusedSlot::kBytes + FusedSlot::kSt);
      if (g == 0) {
        sts[16 * wv + c] = lse2;
        sts[64 + 16 * wv + c] = dlt;
      }
    }
    __syncthreads();

    // key pass of tile t-1
    if (t > t0) {
      f32x4 acc_k[4], acc_v[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc_k[dt] = acc_v[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      fused_kpass<P>(ring, t - 1, wv, c, g, lane, sl2, acc_k, acc_v);
      P::store_o(acc_v, 1.0f, DVr, toff(t - 1) + lrow, g);
      P::store_o(acc_k, a.scale, DKr, toff(t - 1) + lrow, g);
    }
    // tile t+1 replaces tile t-1, which both passes have finished reading
    __syncthreads();
    if (more) {
      fused_store<P>(x, ring + ((t + 1) & 1) * FusedSlot::kBytes, tid);
      __syncthreads();
    }
  }
}

}  // namespace ma_dev
