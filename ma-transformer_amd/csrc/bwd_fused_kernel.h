// bwd_fused_kernel.h -- one-launch backward of the fixed windows whose
// query tiles meet two key blocks and key blocks two query tiles: the causal
// 64 window (keys [m-63, m] on a residue class m of any dilation) and
// [m-32, m+31] (on the shifted key grid, blocks from row -32), bf16/fp16,
// head_dim 64.  Same arithmetic as bwd_q_stream_kernel + bwd_kv_stream_kernel
// (backward_kernel.h), in one pass over the inputs, each probability and
// its dS computed once.
//
// One workgroup (4 waves) streams a chunk [t0, t1) of the 64-row query tiles
// of one (batch, head, residue class).  Query tile t meets key blocks kb and
// kb+1 (kb = t-1 for the causal window, t on the shifted grid), and key
// block kb is seen by query tiles t-1 and t.  LDS holds the K, V rows of
// blocks kb, kb+1 (a two-slot ring), the Q, dO rows of tile t, and an
// exchange area for the probabilities and dS of tile t's queries, all
// row-major.  Step t:
//   query pass: each wave's 16 queries of tile t against their 5 key
//     sub-tiles: S^T = K Q^T, dP^T = V dO^T, lse and delta in registers
//     (two-pass softmax, every score resident), P^T and dS^T = P^T (dP^T -
//     delta) in registers; dQ^T += K^T dS^T and dQ stored.  P and dS (16-bit,
//     the MFMA operands) go to the exchange area as [query][key window] rows:
//     one 8-byte write per lane and sub-tile.
//   key pass: wave w owns keys 16w..16w+15 of blocks kb and kb+1.  Tile t's
//     query sub-tiles that see them (w+1 and 4-w of them) add dV^T += dO^T P
//     and dK^T += Q^T dS: P, dS columns from the exchange area and dO^T, Q^T
//     all through gfx950's LDS transpose read (ds_read_b64_tr_b16), which
//     turns row-major [query][key] into the MFMA operand layout.  Block kb is
//     then complete and stored; block kb+1's partial sums carry to step t+1.
// No slot holds a transposed copy and no statistics leave registers: 80 KB
// of LDS, two workgroups per CU.  While step t computes, step t+1's key
// block and query tile are in flight into registers.
//
// A chunk owns query tiles [t0, t1) and key blocks [t0, t1) (the last chunk
// also the blocks past its last tile).  It also runs the query passes of the
// neighbouring tiles that reach its blocks (tile t1 for the causal window,
// t0-1 on the shifted grid), without storing their dQ, and reads the key
// block before its first step.  On the shifted grid, chunks are dealt to
// XCDs in contiguous runs, so those re-reads of a neighbour's rows meet in one
// L2; the causal window runs its chunks in dispatch order (measured faster).
// Every other Q, K, V, dO row crosses HBM once; dQ, dK, dV are written once,
// with one writer per row.
//
// Rows outside the residue class read as zero.  Keys outside it are masked;
// a query row past the end (zero dO) adds nothing to dK, dV, and gets
// P = dS = 0 if no key of its window is left; stores outside the class are
// dropped by the buffer range check.
#pragma once

#include "backward_kernel.h"
#include "block_kernel.h"

namespace ma_dev {

// Rows of 160 B, the 16-bit path's padded rows (HalfPath's KROW: transpose
// reads on disjoint banks); exchange rows unpadded, so that two workgroups
// still fit a CU.  (At 144 B rows and 176 B exchange rows, 76 KB, the kernel
// took 0.2-0.9 % longer; 136 B rows read as 8-byte pairs halved the
// bank-conflict counter and left the time unchanged.)
struct FusedLds {
  static constexpr int kRow = 160;                // bytes per K/V/Q/dO row (128 + 32 pad)
  static constexpr int kMat = 64 * kRow;          // one 64-row matrix
  static constexpr int kRing = 2 * kMat;          // one ring slot: K rows, V rows
  static constexpr int kQ = 2 * kRing;            // tile t's Q rows
  static constexpr int kG = kQ + kMat;            // tile t's dO rows
  static constexpr int kXRow = 160;               // exchange row: 80 keys (160 B), unpadded
  static constexpr int kXW = 16 * kXRow;          // one wave's 16 query rows
  static constexpr int kXP = kG + kMat;           // P, 4 waves
  static constexpr int kXD = kXP + 4 * kXW;       // dS, 4 waves
  static constexpr int kBytes = kXD + 4 * kXW;    // 81920: two workgroups fill a CU's 160 KB
};

// A operand of M^T for head_dim tile dt from a 16-row sub-tile of a
// row-major K/V/Q/dO matrix: lane (c, g) receives M[4g + e][16dt + c],
// e = 0..3 (head_dim in natural order, so a lane group's pieces are
// contiguous: about 2 % faster on the target than the permuted order
// of the 16-bit path's O^T tiles, whose pieces lie 16 bytes apart).  Lane l addresses row l>>2 at head_dim 16dt + 4(l&3):
// sub-tile base + tr_lane(lane) + 32dt.  The products' accumulators then
// hold head_dim 16dt + 4g..4g+3 of column c in acc[dt] (store_nat).
__device__ __forceinline__ uint32_t tr_lane(int lane) { return (lane >> 2) * FusedLds::kRow + 8 * (lane & 3); }
__device__ __forceinline__ constexpr uint32_t tr_dt(int dt) { return 32 * dt; }

// dQ, dK or dV row c from natural-order accumulators (lane (c, g): head_dim
// 16dt + 4g..4g+3 in acc[dt]), times `scale`, in 16-byte stores: lane groups
// g and g^1 trade halves with v_permlane16_swap (odd 16-lane rows of the
// first operand with even rows of the second), after which an even g holds
// head_dim 4g..4g+7 and 32+4g..32+4g+7, an odd g head_dim 4g+12.. and
// 4g+44.. (8 each).
template <typename T>
__device__ __forceinline__ void store_nat(const f32x4 (&acc)[4], float scale, __amdgpu_buffer_rsrc_t r, uint32_t row,
                                          int g) {
  uint32_t w[4][2];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    w[dt][0] = Mma<T>::pack2(acc[dt][0] * scale, acc[dt][1] * scale);
    w[dt][1] = Mma<T>::pack2(acc[dt][2] * scale, acc[dt][3] * scale);
  }
  const uint32_t off = row + 8 * (g & ~1) + 32 * (g & 1);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t x[4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const auto sw = __builtin_amdgcn_permlane16_swap(w[2 * h][k], w[2 * h + 1][k], false, false);
      x[k] = sw[0];
      x[2 + k] = sw[1];
    }
    bstore16(r, off + 64 * h, make_uint4(x[0], x[1], x[2], x[3]));
  }
}

// B operand of one exchange column block: lane (c, g) receives X[4g + e][16jj
// + c] of a wave's 16 x 80 rows (e = 0..3) when lane l addresses row l>>2 at
// key 16jj + 4(l&3): wave block base + x_lane(lane) + 32jj.
__device__ __forceinline__ uint32_t x_lane(int lane) { return (lane >> 2) * FusedLds::kXRow + 8 * (lane & 3); }

// acc += M^T X^T over two 16-row sub-tiles of M (the contraction), b the
// packed 16-bit values of both (4 each): one 16x16x32 MFMA per head_dim tile.
template <typename T>
__device__ __forceinline__ void pv2_tr(const uint8_t* m0, const uint8_t* m1, uint4 b, f32x4 (&acc)[4]) {
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const uint2 a0 = tr_read(m0 + tr_dt(dt));
    const uint2 a1 = tr_read(m1 + tr_dt(dt));
    acc[dt] = Mma<T>::x32(make_uint4(a0.x, a0.y, a1.x, a1.y), b, acc[dt]);
  }
}

// The same over one sub-tile (16x16x16 MFMA).
template <typename T>
__device__ __forceinline__ void pv_tr(const uint8_t* m0, uint2 b, f32x4 (&acc)[4]) {
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = Mma<T>::x16(tr_read(m0 + tr_dt(dt)), b, acc[dt]);
}

// The register operand of row r of a row-major matrix in LDS (lane (c, g):
// head_dim 8g..8g+7 and 32+8g..32+8g+7), as HalfPath::load_q from memory.
template <class P>
__device__ __forceinline__ void lds_q(typename P::Q& x, const uint8_t* mat, int r, int g) {
  x.r[0] = *reinterpret_cast<const uint4*>(mat + r * FusedLds::kRow + 16 * g);
  x.r[1] = *reinterpret_cast<const uint4*>(mat + r * FusedLds::kRow + 16 * g + 64);
}

// Band geometry of the fused kernel, [m - FL, m + FR] on a residue class:
// key blocks are 64 rows from row OB (the two-launch kernels' shifted grid:
// -16 * (ceil(FL/16) mod 4)), so query tile t meets key blocks t + KB0 and
// t + KB0 + 1 and key block j is seen by query tiles j - KB0 - 1 and j - KB0.
// A wave's 16 queries 16q.. meet key sub-tiles (16 keys) q - CL .. q - CL + 4.
template <int FL, int FR>
struct FusedBand {
  static constexpr int CL = (FL + 15) / 16;
  static constexpr int NSUB = (15 + FR) / 16 + CL + 1;
  static constexpr int OB = -16 * (CL & 3);
  static constexpr int OB16 = OB / 16;
  static constexpr int KB0 = (-FL - OB) >= 0 ? (-FL - OB) / 64 : -((FL + OB + 63) / 64);
  static_assert(NSUB == 5, "the exchange rows hold 5 sub-tiles per query");
  static_assert((63 + FR - OB) / 64 - KB0 == 1, "the band meets two key blocks per query tile");
};

// Query pass of tile t for wave wv: queries 64t + 16wv + c against key
// sub-tiles s = 4t + wv - CL + j, j = 0..4, sub-tile s in key block
// (s - OB16) >> 2, ring slot of its parity.  EDGE (a tile whose window
// reaches below row 0 or past row Nr-1): keys outside [0, Nr) are masked
// too, and a row with no key left (a row past the end) gets P = dS = 0.
// Leaves dQ^T (unscaled) in acc and the wave's P, dS in its exchange rows
// (row c, keys 16j..16j+15 of its window).
template <class P, int FL, int FR, bool EDGE>
__device__ __forceinline__ void fused_qpass(uint8_t* lds, int t, int wv, int c, int g, int lane, float sl2, int Nr,
                                            f32x4 (&acc)[4]) {
  using T = typename P::Elt;
  using B = FusedBand<FL, FR>;
  constexpr int NS = B::NSUB, CL = B::CL;
  typename P::Q qb, gb;
  lds_q<P>(qb, lds + FusedLds::kQ, 16 * wv + c, g);
  lds_q<P>(gb, lds + FusedLds::kG, 16 * wv + c, g);
  const uint32_t kl = c * FusedLds::kRow + 16 * g;
  const uint32_t trl = tr_lane(lane);
  const int dl = 4 * g - c + FL;  // key - query + FL of element 0, minus the sub-tile offset
  f32x4 e[NS], dp[NS];
  uint32_t kt[NS];  // sub-tile j's K rows (transpose-read base)
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int s = 4 * t + wv - CL + j;
    const int sb = s - B::OB16;  // sub-tile index on the key-block grid
    const uint32_t sub = (uint32_t)(((sb >> 2) & 1) * FusedLds::kRing + 16 * (sb & 3) * FusedLds::kRow);
    kt[j] = sub + trl;
    f32x4 z = P::qk(lds + sub + kl, qb);
    dp[j] = P::qk(lds + sub + FusedLds::kMat + kl, gb);
    constexpr int kSpan = FL + FR;
    const int rel = 16 * (j - CL);
    if (rel - 15 < -FL || rel + 15 > FR) {  // resolved at compile time: the band's edge sub-tiles
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(dl + rel + r) <= (uint32_t)kSpan ? z[r] : -INFINITY;
    }
    if constexpr (EDGE) {
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(16 * s + 4 * g + r) < (uint32_t)Nr ? z[r] : -INFINITY;
    }
    e[j] = z;
    mx = fmaxf(mx, fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3])));
  }
  // every row inside the sequence sees its own key; a row past the end may see none
  const float m_all = col_max(mx);
  const float m_use = EDGE && m_all == -INFINITY ? 0.0f : m_all * sl2;
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
  const float inv = EDGE && !(l_tot > 0.0f) ? 0.0f : __builtin_amdgcn_rcpf(l_tot);
  const float dlt = col_sum(a_run) * inv;
  uint8_t* xp = lds + FusedLds::kXP + wv * FusedLds::kXW + c * FusedLds::kXRow + 8 * g;
  uint8_t* xd = xp + (FusedLds::kXD - FusedLds::kXP);
  uint2 pd[NS];  // packed dS of sub-tile j (keys 4g..4g+3)
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    float pr[4], dr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[r] = e[j][r] * inv;
      dr[r] = pr[r] * (dp[j][r] - dlt);
    }
    const uint2 pp = make_uint2(Mma<T>::pack2(pr[0], pr[1]), Mma<T>::pack2(pr[2], pr[3]));
    pd[j] = make_uint2(Mma<T>::pack2(dr[0], dr[1]), Mma<T>::pack2(dr[2], dr[3]));
    *reinterpret_cast<uint2*>(xp + 32 * j) = pp;
    *reinterpret_cast<uint2*>(xd + 32 * j) = pd[j];
  }
#pragma unroll
  for (int j = 0; j < NS; j += 2) {
    if (j + 1 < NS)  // resolved at compile time
      pv2_tr<T>(lds + kt[j], lds + kt[j + 1], make_uint4(pd[j].x, pd[j].y, pd[j + 1].x, pd[j + 1].y), acc);
    else
      pv_tr<T>(lds + kt[j], pd[j], acc);
  }
}

// One (query sub-tile jq of tile t, key column block jj of wave jq's window)
// pair of the key pass: dV^T += dO^T P, dK^T += Q^T dS over the 16 queries.
template <class P>
__device__ __forceinline__ void fused_kpair(const uint8_t* lds, int jq, int jj, uint32_t trl, uint32_t xl,
                                            f32x4 (&acc_k)[4], f32x4 (&acc_v)[4]) {
  using T = typename P::Elt;
  const uint32_t xo = jq * FusedLds::kXW + xl + 32 * jj;
  const uint2 bp = tr_read(lds + FusedLds::kXP + xo);
  const uint2 bd = tr_read(lds + FusedLds::kXD + xo);
  const uint32_t sub = 16 * jq * FusedLds::kRow + trl;
  pv_tr<T>(lds + FusedLds::kG + sub, bp, acc_v);
  pv_tr<T>(lds + FusedLds::kQ + sub, bd, acc_k);
}

// Tile x's four row blocks in flight: thread tid carries rows tid>>3 and
// (tid>>3)+32 at 16-byte column tid&7 of K, V, Q and dO.
template <class P>
struct FusedRows {
  typename P::Rows k, v, q, g;
};

template <class P, int FL, int FR>
__global__ __launch_bounds__(256, 2) void bwd_fused_kernel(BwdArgs a) {
  static_assert(P::kKRow == FusedLds::kRow, "LDS rows are the 16-bit path's");
  using B = FusedBand<FL, FR>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // FusedLds
  using Elt = typename P::Elt;
  // The shifted grid's chunks are dealt to XCDs in contiguous runs
  // (neighbouring chunks share an L2: [i-32, i+31] at B4 H8 N8192, 53.6 us
  // against 61.5 us as dispatched).  The causal window runs best as
  // dispatched: a dilated window's residue classes, which interleave row by
  // row in memory, side by side on different XCDs (cfg5 bf16 backward 120.3
  // -> 115.0 us), and at dilation 1 112.4 against 114.5 us at the target.
  int lin = a.dil == 1 && FR > 0 ? xcd_row_order(blockIdx.x, gridDim.x) : (int)blockIdx.x;
  const int chunk_id = lin % a.chunks;
  lin /= a.chunks;
  const int rho = lin % a.dil;
  lin /= a.dil;
  const int h = lin % (int)a.H;
  const int b = lin / (int)a.H;
  const int Nr = (int)((a.N - rho + a.dil - 1) / a.dil);
  const int nblk = (Nr + 63) >> 6;                        // query tiles
  const int nkb = floordiv32(Nr - 1 - B::OB, 64) + 1;     // key blocks
  const int t0 = chunk_id * a.chunk;
  const int t1 = min(t0 + a.chunk, nblk);
  if (t0 >= t1) return;  // uniform, before any barrier
  // this chunk's key blocks (the last chunk also takes those past its tiles),
  // and its steps: the query tiles whose dQ it owns or that reach its keys
  const int k0 = t0, k1 = t1 == nblk ? nkb : t1;
  const int s0 = max(min(t0, k0 - B::KB0 - 1), 0);
  const int s1 = max(t1 - 1, k1 - 1 - B::KB0);
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
  auto qoff = [&](int x) { return (uint32_t)(64 * x) * tb; };  // query tile x >= 0
  // first row of key block j; rows below 0 wrap past the buffer range, so
  // they read as zero and their stores are dropped
  auto koff = [&](int j) { return (uint32_t)(64 * j + B::OB) * tb; };
  auto slot = [&](int j) { return lds + (j & 1) * FusedLds::kRing; };
  const uint32_t lrow = (uint32_t)(16 * wv + c) * tb;
  const uint32_t trl = tr_lane(lane), xl = x_lane(lane);

  // prologue: the two key blocks of step s0 and its query tile
  FusedRows<P> x;
  const int kb_first = s0 + B::KB0;
  P::load_rows(x.k, Kr, koff(kb_first), tid, tb);
  P::load_rows(x.v, Vr, koff(kb_first), tid, tb);
  P::store_rows(x.k, slot(kb_first), tid);
  P::store_rows(x.v, slot(kb_first) + FusedLds::kMat, tid);
  P::load_rows(x.k, Kr, koff(kb_first + 1), tid, tb);
  P::load_rows(x.v, Vr, koff(kb_first + 1), tid, tb);
  P::load_rows(x.q, Qr, qoff(s0), tid, tb);
  P::load_rows(x.g, Gr, qoff(s0), tid, tb);
  P::store_rows(x.k, slot(kb_first + 1), tid);
  P::store_rows(x.v, slot(kb_first + 1) + FusedLds::kMat, tid);
  P::store_rows(x.q, lds + FusedLds::kQ, tid);
  P::store_rows(x.g, lds + FusedLds::kG, tid);
  __syncthreads();

  const float sl2 = a.scale_log2;
  // dK^T, dV^T of keys 16wv..16wv+15 of the block carried between steps
  f32x4 acc_k[4], acc_v[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc_k[dt] = acc_v[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int t = s0; t <= s1; ++t) {
    const int kb = t + B::KB0;  // key blocks kb, kb+1 in the ring
    // step t+1's new key block and query tile in flight (past the class end
    // they read as zero)
    const bool more = t < s1;
    if (more) {
      P::load_rows(x.k, Kr, koff(kb + 2), tid, tb);
      P::load_rows(x.v, Vr, koff(kb + 2), tid, tb);
      P::load_rows(x.q, Qr, qoff(t + 1), tid, tb);
      P::load_rows(x.g, Gr, qoff(t + 1), tid, tb);
    }

    // query pass of tile t: dQ (stored when this chunk owns it), P and dS exchanged
    {
      f32x4 acc[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if (64 * t - FL < 0 || 64 * t + 63 + FR >= Nr)
        fused_qpass<P, FL, FR, true>(lds, t, wv, c, g, lane, sl2, Nr, acc);
      else
        fused_qpass<P, FL, FR, false>(lds, t, wv, c, g, lane, sl2, Nr, acc);
      if (t >= t0 && t < t1) store_nat<Elt>(acc, a.scale, DQr, qoff(t) + lrow, g);
    }
    __syncthreads();

    // key pass: tile t's queries into keys 16wv.. of block kb (then complete)
    // and of block kb+1 (carried)
    if (kb >= k0 && kb < k1) {
      for (int jq = 0; jq <= wv; ++jq) fused_kpair<P>(lds, jq, wv - jq, trl, xl, acc_k, acc_v);
      store_nat<Elt>(acc_v, 1.0f, DVr, koff(kb) + lrow, g);
      store_nat<Elt>(acc_k, a.scale, DKr, koff(kb) + lrow, g);
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc_k[dt] = acc_v[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (kb + 1 >= k0 && kb + 1 < k1)
      for (int jq = wv; jq < 4; ++jq) fused_kpair<P>(lds, jq, 4 + wv - jq, trl, xl, acc_k, acc_v);
    // step t+1's rows replace key block kb and tile t's Q, dO, which both
    // passes have finished reading
    __syncthreads();
    if (more) {
      P::store_rows(x.k, slot(kb + 2), tid);
      P::store_rows(x.v, slot(kb + 2) + FusedLds::kMat, tid);
      P::store_rows(x.q, lds + FusedLds::kQ, tid);
      P::store_rows(x.g, lds + FusedLds::kG, tid);
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- copy probe
//
// bwd_fused_kernel's memory traffic without its arithmetic: the same
// workgroups, chunks and steps, each step reading the new key block's K, V
// rows and the query tile's Q, dO rows one step ahead, and writing
// dQ = Q xor dO for the tiles the chunk owns and dK = K, dV = V for its key
// blocks, at the kernel's positions.  It measures what this access pattern
// can move on the device.
template <int FL, int FR>
__global__ __launch_bounds__(256) void bwd_probe_kernel(BwdArgs a) {
  using B = FusedBand<FL, FR>;
  int lin = a.dil == 1 && FR > 0 ? xcd_row_order(blockIdx.x, gridDim.x) : (int)blockIdx.x;  // as the kernel
  const int chunk_id = lin % a.chunks;
  lin /= a.chunks;
  const int rho = lin % a.dil;
  lin /= a.dil;
  const int h = lin % (int)a.H;
  const int b = lin / (int)a.H;
  const int Nr = (int)((a.N - rho + a.dil - 1) / a.dil);
  const int nblk = (Nr + 63) >> 6;
  const int nkb = floordiv32(Nr - 1 - B::OB, 64) + 1;
  const int t0 = chunk_id * a.chunk;
  const int t1 = min(t0 + a.chunk, nblk);
  if (t0 >= t1) return;
  const int k0 = t0, k1 = t1 == nblk ? nkb : t1;
  const int s0 = max(min(t0, k0 - B::KB0 - 1), 0);
  const int s1 = max(t1 - 1, k1 - 1 - B::KB0);
  const uint32_t tb = (uint32_t)a.tok_bytes;
  const int64_t base = (((int64_t)b * a.N + rho) * a.H + h) * kHeadDim;
  const uint32_t nrec = (uint32_t)((int64_t)(Nr - 1) * tb + kHeadDim * 2);
  using E = uint16_t;
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const E*>(a.q) + base, nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const E*>(a.k) + base, nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const E*>(a.v) + base, nrec);
  const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const E*>(a.dout) + base, nrec);
  const __amdgpu_buffer_rsrc_t DQr = make_rsrc(static_cast<E*>(a.dq) + base, nrec);
  const __amdgpu_buffer_rsrc_t DKr = make_rsrc(static_cast<E*>(a.dk) + base, nrec);
  const __amdgpu_buffer_rsrc_t DVr = make_rsrc(static_cast<E*>(a.dv) + base, nrec);
  // thread tid: rows tid>>3 and (tid>>3)+32 of a 64-row block, 16-byte column tid&7
  const int tid = threadIdx.x;
  const uint32_t r0 = (uint32_t)(tid >> 3) * tb + 16 * (tid & 7), r1 = r0 + 32 * tb;
  auto qoff = [&](int x) { return (uint32_t)(64 * x) * tb; };
  auto koff = [&](int j) { return (uint32_t)(64 * j + B::OB) * tb; };  // rows below 0 fall out of range
  struct Two {
    uint4 x, y;
  };
  auto ld = [&](__amdgpu_buffer_rsrc_t r, uint32_t o) { return Two{bload16(r, o + r0), bload16(r, o + r1)}; };
  auto st = [&](__amdgpu_buffer_rsrc_t r, uint32_t o, Two v) {
    bstore16(r, o + r0, v.x);
    bstore16(r, o + r1, v.y);
  };
  const int kb_first = s0 + B::KB0;
  Two ka = ld(Kr, koff(kb_first)), va = ld(Vr, koff(kb_first));
  Two kn = ld(Kr, koff(kb_first + 1)), vn = ld(Vr, koff(kb_first + 1));
  Two q = ld(Qr, qoff(s0)), g = ld(Gr, qoff(s0));
  for (int t = s0; t <= s1; ++t) {
    const int kb = t + B::KB0;
    const Two kc = kn, vc = vn;  // block kb+1
    const uint32_t nx = t < s1 ? 0u : kOob;
    kn = ld(Kr, nx + koff(kb + 2));
    vn = ld(Vr, nx + koff(kb + 2));
    const Two qn = ld(Qr, nx + qoff(t + 1)), gn = ld(Gr, nx + qoff(t + 1));
    if (t >= t0 && t < t1)
      st(DQr, qoff(t), Two{make_uint4(q.x.x ^ g.x.x, q.x.y ^ g.x.y, q.x.z ^ g.x.z, q.x.w ^ g.x.w),
                           make_uint4(q.y.x ^ g.y.x, q.y.y ^ g.y.y, q.y.z ^ g.y.z, q.y.w ^ g.y.w)});
    if (kb >= k0 && kb < k1) {
      st(DVr, koff(kb), va);
      st(DKr, koff(kb), ka);
    }
    ka = kc;
    va = vc;
    q = qn;
    g = gn;
  }
}

}  // namespace ma_dev
