// bwd_longformer_kernel.h -- one-pass backward of the Longformer key sets
// from the forward's saved statistics: bf16/fp16, head_dim 64, dilation 1.
// Rows i >= G attend [max(0, i-L), i] U [0, G) with L <= 127 (the union, no
// key twice); rows i < G (the global rows) attend every key.
//
// Gradients from the saved row statistics lse2_i (log2 units of the scaled
// scores, store_lse) and delta_i = dO_i . O_i (O the forward's output):
//   P_ij = 2^(s_ij sl2 - lse2_i),  dS_ij = P_ij (dO_i . V_j - delta_i)
//   dQ_i = scale sum_j dS_ij K_j,  dK_j = scale sum_i dS_ij Q_i,
//   dV_j = sum_i P_ij dO_i.
// With the statistics given, every (i, j) pair contributes independently,
// so the set splits into three parts:
//   band pairs       i >= G, j in [max(0, i-L), i]
//   global keys      i >= G, j < G, i - j > L
//   global rows      i < G, every j.
// Band pairs are selected by i - j alone (0 <= i - j <= L): a row outside
// [G, N) carries lse2 = +inf in the tile's statistics, so its P and dS are 0
// in every pass; a key sub-tile below row 0 has +inf added to the rows'
// lse2.  For L = 127 (the kernel's FIXED127 form) only the diagonal
// sub-tiles at both ends of a window need a mask, one fixed per lane.
//
// Rows and keys come in 128-row tiles / blocks, so query tile t meets key
// blocks t-1 and t, and key block j is seen by query tiles j and j+1.  One
// workgroup (12 waves, one per CU, 3 per SIMD) streams a segment [t0, t1) of
// query tiles of one (batch, head) and owns key blocks [t0, t1) (a run of
// tiles that crosses into the next (batch, head) is two segments); LDS holds
// the K, V rows of blocks t-1 and t (a two-slot ring), tile t's Q and dO rows
// and statistics, and the 16 global keys' K, V rows and global rows' Q, dO
// rows.  Step t:
//   query pass   main wave w (0-7): queries 128t + 16w + c against their 9
//                window key sub-tiles and the global keys (P^T, dS^T with the
//                query as the MFMA column), dQ^T += K^T dS^T, dQ stored;
//   key pass     main wave w owns keys 16w.. of blocks t-1 and t: the tile's
//                query sub-tiles that see them, P, dS recomputed with the key
//                as the MFMA column (no exchange area), dV^T += dO^T P,
//                dK^T += Q^T dS; block t-1 is then complete: the global
//                rows' contributions are added and its dK, dV stored.
//                Block t's sums carry;
//   global sums  helper wave w (0-3): query sub-tiles 2w, 2w+1 against the
//                global keys with the key as the MFMA column (the global
//                keys' dK^T, dV^T) and the global rows against key sub-tiles
//                2w, 2w+1 of each completed block (the global rows' dQ^T),
//                summed over the segment.
// The main waves load the next key block and the helpers the next query
// tile.  A segment also runs the key pass of tile t1 (no dQ) for its block
// t1-1, and reads block t0-1 for tile t0's queries.  The global rows' dQ and
// the global keys' dK, dV are per-segment sums in the workspace (with one more
// slot for block 0's sums of keys 0..G-1); bwd_lf_combine adds them up and
// writes rows 0..G-1 of dQ, dK, dV.  Every other row of dQ, dK, dV has one
// writer; no atomics.  Rows past the end read as zero and their stores are
// dropped by the buffer range check; rows below 0 (block -1) wrap past the
// range the same way.
#pragma once

#include "bwd_fused_kernel.h"

namespace ma_dev {

struct LfArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;
  const void* o;     // the forward's output (delta = dO . O)
  const float* lse;  // the forward's row statistics (store_lse), [B*N*H]
  const float* delta;  // DLT kernels: each row's sum_j P_ij dP_ij from a delta-mode forward, [B*N*H] (o unused)
  void* dq;
  void* dk;
  void* dv;
  float* part;  // [B*H][nslot + 1][3][16][64]: global rows' dQ, global keys' dK, dV (unscaled sums)
  int32_t N, H, L, G;
  int32_t streams;  // B*H
  int32_t per_wg;   // query tiles per workgroup: its run of the streams' tiles, in order
  int32_t nslot;    // partial slots per (batch, head) before the extra one: workgroups meeting it, at most
  int32_t tok_bytes;
  float scale, scale_log2;
};

constexpr int kLfRows = 128;  // rows per query tile and key block
constexpr int kLfWaves = 8;    // main waves: the query and key passes
constexpr int kLfHelpers = 4;  // helper waves: tile loads and the global sums
constexpr int kLfThreads = 64 * (kLfWaves + kLfHelpers);  // 768
constexpr int kLfPart = 3 * 16 * kHeadDim;  // one segment's partials: dQ, dK, dV of 16 rows

struct LfLds {
  // 160 B rows (128 + 32 pad): the four rows of a transpose read's 16-lane
  // group fall on disjoint banks (measured 2 % faster than 144 B rows, which
  // keep the 16-byte row reads conflict-free instead)
  static constexpr int kRow = 160;
  static constexpr int kMat = kLfRows * kRow;     // one 128-row matrix
  static constexpr int kSlot = 2 * kMat;          // a key block: K rows, then V rows
  static constexpr int kQ = 2 * kSlot;            // tile t's Q rows
  static constexpr int kG = kQ + kMat;            // tile t's dO rows
  static constexpr int kGM = 16 * kRow;           // one 16-row global matrix
  static constexpr int kGK = kG + kMat;           // global keys' K rows
  static constexpr int kGV = kGK + kGM;           // global keys' V rows
  static constexpr int kGQ = kGV + kGM;           // global rows' Q rows
  static constexpr int kGG = kGQ + kGM;           // global rows' dO rows
  static constexpr int kSt = kGG + kGM;           // tile t: lse2[128], then delta[128]
  static constexpr int kStG = kSt + 8 * kLfRows;  // global rows: lse2[16], then delta[16]
  static constexpr int kBytes = kStG + 128;       // 134272
};
static_assert(LfLds::kBytes <= 160 * 1024, "one workgroup per CU");

// tr_lane and lds_q of the fused backward, on this kernel's rows.
__device__ __forceinline__ uint32_t lf_tr_lane(int lane) { return (lane >> 2) * LfLds::kRow + 8 * (lane & 3); }
template <class P>
__device__ __forceinline__ void lf_lds_q(typename P::Q& x, const uint8_t* mat, int r, int g) {
  x.r[0] = *reinterpret_cast<const uint4*>(mat + r * LfLds::kRow + 16 * g);
  x.r[1] = *reinterpret_cast<const uint4*>(mat + r * LfLds::kRow + 16 * g + 64);
}
// the segment-end reduction of the helpers' sums reuses the ring: 2 waves x 12 KB
static_assert(4 * 64 * 48 * 4 <= LfLds::kQ, "reduction area");

// 16-bit dot product of two 8-element pieces, in fp32.
template <typename T>
__device__ __forceinline__ float dot8(uint4 x, uint4 y) {
  const uint32_t a[4] = {x.x, x.y, x.z, x.w}, b[4] = {y.x, y.y, y.z, y.w};
  float d = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    d = fmaf(static_cast<float>(__builtin_bit_cast(T, (uint16_t)(a[j] & 0xffffu))),
             static_cast<float>(__builtin_bit_cast(T, (uint16_t)(b[j] & 0xffffu))), d);
    d = fmaf(static_cast<float>(__builtin_bit_cast(T, (uint16_t)(a[j] >> 16))),
             static_cast<float>(__builtin_bit_cast(T, (uint16_t)(b[j] >> 16))), d);
  }
  return d;
}

// Sum over the 8 consecutive lanes that hold one row's 16-byte pieces.
__device__ __forceinline__ float sum8(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  return x + __shfl_xor(x, 4);
}

// A 128-row matrix in flight over the 512 threads of the main waves: thread
// tid carries rows tid>>3 and (tid>>3)+64 at 16-byte column tid&7.
struct Rows128 {
  uint4 r[2];
};
__device__ __forceinline__ void lf_load(Rows128& x, __amdgpu_buffer_rsrc_t R, uint32_t off, int tid, uint32_t tb) {
  const uint32_t o = off + (uint32_t)(tid >> 3) * tb + 16 * (tid & 7);
  x.r[0] = bload16(R, o);
  x.r[1] = bload16(R, o + 64 * tb);
}
__device__ __forceinline__ void lf_store(const Rows128& x, uint8_t* mat, int tid) {
  uint8_t* p = mat + (tid >> 3) * LfLds::kRow + 16 * (tid & 7);
  *reinterpret_cast<uint4*>(p) = x.r[0];
  *reinterpret_cast<uint4*>(p + 64 * LfLds::kRow) = x.r[1];
}

// The same over the 256 threads of the helper waves (ht = tid - 512): rows
// (ht>>3) + 32k, k = 0..3, at 16-byte column ht&7.
struct Rows128x4 {
  uint4 r[4];
};
__device__ __forceinline__ void lf_load4(Rows128x4& x, __amdgpu_buffer_rsrc_t R, uint32_t off, int ht, uint32_t tb) {
  const uint32_t o = off + (uint32_t)(ht >> 3) * tb + 16 * (ht & 7);
#pragma unroll
  for (int k = 0; k < 4; ++k) x.r[k] = bload16(R, o + 32 * k * tb);
}
__device__ __forceinline__ void lf_store4(const Rows128x4& x, uint8_t* mat, int ht) {
  uint8_t* p = mat + (ht >> 3) * LfLds::kRow + 16 * (ht & 7);
#pragma unroll
  for (int k = 0; k < 4; ++k) *reinterpret_cast<uint4*>(p + 32 * k * LfLds::kRow) = x.r[k];
}

// A query tile in flight (helper waves): Q and dO rows, the statistic of row
// ht (ht < 128) and the rows' delta.  From saved statistics delta = dO . O is
// taken as soon as the O rows arrive, so they hold no registers through the
// helpers' sums (with O in flight to the staging point, 14 VGPRs spilled; cfg4
// 243-245 -> 229-231 us).
struct LfTile {
  Rows128x4 q, g;
  float lse2, dlt;  // dlt: DLT kernels, row ht's delta
  float od[4];      // otherwise: rows (ht>>3) + 32k's delta, summed over their 8 threads
};

// Tile t's rows into LDS: Q and dO rows, each row's lse2 and delta.
template <typename T, bool DLT>
__device__ __forceinline__ void lf_stage_tile(const LfTile& x, uint8_t* lds, int ht) {
  lf_store4(x.q, lds + LfLds::kQ, ht);
  lf_store4(x.g, lds + LfLds::kG, ht);
  float* st = reinterpret_cast<float*>(lds + LfLds::kSt);
  if (ht < kLfRows) st[ht] = x.lse2;
  if constexpr (DLT) {
    if (ht < kLfRows) st[kLfRows + ht] = x.dlt;
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if ((ht & 7) == 0) st[kLfRows + (ht >> 3) + 32 * k] = x.od[k];
  }
}

// P (or P^T) and dS of one 16x16 sub-tile: elements where keep[r] holds.
__device__ __forceinline__ void lf_probs(const f32x4& s, const f32x4& dp, const float (&lse2)[4],
                                         const float (&dlt)[4], const bool (&keep)[4], float sl2, float (&p)[4],
                                         float (&ds)[4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    p[r] = keep[r] ? __builtin_amdgcn_exp2f(fmaf(s[r], sl2, -lse2[r])) : 0.0f;
    ds[r] = p[r] * (dp[r] - dlt[r]);
  }
}

// Which pairs of a band sub-tile (MFMA column c, rows 4g + r) are kept:
//   kLfBand       those with 0 <= i - j <= L (dq[r] = i - j);
//   kLfAll        all of them;
//   kLfColBefore  those with c <  4g + r,   kLfColFrom  those with c >= 4g + r;
//   kLfColAfter   those with c >  4g + r,   kLfColUpTo  those with c <= 4g + r.
// The last five are the sub-tiles of a window of L = 127 on the 16-row grid:
// whole sub-tiles between the two diagonal ones at its ends.
enum LfMask { kLfBand, kLfAll, kLfColBefore, kLfColFrom, kLfColAfter, kLfColUpTo };

template <int M>
__device__ __forceinline__ void lf_probs_m(const f32x4& s, const f32x4& dp, const float (&lse2)[4],
                                           const float (&dlt)[4], const int (&dq)[4], int L, int c, int g,
                                           float sl2, float (&p)[4], float (&ds)[4]) {
  if (M == kLfAll) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = __builtin_amdgcn_exp2f(fmaf(s[r], sl2, -lse2[r]));
      ds[r] = p[r] * (dp[r] - dlt[r]);
    }
  } else {
    bool keep[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * g + r;
      keep[r] = M == kLfBand       ? (uint32_t)dq[r] <= (uint32_t)L
                : M == kLfColBefore ? c < row
                : M == kLfColFrom   ? c >= row
                : M == kLfColAfter  ? c > row
                                    : c <= row;
    }
    lf_probs(s, dp, lse2, dlt, keep, sl2, p, ds);
  }
}

template <typename T>
__device__ __forceinline__ uint2 pack4(const float (&x)[4]) {
  return make_uint2(Mma<T>::pack2(x[0], x[1]), Mma<T>::pack2(x[2], x[3]));
}

// acc += M^T X^T over one sub-tile with X split into a 16-bit value and its
// 16-bit remainder (two MFMAs): for the global rows' and global keys' sums,
// which run over every row or key of the sequence, so that the operand's
// rounding (2^-9 relative in bf16) does not accumulate over thousands of
// terms.
template <typename T>
__device__ __forceinline__ void pv_tr_split(const uint8_t* m0, const float (&x)[4], f32x4 (&acc)[4]) {
  const uint2 hi = pack4<T>(x);
  const uint32_t w[4] = {hi.x & 0xffffu, hi.x >> 16, hi.y & 0xffffu, hi.y >> 16};
  float lo[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) lo[r] = x[r] - static_cast<float>(__builtin_bit_cast(T, (uint16_t)w[r]));
  pv_tr<T>(m0, hi, acc);
  pv_tr<T>(m0, pack4<T>(lo), acc);
}

// Key pass of one key sub-tile (16 keys k0.., lane c = key k0 + c, k0 >= 0)
// against query sub-tiles jq in [jlo, jhi] of the tile at row q0, whose Q /
// dO rows and statistics are in LDS: the band pairs, selected as M says
// (rows outside [G, N) have P = 0 through their statistics).  K, V of the
// keys as register operands.
template <class P, int M>
__device__ __forceinline__ void lf_kpass(const uint8_t* lds, const typename P::Q& kr, const typename P::Q& vr,
                                         int k0, int q0, int jlo, int jhi, int L, int c, int g, uint32_t kl,
                                         uint32_t trl, float sl2, f32x4 (&ak)[4], f32x4 (&av)[4]) {
  using T = typename P::Elt;
  const float* st = reinterpret_cast<const float*>(lds + LfLds::kSt);
  // packed P and dS of query sub-tile jq (key as the MFMA column)
  auto probs = [&](int jq, uint2& pp, uint2& dd) __attribute__((always_inline)) {
    const f32x4 s = P::qk(lds + LfLds::kQ + 16 * jq * LfLds::kRow + kl, kr);   // S[query 16jq + 4g + r][key c]
    const f32x4 dp = P::qk(lds + LfLds::kG + 16 * jq * LfLds::kRow + kl, vr);  // dP[query][key c]
    const int dq0 = q0 + 16 * jq + 4 * g - (k0 + c);
    const f32x4 l4 = *reinterpret_cast<const f32x4*>(st + 16 * jq + 4 * g);
    const f32x4 d4 = *reinterpret_cast<const f32x4*>(st + kLfRows + 16 * jq + 4 * g);
    float lse2[4], dlt[4], p[4], ds[4];
    int dq[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      lse2[r] = l4[r];
      dlt[r] = d4[r];
      dq[r] = dq0 + r;
    }
    lf_probs_m<M>(s, dp, lse2, dlt, dq, L, c, g, sl2, p, ds);
    pp = pack4<T>(p);
    dd = pack4<T>(ds);
  };
  int jq = jlo;
  for (; jq < jhi; jq += 2) {  // uniform: two query sub-tiles per 16x16x32 MFMA
    uint2 p0, d0, p1, d1;
    probs(jq, p0, d0);
    probs(jq + 1, p1, d1);
    const uint32_t o0 = 16 * jq * LfLds::kRow + trl, o1 = o0 + 16 * LfLds::kRow;
    pv2_tr<T>(lds + LfLds::kG + o0, lds + LfLds::kG + o1, make_uint4(p0.x, p0.y, p1.x, p1.y), av);
    pv2_tr<T>(lds + LfLds::kQ + o0, lds + LfLds::kQ + o1, make_uint4(d0.x, d0.y, d1.x, d1.y), ak);
  }
  if (jq == jhi) {  // uniform: an odd count's last sub-tile
    uint2 p0, d0;
    probs(jq, p0, d0);
    const uint32_t o0 = 16 * jq * LfLds::kRow + trl;
    pv_tr<T>(lds + LfLds::kG + o0, p0, av);
    pv_tr<T>(lds + LfLds::kQ + o0, d0, ak);
  }
}

// The global rows' contributions to the dK^T, dV^T of one key sub-tile (lane
// c = key k0 + c, key as the MFMA column; K, V of the keys as the register
// operands kr / vr).
template <class P>
__device__ __forceinline__ void lf_global_rows_kv(const uint8_t* lds, const typename P::Q& kr,
                                                  const typename P::Q& vr, int k0, int G, int N, int c, int g,
                                                  uint32_t kl, uint32_t trl, float sl2, f32x4 (&ak)[4],
                                                  f32x4 (&av)[4]) {
  using T = typename P::Elt;
  const float* sg = reinterpret_cast<const float*>(lds + LfLds::kStG);
  const f32x4 s = P::qk(lds + LfLds::kGQ + kl, kr);  // S[global query 4g + r][key c]
  const f32x4 dp = P::qk(lds + LfLds::kGG + kl, vr);
  const f32x4 l4 = *reinterpret_cast<const f32x4*>(sg + 4 * g);
  const f32x4 d4 = *reinterpret_cast<const f32x4*>(sg + 16 + 4 * g);
  float lse2[4], dlt[4], p[4], ds[4];
  bool keep[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    keep[r] = 4 * g + r < G && k0 + c < N;
    lse2[r] = l4[r];
    dlt[r] = d4[r];
  }
  lf_probs(s, dp, lse2, dlt, keep, sl2, p, ds);
  pv_tr<T>(lds + LfLds::kGG + trl, pack4<T>(p), av);
  pv_tr<T>(lds + LfLds::kGQ + trl, pack4<T>(ds), ak);
}

// The global rows' dQ^T from one key sub-tile (keys k0.., K / V rows at
// krows / vrows; global query as the MFMA column).
template <class P>
__device__ __forceinline__ void lf_global_rows_dq(const uint8_t* lds, const uint8_t* krows, const uint8_t* vrows,
                                                  int k0, int G, int N, int c, int g, uint32_t kl, uint32_t trl,
                                                  float sl2, f32x4 (&agq)[4]) {
  using T = typename P::Elt;
  const float* sg = reinterpret_cast<const float*>(lds + LfLds::kStG);
  typename P::Q qg, gg;
  lds_q<P>(qg, lds + LfLds::kGQ, c, g);
  lds_q<P>(gg, lds + LfLds::kGG, c, g);
  const f32x4 s = P::qk(krows + kl, qg);  // S^T[key 4g + r][global query c]
  const f32x4 dp = P::qk(vrows + kl, gg);
  const float lse2c = sg[c], dltc = sg[16 + c];
  float lse2[4], dlt[4], p[4], ds[4];
  bool keep[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    keep[r] = c < G && k0 + 4 * g + r < N;
    lse2[r] = lse2c;
    dlt[r] = dltc;
  }
  lf_probs(s, dp, lse2, dlt, keep, sl2, p, ds);
  pv_tr_split<T>(krows + trl, ds, agq);
}

// One segment: query tiles [t0, t1) of (batch, head) bh and key blocks
// [t0, t1), its global sums into partial slot slot_id.  FIXED127: L = 127,
// the band's sub-tiles selected by the fixed masks.
template <class P, bool FIXED127, bool DLT>
__device__ __forceinline__ void lf_segment(const LfArgs& a, uint8_t* lds, int bh, int t0, int t1, int slot_id) {
  using T = typename P::Elt;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wq = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool main_wave = wq < kLfWaves;
  const int wv = main_wave ? wq : wq - kLfWaves;  // main: 0..7, helper: 0..3
  const int ht = tid - 64 * kLfWaves;             // a helper's thread index (0..255)
  const int c = lane & 15;
  const int g = lane >> 4;

  const int h = bh % a.H;
  const int b = bh / a.H;
  const int N = a.N, L = FIXED127 ? kLfRows - 1 : a.L, G = a.G;
  const int nt = (N + kLfRows - 1) / kLfRows;
  if (t0 >= t1) return;  // uniform, before any barrier
  const int s1 = t1 < nt ? t1 : t1 - 1;  // the last step: tile t1's key pass for block t1-1
  const uint32_t tb = (uint32_t)a.tok_bytes;
  const int64_t base = ((int64_t)b * N * a.H + h) * kHeadDim;
  const uint32_t nrec = (uint32_t)((int64_t)(N - 1) * tb + kHeadDim * sizeof(T));
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const T*>(a.q) + base, nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const T*>(a.k) + base, nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const T*>(a.v) + base, nrec);
  const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const T*>(a.dout) + base, nrec);
  const __amdgpu_buffer_rsrc_t Or = make_rsrc(static_cast<const T*>(a.o) + base, nrec);
  const __amdgpu_buffer_rsrc_t DQr = make_rsrc(static_cast<T*>(a.dq) + base, nrec);
  const __amdgpu_buffer_rsrc_t DKr = make_rsrc(static_cast<T*>(a.dk) + base, nrec);
  const __amdgpu_buffer_rsrc_t DVr = make_rsrc(static_cast<T*>(a.dv) + base, nrec);
  const float* lse = a.lse + (int64_t)b * N * a.H + h;  // row i at i * H
  const float* dlt = DLT ? a.delta + (int64_t)b * N * a.H + h : nullptr;
  float* part = a.part + (int64_t)bh * (a.nslot + 1) * kLfPart;
  // byte offset of row r (r >= -128); rows below 0 wrap past the range
  auto roff = [&](int r) { return (uint32_t)r * tb; };
  auto slot = [&](int j) { return lds + (j & 1) * LfLds::kSlot; };
  auto load_tile = [&](LfTile& x, int t) {  // helper waves
    const uint32_t o = roff(kLfRows * t);
    lf_load4(x.q, Qr, o, ht, tb);
    lf_load4(x.g, Gr, o, ht, tb);
    if constexpr (!DLT) {  // delta = dO . O at once: O's registers free before the sums
      Rows128x4 xo;
      lf_load4(xo, Or, o, ht, tb);
#pragma unroll
      for (int k = 0; k < 4; ++k) x.od[k] = sum8(dot8<T>(x.g.r[k], xo.r[k]));
    }
    const int i = kLfRows * t + ht;  // no band pair for a row outside [G, N): P = 0
    const bool in = ht < kLfRows && i >= G && i < N;
    x.lse2 = in ? lse[(int64_t)i * a.H] : __builtin_inff();
    if constexpr (DLT) x.dlt = in ? dlt[(int64_t)i * a.H] : 0.0f;
  };
  // row c, head_dim 16dt + 4g + r of matrix m (0 dQ, 1 dK, 2 dV) of a slot of partials
  auto store_part = [&](int slot_id, int m, const f32x4(&v)[4]) __attribute__((always_inline)) {
    float* dst = part + (int64_t)slot_id * kLfPart + m * 16 * kHeadDim + c * kHeadDim + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) *reinterpret_cast<f32x4*>(dst + 16 * dt) = v[dt];
  };
  const float sl2 = a.scale_log2;
  const uint32_t kl = c * LfLds::kRow + 16 * g;
  const uint32_t trl = lf_tr_lane(lane);

  // prologue: the global keys' K, V rows and the global rows' Q, dO rows
  // and statistics (main waves 0 and 1: one 16-byte piece per thread), the
  // key blocks t0-1 and t0 (main waves) and tile t0 (helpers)
  if (tid < 128) {  // uniform per wave
    const uint32_t o = (uint32_t)(tid >> 3) * tb + 16 * (tid & 7);
    const uint4 kx = bload16(Kr, o), vx = bload16(Vr, o), qx = bload16(Qr, o), gx = bload16(Gr, o);
    const int r = tid >> 3;
    uint8_t* p = lds + r * LfLds::kRow + 16 * (tid & 7);
    *reinterpret_cast<uint4*>(p + LfLds::kGK) = kx;
    *reinterpret_cast<uint4*>(p + LfLds::kGV) = vx;
    *reinterpret_cast<uint4*>(p + LfLds::kGQ) = qx;
    *reinterpret_cast<uint4*>(p + LfLds::kGG) = gx;
    float d;
    if constexpr (DLT) {
      d = r < G && r < N ? dlt[(int64_t)r * a.H] : 0.0f;
    } else {
      const uint4 ox = bload16(Or, o);
      d = sum8(dot8<T>(gx, ox));
    }
    float* sg = reinterpret_cast<float*>(lds + LfLds::kStG);
    if ((tid & 7) == 0) {
      sg[r] = r < G && r < N ? lse[(int64_t)r * a.H] : 0.0f;
      sg[16 + r] = d;
    }
  }
  if (main_wave) {
    Rows128 xk, xv;
    lf_load(xk, Kr, roff(kLfRows * (t0 - 1)), tid, tb);
    lf_load(xv, Vr, roff(kLfRows * (t0 - 1)), tid, tb);
    lf_store(xk, slot(t0 - 1), tid);
    lf_store(xv, slot(t0 - 1) + LfLds::kMat, tid);
    lf_load(xk, Kr, roff(kLfRows * t0), tid, tb);
    lf_load(xv, Vr, roff(kLfRows * t0), tid, tb);
    lf_store(xk, slot(t0), tid);
    lf_store(xv, slot(t0) + LfLds::kMat, tid);
  } else {
    LfTile x;
    load_tile(x, t0);
    lf_stage_tile<T, DLT>(x, lds, ht);
  }
  __syncthreads();

  if (main_wave) {
    // ---- main waves: query pass, key pass and the completed blocks' dK, dV
    f32x4 ak0[4], av0[4];  // sums of keys 16wv.. of the carried block (t-1 at step t, then t)
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) ak0[dt] = av0[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // block j complete (its sums in ak0, av0): the global rows' part, then
    // dK, dV of keys 16wv.. stored.  Rows 0..G-1 are rewritten by the
    // combine: block 0's sums for them go to the extra slot of partials.
    auto finish_block = [&](int j, const typename P::Q& kr, const typename P::Q& vr) __attribute__((always_inline)) {
      const int k0 = kLfRows * j + 16 * wv;
      lf_global_rows_kv<P>(lds, kr, vr, k0, G, N, c, g, kl, trl, sl2, ak0, av0);
      if (j == 0 && wv == 0 && c < G) {
        store_part(a.nslot, 1, ak0);
        store_part(a.nslot, 2, av0);
      }
      const uint32_t row = roff(k0 + c);
      store_nat<T>(av0, 1.0f, DVr, row, g);
      store_nat<T>(ak0, a.scale, DKr, row, g);
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) ak0[dt] = av0[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };

    for (int t = t0; t <= s1; ++t) {
      const bool more = t < s1;
      const bool own = t < t1;  // tile t's queries are this segment's
      Rows128 nk, nv;
      if (more) {  // step t+1's key block in flight
        lf_load(nk, Kr, roff(kLfRows * (t + 1)), tid, tb);
        lf_load(nv, Vr, roff(kLfRows * (t + 1)), tid, tb);
      }
      const float* st = reinterpret_cast<const float*>(lds + LfLds::kSt);

      if (own) {
        // ---- query pass: queries i = 128t + 16wv + c, keys 4g + r of each sub-tile
        const int i = kLfRows * t + 16 * wv + c;
        typename P::Q qb, gb;
        lf_lds_q<P>(qb, lds + LfLds::kQ, 16 * wv + c, g);
        lf_lds_q<P>(gb, lds + LfLds::kG, 16 * wv + c, g);
        const float lse2c = st[16 * wv + c], dltc = st[kLfRows + 16 * wv + c];
        float lse2[4], dlt[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          lse2[r] = lse2c;
          dlt[r] = dltc;
        }
        f32x4 acc[4];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        {  // the global keys 0..G-1 outside the row's band
          const f32x4 s = P::qk(lds + LfLds::kGK + kl, qb);
          const f32x4 dp = P::qk(lds + LfLds::kGV + kl, gb);
          bool keep[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) keep[r] = 4 * g + r < G && i - (4 * g + r) > L;
          float p[4], ds[4];
          lf_probs(s, dp, lse2, dlt, keep, sl2, p, ds);
          pv_tr<T>(lds + LfLds::kGK + trl, pack4<T>(ds), acc);
        }
        // window sub-tiles s = 8t + wv - 8 + jj (keys 16s..16s+15), jj = 0..8,
        // in blocks t-1 and t, i - key = 16(8 - jj) + c - (4g + r); one
        // 16x16x16 MFMA per sub-tile and head_dim tile.  (Pairing sub-tiles on
        // 16x16x32 MFMA here, with each pair's products issued between the
        // next sub-tile's scores, gave intermittently wrong dQ for whole waves
        // on the device; the one-sub-tile form, the same MFMA work, did not
        // in any of the repeated runs.)
#pragma unroll
        for (int jj = 0; jj < 9; ++jj) {
          const int s = 8 * t + wv - 8 + jj;
          const uint32_t sub = (uint32_t)((s >> 3) & 1) * LfLds::kSlot + 16 * (s & 7) * LfLds::kRow;
          const f32x4 sc = P::qk(lds + sub + kl, qb);
          const f32x4 dp = P::qk(lds + sub + LfLds::kMat + kl, gb);
          const float l2 = s < 0 ? __builtin_inff() : lse2c;  // keys below row 0 (tile 0): no pair
          float ls[4], p[4], ds[4];
          int dq[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            ls[r] = l2;
            dq[r] = 16 * (8 - jj) + c - (4 * g + r);
          }
          if (!FIXED127)
            lf_probs_m<kLfBand>(sc, dp, ls, dlt, dq, L, c, g, sl2, p, ds);
          else if (jj == 0)
            lf_probs_m<kLfColBefore>(sc, dp, ls, dlt, dq, L, c, g, sl2, p, ds);
          else if (jj == 8)
            lf_probs_m<kLfColFrom>(sc, dp, ls, dlt, dq, L, c, g, sl2, p, ds);
          else
            lf_probs_m<kLfAll>(sc, dp, ls, dlt, dq, L, c, g, sl2, p, ds);
          pv_tr<T>(lds + sub + trl, pack4<T>(ds), acc);
        }
        store_nat<T>(acc, a.scale, DQr, i >= G && i < N ? roff(i) : kOob, g);
      }

      // ---- key pass: tile t's queries into keys 16wv.. of blocks t-1 and t
      const int q0 = kLfRows * t;
      if (t > t0) {  // block t-1 is this segment's: query sub-tiles 0..wv reach its keys
        typename P::Q kr, vr;
        lf_lds_q<P>(kr, slot(t - 1), 16 * wv + c, g);
        lf_lds_q<P>(vr, slot(t - 1) + LfLds::kMat, 16 * wv + c, g);
        const int k0 = kLfRows * (t - 1) + 16 * wv;
        if (FIXED127) {  // i - key = 128 + 16(jq - wv) + (4g + r) - c
          lf_kpass<P, kLfAll>(lds, kr, vr, k0, q0, 0, wv - 1, L, c, g, kl, trl, sl2, ak0, av0);
          lf_kpass<P, kLfColAfter>(lds, kr, vr, k0, q0, wv, wv, L, c, g, kl, trl, sl2, ak0, av0);
        } else {
          lf_kpass<P, kLfBand>(lds, kr, vr, k0, q0, 0, wv, L, c, g, kl, trl, sl2, ak0, av0);
        }
        finish_block(t - 1, kr, vr);
      }
      if (own) {  // block t: query sub-tiles wv..7
        typename P::Q kr, vr;
        lf_lds_q<P>(kr, slot(t), 16 * wv + c, g);
        lf_lds_q<P>(vr, slot(t) + LfLds::kMat, 16 * wv + c, g);
        const int k0 = kLfRows * t + 16 * wv;
        if (FIXED127) {  // i - key = 16(jq - wv) + (4g + r) - c
          lf_kpass<P, kLfColUpTo>(lds, kr, vr, k0, q0, wv, wv, L, c, g, kl, trl, sl2, ak0, av0);
          lf_kpass<P, kLfAll>(lds, kr, vr, k0, q0, wv + 1, kLfWaves - 1, L, c, g, kl, trl, sl2, ak0, av0);
        } else {
          lf_kpass<P, kLfBand>(lds, kr, vr, k0, q0, wv, kLfWaves - 1, L, c, g, kl, trl, sl2, ak0, av0);
        }
        if (t == nt - 1) finish_block(t, kr, vr);  // no tile t+1: block t is complete too
      }

      // step t+1's rows replace block t-1 and tile t, which every pass has read
      __syncthreads();
      if (more) {
        lf_store(nk, slot(t + 1), tid);
        lf_store(nv, slot(t + 1) + LfLds::kMat, tid);
        __syncthreads();
      }
    }
    // the helpers' segment-end reduction: the same barriers
    for (int half = kLfHelpers / 2; half >= 1; half >>= 1) {  // uniform
      __syncthreads();
      __syncthreads();
    }
  } else {
    // ---- helper waves: the next tile's loads; the global keys' dK, dV from
    // query sub-tiles 2wv, 2wv+1 (key as the MFMA column, pairs outside the
    // band) and the global rows' dQ from key sub-tiles 2wv, 2wv+1 of each
    // completed block, summed over the segment
    f32x4 agq[4], agk[4], agv[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) agq[dt] = agk[dt] = agv[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto global_rows_dq = [&](int j) __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int ks = 2 * wv + e;
        const uint8_t* krows = slot(j) + 16 * ks * LfLds::kRow;
        lf_global_rows_dq<P>(lds, krows, krows + LfLds::kMat, kLfRows * j + 16 * ks, G, N, c, g, kl, trl, sl2,
                             agq);
      }
    };
    for (int t = t0; t <= s1; ++t) {
      const bool more = t < s1;
      const bool own = t < t1;
      LfTile nx;
      if (more) load_tile(nx, t + 1);  // step t+1's query tile in flight
      const float* st = reinterpret_cast<const float*>(lds + LfLds::kSt);
      if (own) {
        typename P::Q kg, vg;
        lf_lds_q<P>(kg, lds + LfLds::kGK, c, g);
        lf_lds_q<P>(vg, lds + LfLds::kGV, c, g);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int qs = 2 * wv + e;  // query sub-tile
          const uint8_t* qrows = lds + LfLds::kQ + 16 * qs * LfLds::kRow;
          const uint8_t* grows = lds + LfLds::kG + 16 * qs * LfLds::kRow;
          const f32x4 s = P::qk(qrows + kl, kg);  // S[query 4g + r][global key c]
          const f32x4 dp = P::qk(grows + kl, vg);
          const f32x4 l4 = *reinterpret_cast<const f32x4*>(st + 16 * qs + 4 * g);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(st + kLfRows + 16 * qs + 4 * g);
          float lq[4], dq4[4], p[4], ds[4];
          bool keep[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            keep[r] = c < G && kLfRows * t + 16 * qs + 4 * g + r - c > L;
            lq[r] = l4[r];
            dq4[r] = d4[r];
          }
          lf_probs(s, dp, lq, dq4, keep, sl2, p, ds);
          pv_tr_split<T>(grows + trl, p, agv);
          pv_tr_split<T>(qrows + trl, ds, agk);
        }
      }
      if (t > t0) global_rows_dq(t - 1);
      if (own && t == nt - 1) global_rows_dq(t);
      __syncthreads();
      if (more) {
        lf_stage_tile<T, DLT>(nx, lds, ht);
        __syncthreads();
      }
    }
    // ---- the segment's global sums: the 4 helpers' sums added pairwise in LDS
    // (the ring is free: the loop ended on a barrier), then written by helper
    // 0 as natural-order rows: [3][16][64], row c, head_dim 16dt + 4g + r
    f32x4* red = reinterpret_cast<f32x4*>(lds);
    for (int half = kLfHelpers / 2; half >= 1; half >>= 1) {  // uniform
      if (wv >= half && wv < 2 * half) {
        f32x4* w = red + (wv - half) * 12 * 64 + lane;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          w[(0 + dt) * 64] = agq[dt];
          w[(4 + dt) * 64] = agk[dt];
          w[(8 + dt) * 64] = agv[dt];
        }
      }
      __syncthreads();
      if (wv < half) {
        const f32x4* w = red + wv * 12 * 64 + lane;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          agq[dt] += w[(0 + dt) * 64];
          agk[dt] += w[(4 + dt) * 64];
          agv[dt] += w[(8 + dt) * 64];
        }
      }
      __syncthreads();
    }
    if (wv == 0) {
      store_part(slot_id, 0, agq);
      store_part(slot_id, 1, agk);
      store_part(slot_id, 2, agv);
    }
  }
}

// The streams' query tiles in order, (batch, head) after (batch, head), are
// dealt to the workgroups in equal runs of per_wg tiles (per_wg at most one
// stream's tiles), so that one round of one workgroup per CU has no idle CU
// and no run longer than the average (cfg4: 24 tiles each on 256 CUs,
// against 26 on 240 with whole chunks per stream).  A run that crosses the
// end of a stream continues at the next stream's start: a second segment,
// with its own prologue and partial slot (the workgroup's index among those
// whose runs meet that stream).
template <class P, bool FIXED127, bool DLT>
__global__ __launch_bounds__(kLfThreads, 1) void bwd_lf_kernel(LfArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // LfLds
  const int nt = (a.N + kLfRows - 1) / kLfRows;
  const int64_t g0 = (int64_t)blockIdx.x * a.per_wg;
  const int64_t g1 = min(g0 + a.per_wg, (int64_t)a.streams * nt);
  const int bh = (int)(g0 / nt);
  const int64_t s0 = (int64_t)bh * nt;
  const int t0 = (int)(g0 - s0);
  const int t1 = (int)min(g1 - s0, (int64_t)nt);
  const int t1b = (int)(g1 - s0 - nt);  // > 0: tiles [0, t1b) of stream bh + 1
  const int slot2 = (int)(blockIdx.x - (s0 + nt) / a.per_wg);
  lf_segment<P, FIXED127, DLT>(a, lds, bh, t0, t1, (int)(blockIdx.x - s0 / a.per_wg));
  if (t1b > 0) {  // uniform
    __syncthreads();  // the first segment's LDS reads are done
    lf_segment<P, FIXED127, DLT>(a, lds, bh + 1, 0, t1b, slot2);
  }
}

// Rows 0..G-1 of dQ, dK, dV: the sums of a (batch, head)'s segment partials
// (in tile order; for dK and dV also the extra slot of block 0's sums), dQ
// and dK times the scale.  One thread per element of the [3][16][64] part:
// kLfCombineBlocks workgroups of 256 per (batch, head), so the partial loads of
// many elements are in flight together.
constexpr int kLfCombineBlocks = kLfPart / 256;
template <typename T>
__global__ __launch_bounds__(256) void bwd_lf_combine(LfArgs a) {
  const int bh = blockIdx.x / kLfCombineBlocks;
  const int e = (blockIdx.x % kLfCombineBlocks) * 256 + threadIdx.x;
  const int m = e / (16 * kHeadDim), r = (e / kHeadDim) % 16, d = e % kHeadDim;
  if (r >= min(a.G, a.N)) return;
  const int h = bh % a.H;
  const int b = bh / a.H;
  const float* p = a.part + (int64_t)bh * (a.nslot + 1) * kLfPart + e;
  const int nt = (a.N + kLfRows - 1) / kLfRows;
  // the workgroups whose runs meet this stream, in tile order
  const int slots = (int)(((int64_t)(bh + 1) * nt - 1) / a.per_wg - (int64_t)bh * nt / a.per_wg + 1);
  // 16 partial loads in flight at once (indices clamped, so unconditional),
  // then the adds in tile order: one load round trip per 16 partials (a
  // rolled remainder loop waited out one per partial: 5.1 us at cfg4)
  float s = 0.0f;
  for (int c0 = 0; c0 < slots; c0 += 16) {
    float v[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k] = p[(int64_t)min(c0 + k, slots - 1) * kLfPart];
#pragma unroll
    for (int k = 0; k < 16; ++k)
      if (c0 + k < slots) s += v[k];
  }
  if (m != 0) s += p[(int64_t)a.nslot * kLfPart];  // block 0's sums of keys 0..G-1
  T* out = static_cast<T*>(m == 0 ? a.dq : m == 1 ? a.dk : a.dv);
  out[((int64_t)b * a.N * a.H + h) * kHeadDim + (int64_t)r * a.H * kHeadDim + d] =
      static_cast<T>(m == 2 ? s : s * a.scale);
}

}  // namespace ma_dev
