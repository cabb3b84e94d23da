// tile_kernel.h -- explicit key sets (INDEX_SET) on 64x64 MFMA tiles, head
// dim 64, bf16/fp16 (16x16x32 MFMA) and fp32 (16x16x4).
//
// The set comes as a tile plan (ma_attn_tile_plan): the (query tile, key
// block) entries that hold any key, each with 64 row masks (bit k of word r:
// key 64*blk + k in S_(64*tile + r)) and their transpose.  An entry whose
// 64x64 pairs are all in the set is flagged full and computed unmasked.
// Work items are runs of at most `seg` entries of one query tile (or one
// key block): a tile with more is split over several items whose partial
// results a combine kernel merges, so one long row (a Longformer global row,
// a global key's column) does not hold up the launch.
//
//   tile_fwd_kernel      O (or, with STATS, a split tile's backward {lse2,
//                        delta} partials): one workgroup per (batch, head,
//                        item), 4 waves x 16
//                        queries; key blocks through a two-buffer LDS ring
//                        with the next block (and its mask word) in flight,
//                        online softmax in registers.
//   tile_combine_kernel  log-sum-exp merge of a split tile's partials.
//   tile_dq_kernel       dQ over a query tile's entries (an unsplit tile
//                        first computes its own statistics in a pass over
//                        them): K and V rows (16-bit, K^T through the
//                        LDS transpose read; fp32 stages K as (K, K^T)); dS in
//                        registers, dQ^T += K^T dS^T.
//   tile_dkv_kernel      dK, dV over a key block's entries: each entry's
//                        query tile staged as Q and dO rows (16-bit; fp32
//                        (Q, Q^T), (dO, dO^T)) and its 64 statistics;
//                        dV^T += dO^T P, dK^T += Q^T dS.
//   tile_sum_kernel      sums a split tile's (or key block's) partial dQ /
//                        dK, dV.
// Each output row has one writer; no atomics.  Every global access is a
// range-checked buffer operation on the (batch, head) stream or an index
// inside the plan's arrays.
#pragma once

#include "backward_kernel.h"
#include "block_kernel.h"

namespace ma_dev {

constexpr int kTileFull = 1 << 30;   // entry flag: every pair of the 64x64 block is in the set
constexpr int kTileSeg = 32;        // default entries per work item
constexpr int kTilePart = 68;        // floats per row of a forward partial: 64 O, log2 max, sum, 2 pad

struct TileArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;
  void* o;  // forward: O; backward: dQ
  void* dk;
  void* dv;
  const int32_t* blk;     // [entries] key block | kTileFull
  const uint64_t* mask;   // [entries][64] row masks
  const uint64_t* kmask;  // [entries][64] column masks
  const int32_t* etile;   // [entries] query tile of the entry
  const int32_t* kentry;  // [entries] entry ids by key block
  const int32_t* items;   // [nitems][4]
  const int32_t* split;   // [nsplit][4]
  float* stats;           // [B*N*H][2] {lse2, delta}
  float* part;            // [B*H][npart][...] partial results of split items
  float* lse;             // forward: optional output of each row's statistic (store_lse); backward from
                          // saved statistics: the forward's, read
  const void* fo;         // backward from saved statistics: the forward's O (delta = dO . O)
  int32_t N, H, nitems, nsplit, npart;
  int32_t nent, ntiles;  // plan sizes: every index read from the plan is clamped to them
  float scale, scale_log2;
};

__device__ __forceinline__ int clampi(int x, int lo, int hi) { return x < lo ? lo : (x > hi ? hi : x); }

// Work item `it` of the plan: (tile or key block, first, end, slot), clamped
// so that any plan content stays inside the plan's arrays.
struct TileItem {
  int id, e0, e1, slot;
};
__device__ __forceinline__ TileItem tile_item(const TileArgs& a, int it) {
  TileItem w;
  w.id = clampi(a.items[4 * it], 0, a.ntiles - 1);
  w.e0 = clampi(a.items[4 * it + 1], 0, a.nent);
  w.e1 = clampi(a.items[4 * it + 2], w.e0, a.nent);
  w.slot = clampi(a.items[4 * it + 3], -1, a.npart - 1);
  return w;
}

// Scores of one 64-key (or 64-query) block whose bit w of `m` keeps element
// 16u + 4g + rr: sc[u][rr] with w = 16u + 4g + rr.
__device__ __forceinline__ void apply_mask(f32x4 (&sc)[4], uint64_t m, int g) {
  const uint32_t lo = (uint32_t)m, hi = (uint32_t)(m >> 32);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t w = (u < 2 ? lo : hi) >> (16 * (u & 1) + 4 * g);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sc[u][rr] = (w >> rr) & 1u ? sc[u][rr] : -INFINITY;
  }
}

// Wave-uniform mask of the 16-wide sub-tiles of an entry that hold a pair of
// this wave's 16 rows: bit u is set when some lane's mask word (its row's
// keys, or its key's queries) has a bit in 16u..16u+15.  Empty sub-tiles are
// not computed: a Longformer global key block holds one live sub-tile of
// four, and a causal window's edge blocks are triangles of sub-tiles.
__device__ __forceinline__ int live_subtiles(uint64_t mw, bool full) {
  if (full) return 0xF;  // uniform
  int live = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u)
    live |= (__builtin_amdgcn_ballot_w64(((mw >> (16 * u)) & 0xFFFFull) != 0) != 0 ? 1 : 0) << u;
  return live;
}

// Compile-time "every sub-tile live": a full entry's products issue back to
// back with no per-sub-tile branch.
template <bool B>
struct AllLive {
  static constexpr bool value = B;
};

// dot(x, O) of one query row over the head_dim values this lane holds (x in
// the Q register layout of P, which is also the accumulator layout).
template <class P>
__device__ __forceinline__ float lane_dot(const typename P::Q& x, const f32x4 (&acc)[4]) {
  float d = 0.0f;
  if constexpr (P::kSPB == 1) {
    using T = typename P::Elt;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t w[4] = {x.r[h].x, x.r[h].y, x.r[h].z, x.r[h].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = static_cast<float>(__builtin_bit_cast(T, (uint16_t)(w[j] & 0xffffu)));
        const float hi = static_cast<float>(__builtin_bit_cast(T, (uint16_t)(w[j] >> 16)));
        const f32x4& a = acc[2 * h + (j >> 1)];
        d = fmaf(lo, a[2 * (j & 1)], d);
        d = fmaf(hi, a[2 * (j & 1) + 1], d);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 xv = __builtin_bit_cast(f32x4, x.r[j]);
#pragma unroll
      for (int r = 0; r < 4; ++r) d = fmaf(xv[r], acc[j][r], d);
    }
  }
  return d;
}

// One 64-key block of the lane's query row into the online softmax.
template <class P, bool ALL>
__device__ __forceinline__ void tile_update_live(const uint8_t* slot, uint32_t kl, uint32_t vl,
                                                 const typename P::Q& q, bool full, uint64_t mw, int live, int g,
                                                 float sl2, float& m_run, float& l_run, f32x4 (&acc)[4]) {
  f32x4 sc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if (ALL || (live >> u & 1))
      sc[u] = P::qk(slot + P::blk_k(u) + kl, q);
    else
      sc[u] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  }
  if (!full) apply_mask(sc, mw, g);  // uniform
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < 4; ++u) mx = fmaxf(mx, fmaxf(fmaxf(sc[u][0], sc[u][1]), fmaxf(sc[u][2], sc[u][3])));
  const float m_new = fmaxf(m_run, col_max(mx));
  const float m_use = m_new == -INFINITY ? 0.0f : m_new * sl2;
  if (__builtin_amdgcn_ballot_w64(m_new != m_run) != 0) {
    const float corr = __builtin_amdgcn_exp2f(m_run * sl2 - m_use);  // 0 on a row's first live block
    l_run *= corr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] *= corr;
  }
  m_run = m_new;
#pragma unroll
  for (int u = 0; u < 4; u += 2) {
    if (!ALL && !(live >> u & 3)) continue;  // uniform: both sub-tiles empty
    float p0[4], p1[4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      p0[rr] = __builtin_amdgcn_exp2f(fmaf(sc[u][rr], sl2, -m_use));
      p1[rr] = __builtin_amdgcn_exp2f(fmaf(sc[u + 1][rr], sl2, -m_use));
      l_run += p0[rr] + p1[rr];
    }
    P::pv2(slot + P::blk_v(u) + vl, slot + P::blk_v(u + 1) + vl, p0, p1, acc);
  }
}

// MASKED false: the plan has no masked entry, every sub-tile is live.
template <class P, bool MASKED>
__device__ __forceinline__ void tile_update(const uint8_t* slot, uint32_t kl, uint32_t vl, const typename P::Q& q,
                                            bool full, uint64_t mw, int g, float sl2, float& m_run, float& l_run,
                                            f32x4 (&acc)[4]) {
  const int live = MASKED ? live_subtiles(mw, full) : 0xF;
  if (live == 0xF)  // uniform
    tile_update_live<P, true>(slot, kl, vl, q, full, mw, live, g, sl2, m_run, l_run, acc);
  else if (live)  // no key of this block for the wave's rows: nothing to add
    tile_update_live<P, false>(slot, kl, vl, q, full, mw, live, g, sl2, m_run, l_run, acc);
}

struct TileCtx {
  int b, h, bh;
  uint32_t tb;
  int64_t base;
  uint32_t nrec;
};

template <class P>
__device__ __forceinline__ TileCtx tile_ctx(const TileArgs& a, int bh) {
  TileCtx x;
  x.bh = bh;
  x.h = bh % a.H;
  x.b = bh / a.H;
  x.tb = (uint32_t)a.H * kHeadDim * sizeof(typename P::Elt);
  x.base = ((int64_t)x.b * a.N * a.H + x.h) * kHeadDim;
  x.nrec = (uint32_t)((int64_t)(a.N - 1) * x.tb + kHeadDim * sizeof(typename P::Elt));
  return x;
}

// ---------------------------------------------------------------- forward / statistics

template <class P, bool STATS, bool MASKED>
__global__ __launch_bounds__(256, P::kMinBlocks) void tile_fwd_kernel(TileArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // 2 block buffers of P::kBlk bytes
  using Elt = typename P::Elt;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  const int wg = xcd_row_order(blockIdx.x, gridDim.x);
  const int it = wg % a.nitems;
  const TileCtx x = tile_ctx<P>(a, wg / a.nitems);
  const TileItem w = tile_item(a, it);
  const int t = w.id, e0 = w.e0, e1 = w.e1, slot = w.slot;
  if (STATS && slot < 0) return;  // uniform: an unsplit tile's statistics come from its dQ pass
  const uint32_t tb = x.tb;
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + x.base, x.nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + x.base, x.nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + x.base, x.nrec);

  const int ql = 16 * wv + c;  // the lane's query row within the tile
  const uint32_t qrow = (uint32_t)(64 * t + ql) * tb;
  typename P::Q q;
  P::load_q(q, Qr, qrow, g);
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);

  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const float sl2 = a.scale_log2;

  if (e1 - e0 <= 2 && e0 < e1) {  // uniform
    // Both blocks are loaded at once and the two entries run with no
    // barrier between them, so each wave computes only its own live
    // sub-tiles of the two (a causal window's edge blocks are triangles).
    const int fa = a.blk[e0], fb = e0 + 1 < e1 ? a.blk[e0 + 1] : 0;
    BlkSlots<P> xa, xb;
    load_blk<P>(xa, Kr, Vr, (uint32_t)(64 * (fa & (kTileFull - 1))) * tb, tid, tb);
    load_blk<P>(xb, Kr, Vr, e0 + 1 < e1 ? (uint32_t)(64 * (fb & (kTileFull - 1))) * tb : kOob, tid, tb);
    const uint64_t ma = a.mask[(int64_t)e0 * 64 + ql];
    const uint64_t mb = e0 + 1 < e1 ? a.mask[(int64_t)(e0 + 1) * 64 + ql] : 0;
    store_blk<P>(xa, ring, tid);
    if (e0 + 1 < e1) store_blk<P>(xb, ring + P::kBlk, tid);
    __syncthreads();
    tile_update<P, MASKED>(ring, kl, vl, q, (fa & kTileFull) != 0, ma, g, sl2, m_run, l_run, acc);
    if (e0 + 1 < e1)
      tile_update<P, MASKED>(ring + P::kBlk, kl, vl, q, (fb & kTileFull) != 0, mb, g, sl2, m_run, l_run, acc);
  } else if (e0 < e1) {  // uniform
    // entry e+2's flags word is read at step e (f0, f1: entries e, e+1)
    int f0 = a.blk[e0];
    int f1 = e0 + 1 < e1 ? a.blk[e0 + 1] : 0;
    auto off_of = [&](int e, int f) { return e < e1 ? (uint32_t)(64 * (f & (kTileFull - 1))) * tb : kOob; };
    BlkSlots<P> nxt;
    load_blk<P>(nxt, Kr, Vr, off_of(e0, f0), tid, tb);
    uint64_t mw_next = a.mask[(int64_t)e0 * 64 + ql];
    store_blk<P>(nxt, ring, tid);
    __syncthreads();
    for (int e = e0; e < e1; ++e) {
      const bool full = (f0 & kTileFull) != 0;
      const uint64_t mw = mw_next;
      load_blk<P>(nxt, Kr, Vr, off_of(e + 1, f1), tid, tb);
      if (e + 1 < e1) mw_next = a.mask[(int64_t)(e + 1) * 64 + ql];
      const int f2 = e + 2 < e1 ? a.blk[e + 2] : 0;
      tile_update<P, MASKED>(ring + ((e - e0) & 1) * P::kBlk, kl, vl, q, full, mw, g, sl2, m_run, l_run, acc);
      // the next block goes into the buffer the previous one used (every
      // wave passed the barrier that ended it)
      if (e + 1 < e1) store_blk<P>(nxt, ring + ((e + 1 - e0) & 1) * P::kBlk, tid);
      __syncthreads();
      f0 = f1;
      f1 = f2;
    }
  }
  const float l_tot = col_sum(l_run);
  if (slot < 0) {
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if constexpr (!STATS) {
      const __amdgpu_buffer_rsrc_t Or = make_rsrc(static_cast<Elt*>(a.o) + x.base, x.nrec);
      P::store_o(acc, inv, Or, qrow, g);
      const int64_t i = 64 * (int64_t)t + ql;
      store_lse(a.lse, ((int64_t)x.b * a.N + i) * a.H + x.h, i < a.N, m_run, l_tot, sl2, g);
    } else {
      // delta = dout . O of the row (O in fp32 registers), lse2 in log2 units
      const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const Elt*>(a.dout) + x.base, x.nrec);
      typename P::Q gq;
      P::load_q(gq, Gr, qrow, g);
      const float dlt = col_sum(lane_dot<P>(gq, acc)) * inv;
      const float lse2 = l_tot > 0.0f ? m_run * sl2 + __log2f(l_tot) : 0.0f;
      const int64_t i = 64 * (int64_t)t + ql;
      if (g == 0 && i < a.N)
        *reinterpret_cast<float2*>(a.stats + 2 * (((int64_t)x.b * a.N + i) * a.H + x.h)) = make_float2(lse2, dlt);
    }
  } else {
    float* dst = a.part + (((int64_t)x.bh * a.npart + slot) * 64 + ql) * kTilePart;
    P::store_acc(acc, dst, g);
    if (g == 0) *reinterpret_cast<float2*>(dst + 64) = make_float2(m_run == -INFINITY ? -INFINITY : m_run * sl2, l_tot);
  }
}

// Merge of a split query tile's partials.  Workgroup (split tile, 16-row
// quarter of the tile); thread (row tid/16, column tid%16) owns head_dim
// 4*column .. +3 of one row, so a tile's merge spreads over 4 workgroups of
// independent, unrolled partial loads (the partials of one split tile are
// read once).
constexpr int kMergeRows = 16;  // rows per merge workgroup
template <typename Elt, bool STATS>
__global__ __launch_bounds__(256) void tile_combine_kernel(TileArgs a) {
  constexpr int kQuarters = 64 / kMergeRows;
  const int rq = blockIdx.x % kQuarters;
  const int s = (blockIdx.x / kQuarters) % a.nsplit;
  const int bh = blockIdx.x / kQuarters / a.nsplit;
  const int h = bh % a.H, b = bh / a.H;
  const int t = clampi(a.split[4 * s], 0, a.ntiles - 1);
  const int first = clampi(a.split[4 * s + 1], 0, a.npart);
  const int cnt = clampi(a.split[4 * s + 2], 0, a.npart - first);
  const int row = kMergeRows * rq + (threadIdx.x >> 4), col = threadIdx.x & 15;
  const float* p0 = a.part + (((int64_t)bh * a.npart + first) * 64 + row) * kTilePart;
  constexpr int64_t kStride = 64 * kTilePart;
  float m = -INFINITY;
#pragma unroll 8
  for (int k = 0; k < cnt; ++k) m = fmaxf(m, p0[k * kStride + 64]);
  float l = 0.0f;
  f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  if (m != -INFINITY) {
#pragma unroll 8
    for (int k = 0; k < cnt; ++k) {
      const float* src = p0 + k * kStride;
      const float w = __builtin_amdgcn_exp2f(src[64] - m);  // 0 for a partial that saw no key
      l = fmaf(src[65], w, l);
      const f32x4 v = *reinterpret_cast<const f32x4*>(src + 4 * col);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = fmaf(v[j], w, o[j]);
    }
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const int64_t i = 64 * (int64_t)t + row;
  const int64_t off = (((int64_t)b * a.N + i) * a.H + h) * kHeadDim + 4 * col;
  if constexpr (!STATS) {
    if (i >= a.N) return;
    Elt* dst = static_cast<Elt*>(a.o) + off;
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j] = static_cast<Elt>(o[j] * inv);
    // m is already in log2 units of the scaled scores here
    if (a.lse && col == 0) a.lse[((int64_t)b * a.N + i) * a.H + h] = l > 0.0f ? m + __log2f(l) : 0.0f;
  } else {
    float dlt = 0.0f;
    if (i < a.N) {
      const Elt* gsrc = static_cast<const Elt*>(a.dout) + off;
#pragma unroll
      for (int j = 0; j < 4; ++j) dlt = fmaf(static_cast<float>(gsrc[j]), o[j], dlt);
    }
    // the row's 16 columns are 16 consecutive lanes
    dlt += __shfl_xor(dlt, 1, 64);
    dlt += __shfl_xor(dlt, 2, 64);
    dlt += __shfl_xor(dlt, 4, 64);
    dlt += __shfl_xor(dlt, 8, 64);
    if (col == 0 && i < a.N)
      *reinterpret_cast<float2*>(a.stats + 2 * (((int64_t)b * a.N + i) * a.H + h)) =
          make_float2(l > 0.0f ? m + __log2f(l) : 0.0f, dlt * inv);
  }
}

// ---------------------------------------------------------------- dQ
//
// SAVED (a backward from the forward's saved statistics): every tile takes
// lse2 from the forward and delta = dO . O of its rows, and runs pass 2 only.
// Otherwise an unsplit tile (one work item) computes its own statistics: pass 1 over
// its entries gives {lse2, delta} (online max, sum of e and of e*dP, no O),
// pass 2 dQ; with at most two entries both blocks stay resident in the two
// buffers between the passes, and with more pass 2 runs backwards so that
// it starts on the two blocks pass 1 ended with.  A split tile's items read the statistics the
// merge of its partials wrote.  Every tile's statistics land in the
// workspace for the dK/dV pass.

// {lse2, delta} of the lane's query from pass 1's running sums (0, 0 for a
// row with no key).
__device__ __forceinline__ void tile_stats(float m_run, float l_run, float a_run, float sl2, float& lse2,
                                           float& dlt) {
  const float l_tot = col_sum(l_run), a_tot = col_sum(a_run);
  lse2 = l_tot > 0.0f ? m_run * sl2 + __log2f(l_tot) : 0.0f;
  dlt = l_tot > 0.0f ? a_tot / l_tot : 0.0f;
}

template <class P, bool MASKED, bool SAVED>
__global__ __launch_bounds__(256, P::kTrRows ? 3 : 2) void tile_dq_kernel(TileArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // 2 buffers x PairLds (K, V)
  using Elt = typename P::Elt;
  using PL = PairLds<P>;
  constexpr int kBuf = PL::kBytes;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  const int wg = xcd_row_order(blockIdx.x, gridDim.x);
  const int it = wg % a.nitems;
  const TileCtx x = tile_ctx<P>(a, wg / a.nitems);
  const TileItem w = tile_item(a, it);
  const int t = w.id, e0 = w.e0, e1 = w.e1, slot = w.slot;
  const uint32_t tb = x.tb;
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + x.base, x.nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + x.base, x.nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + x.base, x.nrec);
  const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const Elt*>(a.dout) + x.base, x.nrec);

  const int ql = 16 * wv + c;
  const int64_t i = 64 * (int64_t)t + ql;
  const uint32_t qrow = (uint32_t)i * tb;
  typename P::Q qr, gr;
  P::load_q(qr, Qr, qrow, g);
  P::load_q(gr, Gr, qrow, g);
  float* srow = a.stats + 2 * (((int64_t)x.b * a.N + i) * a.H + x.h);
  const bool own = !SAVED && slot < 0;  // uniform: statistics from its own first pass
  float lse2 = 0.0f, dlt = 0.0f;
  typename P::Q fo_row;  // SAVED: the row's O (delta = dO . O)
  if constexpr (SAVED) {
    const __amdgpu_buffer_rsrc_t Fr = make_rsrc(static_cast<const Elt*>(a.fo) + x.base, x.nrec);
    P::load_q(fo_row, Fr, qrow, g);
    if (i < a.N) lse2 = a.lse[((int64_t)x.b * a.N + i) * a.H + x.h];
  } else if (!own && i < a.N) {
    const float2 st = *reinterpret_cast<const float2*>(srow);
    lse2 = st.x;
    dlt = st.y;
  }
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);

  // items: pass 1 (own statistics only) over the entries, then pass 2
  const int ne = e1 - e0;
  const int nit = own ? 2 * ne : ne;
  const bool resident = ne <= 2;
  // Streamed order (more than two entries): pass 2 walks the entries in
  // reverse, so its first two blocks are still in the two buffers where
  // pass 1 left them; every block sits in the buffer of its entry's parity.
  auto entry_of = [&](int k) { return e0 + (own && k >= ne ? 2 * ne - 1 - k : k); };
  auto buf_of = [&](int k) { return (entry_of(k) - e0) & 1; };
  auto loads = [&](int k) { return k < nit && (!own || k < ne || k >= ne + 2); };

  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const float sl2 = a.scale_log2;
  float m_run = -INFINITY, l_run = 0.0f, a_run = 0.0f;

  // SAVED: delta once the first blocks' loads are in flight (it waits on the
  // O row's load), and both statistics for the dK/dV pass (every item of a
  // split tile writes the same values).
  auto saved_stats = [&]() __attribute__((always_inline)) {
    if constexpr (SAVED) {
      dlt = col_sum(bwd_row_dot<P>(gr, fo_row));
      if (g == 0 && i < a.N) *reinterpret_cast<float2*>(srow) = make_float2(lse2, dlt);
    }
  };

  // Step k's products on the block in buffer sk: pass 1 (statistics) or
  // pass 2 (dQ) of its entry.
  auto step_live = [&](auto all, int k, const uint8_t* sk, bool full, uint64_t mw, int live)
                       __attribute__((always_inline)) {
    constexpr bool kAll = decltype(all)::value;
    if (kAll) live = 0xF;
    f32x4 s[4], dp[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (kAll || (live >> u & 1)) {  // uniform
        s[u] = P::qk(sk + P::blk_k(u) + kl, qr);
        dp[u] = P::qk(sk + PL::kRows2 + P::blk_k(u) + kl, gr);
      } else {
        s[u] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        dp[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
    if (!full) apply_mask(s, mw, g);
    if (own && k < ne) {  // pass 1
      bwdq_pass1(s, dp, live, sl2, m_run, l_run, a_run);
      if (k == ne - 1) tile_stats(m_run, l_run, a_run, sl2, lse2, dlt);
    } else {
      bwdq_pass2<P>(sk, vl + PL::kT1, s, dp, live, sl2, lse2, dlt, acc);
    }
  };
  auto step = [&](int k, const uint8_t* sk, bool full, uint64_t mw) __attribute__((always_inline)) {
    const int live = MASKED ? live_subtiles(mw, full) : 0xF;
    if (live == 0xF)  // uniform
      step_live(AllLive<true>{}, k, sk, full, mw, live);
    else
      step_live(AllLive<false>{}, k, sk, full, mw, live);
  };

  if (resident && ne > 0) {  // uniform
    // Both blocks are loaded at once and the steps run with no barrier
    // between them, so each wave computes only its own live sub-tiles of
    // the two entries.  On a causal window one wave has all four sub-tiles
    // of one block and one of the other; with a barrier per step every step
    // would last as long as its busiest wave.
    const int fa = a.blk[e0];
    const int fb = ne > 1 ? a.blk[e0 + 1] : 0;
    KvRegs<P> xa, xb;
    kv_load<P>(xa, Kr, Vr, (uint32_t)(64 * (fa & (kTileFull - 1))) * tb, tid, tb);
    kv_load<P>(xb, Kr, Vr, ne > 1 ? (uint32_t)(64 * (fb & (kTileFull - 1))) * tb : kOob, tid, tb);
    const uint64_t ma = a.mask[(int64_t)e0 * 64 + ql];
    const uint64_t mb = ne > 1 ? a.mask[(int64_t)(e0 + 1) * 64 + ql] : 0;
    saved_stats();
    kv_store<P>(xa, ring, tid);
    if (ne > 1) kv_store<P>(xb, ring + kBuf, tid);
    __syncthreads();
    for (int k = 0; k < nit; ++k) {
      const int j = k < ne ? k : k - ne;
      step(k, ring + j * kBuf, ((j ? fb : fa) & kTileFull) != 0, j ? mb : ma);
    }
  } else if (nit > 0) {  // uniform
    // The flags word of step k+2's entry is read at step k, so that no
    // block's loads wait on a plan lookup (f0, f1: steps k, k+1).
    int f0 = a.blk[entry_of(0)];
    int f1 = nit > 1 ? a.blk[entry_of(1)] : 0;
    auto off_of = [&](int k, int f) { return loads(k) ? (uint32_t)(64 * (f & (kTileFull - 1))) * tb : kOob; };
    KvRegs<P> xk;
    kv_load<P>(xk, Kr, Vr, off_of(0, f0), tid, tb);
    uint64_t mw_next = a.mask[(int64_t)entry_of(0) * 64 + ql];
    saved_stats();
    kv_store<P>(xk, ring, tid);
    __syncthreads();
    for (int k = 0; k < nit; ++k) {
      const bool full = (f0 & kTileFull) != 0;
      const uint64_t mw = mw_next;
      kv_load<P>(xk, Kr, Vr, off_of(k + 1, f1), tid, tb);
      if (k + 1 < nit) mw_next = a.mask[(int64_t)entry_of(k + 1) * 64 + ql];
      const int f2 = k + 2 < nit ? a.blk[entry_of(k + 2)] : 0;
      step(k, ring + buf_of(k) * kBuf, full, mw);
      if (loads(k + 1)) {
        uint8_t* nx = ring + buf_of(k + 1) * kBuf;
        kv_store<P>(xk, nx, tid);
      }
      __syncthreads();
      f0 = f1;
      f1 = f2;
    }
  }
  if (nit == 0) saved_stats();  // SAVED, a tile with no key: its statistics still go to the dK/dV pass
  if (own) {
    if (ne == 0) tile_stats(m_run, l_run, a_run, sl2, lse2, dlt);  // a tile with no key: zeros
    if (g == 0 && i < a.N) *reinterpret_cast<float2*>(srow) = make_float2(lse2, dlt);
  }
  if (slot < 0) {
    const __amdgpu_buffer_rsrc_t DQr = make_rsrc(static_cast<Elt*>(a.o) + x.base, x.nrec);
    P::store_o(acc, a.scale, DQr, qrow, g);
  } else {
    P::store_acc(acc, a.part + (((int64_t)x.bh * a.npart + slot) * 64 + ql) * 64, g);
  }
}

// ---------------------------------------------------------------- dK, dV

template <class P, bool MASKED>
__global__ __launch_bounds__(256, P::kTrRows ? 3 : 2) void tile_dkv_kernel(TileArgs a) {
  // 2 buffers x (PairLds (Q, dO), 64 lse2, 64 delta)
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];
  using Elt = typename P::Elt;
  using PL = PairLds<P>;
  constexpr int kBuf = PL::kBytes + 512;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  const int wg = xcd_row_order(blockIdx.x, gridDim.x);
  const int it = wg % a.nitems;
  const TileCtx x = tile_ctx<P>(a, wg / a.nitems);
  const TileItem w = tile_item(a, it);
  const int kb = w.id, p0 = w.e0, p1 = w.e1, slot = w.slot;
  const uint32_t tb = x.tb;
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + x.base, x.nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + x.base, x.nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + x.base, x.nrec);
  const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const Elt*>(a.dout) + x.base, x.nrec);
  // statistics of the (batch, head): row i at float2 index i * H
  const uint32_t sstride = (uint32_t)a.H * 8u;
  const __amdgpu_buffer_rsrc_t Sr =
      make_rsrc(a.stats + 2 * ((int64_t)x.b * a.N * a.H + x.h), (uint32_t)(a.N - 1) * sstride + 8u);

  const int kl_ = 16 * wv + c;  // the lane's key within the block
  const uint32_t krow = (uint32_t)(64 * kb + kl_) * tb;
  typename P::Q kr, vr;
  P::load_q(kr, Kr, krow, g);
  P::load_q(vr, Vr, krow, g);
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);
  const uint32_t vq = vl + PL::kT1, vg = vl + PL::kT2;  // lane offsets of the Q^T and dO^T reads

  auto ent = [&](int p) { return clampi(a.kentry[p], 0, a.nent - 1); };
  auto tile_of = [&](int p) { return clampi(a.etile[ent(p)], 0, a.ntiles - 1); };
  auto q_off = [&](int p) { return p < p1 ? (uint32_t)(64 * tile_of(p)) * tb : kOob; };
  // thread tid < 64 carries the statistics of query row tid of the entry's tile
  auto st_off = [&](int p) { return p < p1 && tid < 64 ? (uint32_t)(64 * tile_of(p) + tid) * sstride : kOob; };

  f32x4 acc_k[4], acc_v[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc_k[dt] = acc_v[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const float sl2 = a.scale_log2;

  // One entry's products on the query block in buffer sq (Q, dO rows, then
  // the block's statistics).
  auto step_live = [&](auto all, const uint8_t* sq, bool full, uint64_t mw, int live)
                       __attribute__((always_inline)) {
    constexpr bool kAll = decltype(all)::value;
    const uint8_t* sg = sq + PL::kRows2;
    const float* stf = reinterpret_cast<const float*>(sq + PL::kBytes);
    f32x4 s[4], dp[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (kAll || (live >> u & 1)) {  // uniform
        s[u] = P::qk(sq + P::blk_k(u) + kl, kr);   // S[query 16u+4g+r][key c]
        dp[u] = P::qk(sg + P::blk_k(u) + kl, vr);  // dP[query][key c]
      } else {
        s[u] = f32x4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
        dp[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
    if (!full) apply_mask(s, mw, g);
#pragma unroll
    for (int u = 0; u < 4; u += 2) {
      if (!kAll && !(live >> u & 3)) continue;  // uniform: both sub-tiles empty
      const f32x4 lse0 = *reinterpret_cast<const f32x4*>(stf + 16 * u + 4 * g);
      const f32x4 dl0 = *reinterpret_cast<const f32x4*>(stf + 64 + 16 * u + 4 * g);
      const f32x4 lse1 = *reinterpret_cast<const f32x4*>(stf + 16 * (u + 1) + 4 * g);
      const f32x4 dl1 = *reinterpret_cast<const f32x4*>(stf + 64 + 16 * (u + 1) + 4 * g);
      float pa[4], pb[4], da[4], db[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        pa[r] = __builtin_amdgcn_exp2f(fmaf(s[u][r], sl2, -lse0[r]));
        pb[r] = __builtin_amdgcn_exp2f(fmaf(s[u + 1][r], sl2, -lse1[r]));
        da[r] = pa[r] * (dp[u][r] - dl0[r]);
        db[r] = pb[r] * (dp[u + 1][r] - dl1[r]);
      }
      P::pv2(sq + P::blk_v(u) + vg, sq + P::blk_v(u + 1) + vg, pa, pb, acc_v);  // dV^T += dO^T P
      P::pv2(sq + P::blk_v(u) + vq, sq + P::blk_v(u + 1) + vq, da, db, acc_k);  // dK^T += Q^T dS
    }
  };
  auto step = [&](const uint8_t* sq, bool full, uint64_t mw) __attribute__((always_inline)) {
    // query sub-tiles that list one of the wave's keys
    const int live = MASKED ? live_subtiles(mw, full) : 0xF;
    if (live == 0xF)  // uniform
      step_live(AllLive<true>{}, sq, full, mw, live);
    else if (live)
      step_live(AllLive<false>{}, sq, full, mw, live);
  };

  if (p1 - p0 <= 2 && p0 < p1) {  // uniform
    // Both query blocks are loaded at once and the two entries run with no
    // barrier between them, so each wave computes only its own live
    // sub-tiles of the two (a causal window gives one wave all four query
    // sub-tiles of one block and one of the other).
    const int ta = tile_of(p0), tb2 = p0 + 1 < p1 ? tile_of(p0 + 1) : 0;
    const int fa = a.blk[ent(p0)], fb = p0 + 1 < p1 ? a.blk[ent(p0 + 1)] : 0;
    QgRegs<P> xa, xb;
    qg_load<P>(xa, Qr, Gr, (uint32_t)(64 * ta) * tb, tid, tb);
    qg_load<P>(xb, Qr, Gr, p0 + 1 < p1 ? (uint32_t)(64 * tb2) * tb : kOob, tid, tb);
    const uint2 sa = bload8(Sr, st_off(p0));
    const uint2 sb = bload8(Sr, st_off(p0 + 1));
    const uint64_t ma = a.kmask[(int64_t)ent(p0) * 64 + kl_];
    const uint64_t mb = p0 + 1 < p1 ? a.kmask[(int64_t)ent(p0 + 1) * 64 + kl_] : 0;
    qg_store<P>(xa, ring, tid);
    bwd_stage_stats(ring + PL::kBytes, sa, tid);
    if (p0 + 1 < p1) {
      qg_store<P>(xb, ring + kBuf, tid);
      bwd_stage_stats(ring + kBuf + PL::kBytes, sb, tid);
    }
    __syncthreads();
    step(ring, (fa & kTileFull) != 0, ma);
    if (p0 + 1 < p1) step(ring + kBuf, (fb & kTileFull) != 0, mb);
  } else if (p0 < p1) {  // uniform
    // Plan words are read once each and a step ahead of use, so that no
    // step's block loads wait on a chain of plan lookups: entry p+3 is read at
    // step p, its tile and flags word at step p+1, and the block loads of
    // step p+2 use them.  Words are kept as read and clamped at their use, so
    // that no load is waited on in the step that issues it.  (e*, t*, f*:
    // entry, query tile, flags word of entries p+1, p+2.)
    auto ce = [&](int e) { return clampi(e, 0, a.nent - 1); };
    auto ct = [&](int t) { return clampi(t, 0, a.ntiles - 1); };
    int e1 = p0 + 1 < p1 ? a.kentry[p0 + 1] : 0;
    int e2 = p0 + 2 < p1 ? a.kentry[p0 + 2] : 0;
    int f0 = a.blk[ent(p0)];
    int t1 = p0 + 1 < p1 ? a.etile[ce(e1)] : 0, f1 = p0 + 1 < p1 ? a.blk[ce(e1)] : 0;
    QgRegs<P> xq;
    qg_load<P>(xq, Qr, Gr, q_off(p0), tid, tb);
    uint2 xs = bload8(Sr, st_off(p0));
    uint64_t mw_next = a.kmask[(int64_t)ent(p0) * 64 + kl_];
    qg_store<P>(xq, ring, tid);
    bwd_stage_stats(ring + PL::kBytes, xs, tid);
    __syncthreads();
    for (int p = p0; p < p1; ++p) {
      const bool full = (f0 & kTileFull) != 0;
      const uint64_t mw = mw_next;
      const bool more = p + 1 < p1;
      qg_load<P>(xq, Qr, Gr, more ? (uint32_t)(64 * ct(t1)) * tb : kOob, tid, tb);
      xs = bload8(Sr, more && tid < 64 ? (uint32_t)(64 * ct(t1) + tid) * sstride : kOob);
      if (more) mw_next = a.kmask[(int64_t)ce(e1) * 64 + kl_];
      const int e3 = p + 3 < p1 ? a.kentry[p + 3] : 0;
      const int t2 = p + 2 < p1 ? a.etile[ce(e2)] : 0, f2 = p + 2 < p1 ? a.blk[ce(e2)] : 0;
      step(ring + ((p - p0) & 1) * kBuf, full, mw);
      if (more) {
        uint8_t* nx = ring + ((p + 1 - p0) & 1) * kBuf;
        qg_store<P>(xq, nx, tid);
        bwd_stage_stats(nx + PL::kBytes, xs, tid);
      }
      __syncthreads();
      f0 = f1;
      e1 = e2;
      t1 = t2;
      f1 = f2;
      e2 = e3;
    }
  }
  if (slot < 0) {
    const __amdgpu_buffer_rsrc_t DKr = make_rsrc(static_cast<Elt*>(a.dk) + x.base, x.nrec);
    const __amdgpu_buffer_rsrc_t DVr = make_rsrc(static_cast<Elt*>(a.dv) + x.base, x.nrec);
    P::store_o(acc_v, 1.0f, DVr, krow, g);
    P::store_o(acc_k, a.scale, DKr, krow, g);
  } else {
    float* dst = a.part + (((int64_t)x.bh * a.npart + slot) * 64 + kl_) * 128;
    P::store_acc(acc_k, dst, g);
    P::store_acc(acc_v, dst + 64, g);
  }
}

// Sum of a split tile's (or key block's) partial rows into the output(s).
// Workgroup (split tile, 16-row quarter); thread (row tid/16, column tid%16)
// owns head_dim 4*column .. +3 of one row and loops over the partials with
// unrolled, independent loads.  WIDTH 64: dQ (scaled); WIDTH 128: dK (scaled)
// then dV.
template <typename Elt, int WIDTH>
__global__ __launch_bounds__(256) void tile_sum_kernel(TileArgs a) {
  constexpr int kQuarters = 64 / kMergeRows;
  const int rq = blockIdx.x % kQuarters;
  const int s = (blockIdx.x / kQuarters) % a.nsplit;
  const int bh = blockIdx.x / kQuarters / a.nsplit;
  const int h = bh % a.H, b = bh / a.H;
  const int t = clampi(a.split[4 * s], 0, a.ntiles - 1);
  const int first = clampi(a.split[4 * s + 1], 0, a.npart);
  const int cnt = clampi(a.split[4 * s + 2], 0, a.npart - first);
  const int row = kMergeRows * rq + (threadIdx.x >> 4), col = threadIdx.x & 15;
  const int64_t i = 64 * (int64_t)t + row;
  if (i >= a.N) return;
  const float* p0 = a.part + (((int64_t)bh * a.npart + first) * 64 + row) * WIDTH + 4 * col;
  constexpr int64_t kStride = 64 * WIDTH;
  const int64_t off = (((int64_t)b * a.N + i) * a.H + h) * kHeadDim + 4 * col;
#pragma unroll
  for (int part = 0; part < WIDTH / 64; ++part) {
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 8
    for (int k = 0; k < cnt; ++k) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p0 + k * kStride + 64 * part);
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] += v[j];
    }
    const float sc = part == 0 ? a.scale : 1.0f;  // dQ and dK carry the softmax scale, dV not
    Elt* dst = static_cast<Elt*>(part == 0 ? (WIDTH == 64 ? a.o : a.dk) : a.dv) + off;
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j] = static_cast<Elt>(o[j] * sc);
  }
}

}  // namespace ma_dev
