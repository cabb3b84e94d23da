// block_kernel.h -- block-sparse attention forward (block size 64, head_dim
// 64, bf16/fp16 on 16x16x32 MFMA, fp32 on 16x16x4 MFMA with 64-row blocks of
// two 32-row fp32 slots).
//
// Query block r attends the key blocks listed in row r of the block table
// (ascending, -1 padded), each a dense 64x64 block product on MFMA.  One
// workgroup (4 waves, 16 queries each) per (batch, head, query block).  Key
// blocks pass through a two-slot LDS ring (K row major, V transposed: the
// 16-bit stream layout): block e+1 is in flight into registers while block e
// computes.  Softmax is online across a row's blocks, in registers; one O
// store per row.  Loads and stores go through range-checked buffer resources
// over the (batch, head) stream, so a ragged last block reads zero rows
// (masked) and its stores are dropped.
//
// Measured alternatives that did not pay on 4-wide tables (diagonal, previous
// and two random blocks): a
// workgroup walking a run of consecutive rows with two blocks in flight
// (the same time at best, slower with more rows per run), because a row's
// time is not its load latency alone; and a row-pipelined walk (all 4
// blocks of a row in LDS, the next row's loads in flight, 2 workgroups per
// CU): 65 against 50 us, since a row's dependent MFMA / softmax chain needs
// the 4 workgroups per CU of this kernel to hide it.
#pragma once

#include "stream_kernel.h"

namespace ma_dev {

struct BlockArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* table;  // [nbq, bpr]; null: every block (dense), or blocks 0..r (causal)
  int32_t N, H, bpr, nbq;
  float scale_log2;
  int32_t causal;  // with a null table: keys [0, i]
  float* lse;      // optional: each query row's softmax statistic (store_lse), [B*N*H]
};

// Workgroup ids go through xcd_row_order: XCD x runs rows [x*G/8,
// (x+1)*G/8) in order, which puts row r and row r+1 (which read block r as
// diagonal and as previous) and a head's random blocks on one L2.

// Online-softmax update of one 64-key block (4 sub-tiles) from an LDS slot.
// cb < 0: an absent entry, every score masked.  diag: the block is the query
// block itself under a causal mask, so key k of the block is kept only up to
// the lane's query ql (0..63 within the block).
template <class P>
__device__ __forceinline__ void block_update(const uint8_t* slot, uint32_t kl, uint32_t vl, const typename P::Q& q,
                                             int cb, bool diag, int ql, int N, int g, float sl2, float& m_run,
                                             float& l_run, f32x4 (&acc)[4]) {
  const int key0 = 64 * cb;
  f32x4 sc[4];
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < 4; ++u) sc[u] = P::qk(slot + P::blk_k(u) + kl, q);
  // One uniform branch after all four products, so they issue back to back.
  if (cb < 0 || diag || key0 + 63 >= N) {  // absent entry, causal diagonal, or keys past the end
    // key 16u + 4g + rr of the block is kept up to hi; the lane term stays
    // alone on the left (a hoisted table of all 16 lane keys would cost
    // 16 registers for the whole kernel)
    const int hi = min(cb < 0 ? -1 : N - key0 - 1, diag ? ql : 63);
    const int lk = 4 * g;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) sc[u][rr] = lk <= hi - 16 * u - rr ? sc[u][rr] : -INFINITY;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) mx = fmaxf(mx, fmaxf(fmaxf(sc[u][0], sc[u][1]), fmaxf(sc[u][2], sc[u][3])));
  const float m_new = fmaxf(m_run, col_max(mx));
  const float m_use = m_new == -INFINITY ? 0.0f : m_new * sl2;
  // Rescale only when some lane's running max rose (wave-uniform test): on
  // long rows the max settles after a few blocks and most blocks skip it.
  if (__builtin_amdgcn_ballot_w64(m_new != m_run) != 0) {
    const float corr = __builtin_amdgcn_exp2f(m_run * sl2 - m_use);  // 0 on a row's first block
    l_run *= corr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] *= corr;
  }
  m_run = m_new;
#pragma unroll
  for (int u = 0; u < 4; u += 2) {
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

// The same update over two blocks at once (the slot pair at `slots`), one
// max and one rescale for their 128 keys: the two blocks' eight QK products
// and then their sixteen P.V products issue back to back, so a row of four
// blocks is two dependent score -> max -> exp -> P.V chains instead of four.
// No causal diagonal here (table rows only).
template <class P>
__device__ __forceinline__ void block_pair_update(const uint8_t* slots, uint32_t kl, uint32_t vl,
                                                  const typename P::Q& q, int cb0, int cb1, int N, int g, float sl2,
                                                  float& m_run, float& l_run, f32x4 (&acc)[4]) {
  const int cb[2] = {cb0, cb1};
  f32x4 sc[2][4];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 4; ++u) sc[b][u] = P::qk(slots + b * P::kSlot + P::blk_k(u) + kl, q);
  const int lk = 4 * g;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    if (cb[b] < 0 || 64 * cb[b] + 63 >= N) {  // uniform: absent entry or keys past the end
      const int hi = cb[b] < 0 ? -1 : N - 64 * cb[b] - 1;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sc[b][u][rr] = lk <= hi - 16 * u - rr ? sc[b][u][rr] : -INFINITY;
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      mx = fmaxf(mx, fmaxf(fmaxf(sc[b][u][0], sc[b][u][1]), fmaxf(sc[b][u][2], sc[b][u][3])));
  const float m_new = fmaxf(m_run, col_max(mx));
  const float m_use = m_new == -INFINITY ? 0.0f : m_new * sl2;
  if (__builtin_amdgcn_ballot_w64(m_new != m_run) != 0) {
    const float corr = __builtin_amdgcn_exp2f(m_run * sl2 - m_use);  // 0 on a row's first pair
    l_run *= corr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] *= corr;
  }
  m_run = m_new;
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int u = 0; u < 4; u += 2) {
      float p0[4], p1[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        p0[rr] = __builtin_amdgcn_exp2f(fmaf(sc[b][u][rr], sl2, -m_use));
        p1[rr] = __builtin_amdgcn_exp2f(fmaf(sc[b][u + 1][rr], sl2, -m_use));
        l_run += p0[rr] + p1[rr];
      }
      const uint8_t* slot = slots + b * P::kSlot;
      P::pv2(slot + P::blk_v(u) + vl, slot + P::blk_v(u + 1) + vl, p0, p1, acc);
    }
}

template <class P>
__global__ __launch_bounds__(256, P::kMinBlocks) void block_row_kernel(BlockArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // 2 block buffers of P::kBlk bytes
  using Elt = typename P::Elt;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  const bool dense = a.table == nullptr;
  const int wg = xcd_row_order(blockIdx.x, gridDim.x);
  // causal rows run longest (last query block) first, so short ones fill the tail
  const int r = dense && a.causal ? a.nbq - 1 - wg % a.nbq : wg % a.nbq;
  const int bh = wg / a.nbq;  // b * H + h
  const int h = bh % a.H;
  const int b = bh / a.H;
  const int N = a.N;
  const uint32_t tb = (uint32_t)a.H * kHeadDim * sizeof(Elt);

  const int64_t base = ((int64_t)b * N * a.H + h) * kHeadDim;
  const uint32_t nrec = (uint32_t)((int64_t)(N - 1) * tb + kHeadDim * sizeof(Elt));
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + base, nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + base, nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + base, nrec);
  const __amdgpu_buffer_rsrc_t Or = make_rsrc(static_cast<const Elt*>(a.o) + base, nrec);

  // valid entries of this row (the table is -1 padded at the end)
  const int32_t* row = dense ? nullptr : a.table + (int64_t)r * a.bpr;
  int ne = dense ? (a.causal ? r + 1 : a.nbq) : 0;
  if (!dense)
    for (int e = 0; e < a.bpr; ++e) ne += row[e] >= 0 ? 1 : 0;
  auto block_of = [&](int e) { return e < ne ? (dense ? e : row[min(e, a.bpr - 1)]) : -1; };

  const uint32_t qrow = (uint32_t)(64 * r + 16 * wv + c) * tb;
  typename P::Q q;
  P::load_q(q, Qr, qrow, g);
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);
  auto blk_off = [&](int e) {
    const int cb = block_of(e);
    return cb >= 0 ? (uint32_t)(64 * cb) * tb : kOob;
  };

  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const float sl2 = a.scale_log2;
  const int ql = 16 * wv + c;

  // 16-bit blocks only: four blocks of registers in flight fit there
  if constexpr (P::kSPB == 1) {
    if (!dense && a.bpr <= 4) {
      // Short rows (diagonal + previous + 2 random blocks: 4 entries): every block's loads are
      // issued at once, so the row pays one HBM latency instead of one per
      // block; the two-slot ring is filled twice.
      typename P::Slot x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) P::load_slot(x[e], Kr, Vr, blk_off(e), tid, tb);
      P::store_slot(x[0], ring, tid);
      P::store_slot(x[1], ring + P::kSlot, tid);
      __syncthreads();
      // an absent second entry of a pair is a masked block (its loads read zeros)
      if (ne > 0) block_pair_update<P>(ring, kl, vl, q, block_of(0), block_of(1), N, g, sl2, m_run, l_run, acc);
      if (ne > 2) {  // uniform
        __syncthreads();
        P::store_slot(x[2], ring, tid);
        P::store_slot(x[3], ring + P::kSlot, tid);
        __syncthreads();
        block_pair_update<P>(ring, kl, vl, q, block_of(2), block_of(3), N, g, sl2, m_run, l_run, acc);
      }
      const float l_tot = col_sum(l_run);
      P::store_o(acc, l_tot > 0.0f ? __builtin_amdgcn_rcpf(l_tot) : 0.0f, Or, qrow, g);
      store_lse(a.lse, ((int64_t)b * N + 64 * r + ql) * a.H + h, 64 * r + ql < N, m_run, l_tot, sl2, g);
      return;
    }
  }

  BlkSlots<P> nxt;
  load_blk<P>(nxt, Kr, Vr, blk_off(0), tid, tb);
  store_blk<P>(nxt, ring, tid);
  __syncthreads();

  for (int e = 0; e < ne; ++e) {
    load_blk<P>(nxt, Kr, Vr, blk_off(e + 1), tid, tb);
    __builtin_amdgcn_sched_barrier(0);
    const int cb = block_of(e);
    block_update<P>(ring + (e & 1) * P::kBlk, kl, vl, q, cb, dense && a.causal && cb == r, 16 * wv + c, N, g,
                    a.scale_log2, m_run, l_run, acc);
    // block e+1 goes into the slot block e-1 used (all waves passed the
    // barrier that ended iteration e-1)
    if (e + 1 < ne) store_blk<P>(nxt, ring + ((e + 1) & 1) * P::kBlk, tid);
    __syncthreads();
  }
  const float l_tot = col_sum(l_run);
  P::store_o(acc, l_tot > 0.0f ? __builtin_amdgcn_rcpf(l_tot) : 0.0f, Or, qrow, g);
  store_lse(a.lse, ((int64_t)b * N + 64 * r + ql) * a.H + h, 64 * r + ql < N, m_run, l_tot, sl2, g);
}

// ---------------------------------------------------------------- copy probe
//
// block_row_kernel's memory traffic without its arithmetic: the same grid and
// workgroup order, each workgroup reading its row's Q tile and the K and V
// blocks its table row lists (every block's loads in flight at once, as the
// kernel issues them for rows of up to 4 entries), and writing
// O[i] = Q[i] xor (xor over the row's entries c of K[64c + i%64] xor
// V[64c + i%64]) bitwise.  Gives the copy speed of that access pattern on the
// device.  EB: bytes per head row (128 for 16-bit, 256 for fp32); table-driven
// rows of at most 4 entries.
template <int EB>
__global__ __launch_bounds__(256) void block_probe_kernel(BlockArgs a) {
  constexpr int CPR = EB / 16;        // 16-byte chunks per row
  constexpr int NU = 64 * CPR / 256;  // uint4 per thread per 64-row tile
  const int tid = threadIdx.x;
  const int wg = xcd_row_order(blockIdx.x, gridDim.x);
  const int r = wg % a.nbq;
  const int bh = wg / a.nbq;
  const int h = bh % a.H;
  const int b = bh / a.H;
  const int N = a.N;
  const uint32_t tb = (uint32_t)a.H * EB;
  const int64_t base = ((int64_t)b * N * a.H + h) * EB;  // bytes
  const uint32_t nrec = (uint32_t)((int64_t)(N - 1) * tb + EB);
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const uint8_t*>(a.q) + base, nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const uint8_t*>(a.k) + base, nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const uint8_t*>(a.v) + base, nrec);
  const __amdgpu_buffer_rsrc_t Or = make_rsrc(static_cast<uint8_t*>(a.o) + base, nrec);
  const int32_t* row = a.table + (int64_t)r * a.bpr;
  auto off = [&](int j) {
    const int e = tid + 256 * j;
    return (uint32_t)(e / CPR) * tb + (uint32_t)(e % CPR) * 16;
  };
  uint4 x[NU];
  const uint32_t qo = (uint32_t)(64 * r) * tb;
#pragma unroll
  for (int j = 0; j < NU; ++j) x[j] = bload16(Qr, qo + off(j));
  uint4 kv[4][2][NU];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int cb = e < a.bpr ? row[e] : -1;
    const uint32_t bo = cb >= 0 ? (uint32_t)(64 * cb) * tb : kOob;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      kv[e][0][j] = bload16(Kr, bo + off(j));
      kv[e][1][j] = bload16(Vr, bo + off(j));
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int j = 0; j < NU; ++j)
      x[j] = make_uint4(x[j].x ^ kv[e][0][j].x ^ kv[e][1][j].x, x[j].y ^ kv[e][0][j].y ^ kv[e][1][j].y,
                        x[j].z ^ kv[e][0][j].z ^ kv[e][1][j].z, x[j].w ^ kv[e][0][j].w ^ kv[e][1][j].w);
#pragma unroll
  for (int j = 0; j < NU; ++j) bstore16(Or, qo + off(j), x[j]);
}

}  // namespace ma_dev
