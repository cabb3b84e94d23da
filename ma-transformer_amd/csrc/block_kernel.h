// block_kernel.h -- block-sparse attention forward (block size 64, head_dim
// 64, bf16/fp16) on MFMA.
//
// One workgroup (4 waves) per (batch, head, query block r): its 64 queries
// attend the key blocks listed in row r of the block table (ascending, -1
// padded), each a dense 64x64 block product.  Key blocks pass through a
// two-slot LDS ring (K row major, V transposed, the 16-bit stream layout):
// block e+1 is in flight into registers while block e computes, and is
// written into the other slot once block e is done.  Softmax is online
// across blocks, in registers; one O store per row.  Loads and stores go
// through range-checked buffer resources over the (batch, head) stream, so
// a ragged last block reads zero rows (masked) and its stores are dropped.
#pragma once

#include "stream_kernel.h"

namespace ma_dev {

struct BlockArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  const int32_t* table;  // [ceil(N/64), bpr]
  int32_t N, H, bpr, nbq;
  float scale_log2;
};

template <class P>
__global__ __launch_bounds__(256, P::kMinBlocks) void block_kernel(BlockArgs a) {
  static_assert(P::kRows == 64, "block kernel walks 64-key slots");
  __shared__ __attribute__((aligned(16))) uint8_t ring[2 * P::kSlot];
  using Elt = typename P::Elt;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15;
  const int g = lane >> 4;

  const int r = blockIdx.x % a.nbq;
  const int bh = blockIdx.x / a.nbq;  // b * H + h
  const int h = bh % a.H;
  const int b = bh / a.H;
  const int N = a.N;
  const uint32_t tb = (uint32_t)a.H * kHeadDim * sizeof(Elt);  // bytes between tokens

  const int64_t base = ((int64_t)b * N * a.H + h) * kHeadDim;
  const uint32_t nrec = (uint32_t)((int64_t)(N - 1) * tb + kHeadDim * sizeof(Elt));
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + base, nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + base, nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + base, nrec);
  const __amdgpu_buffer_rsrc_t Or = make_rsrc(static_cast<const Elt*>(a.o) + base, nrec);

  // valid entries of this row (the table is -1 padded at the end)
  const int32_t* row = a.table + (int64_t)r * a.bpr;
  int ne = 0;
  for (int e = 0; e < a.bpr; ++e) ne += row[e] >= 0 ? 1 : 0;

  const uint32_t qrow = (uint32_t)(64 * r + 16 * wv + c) * tb;
  typename P::Q q;
  P::load_q(q, Qr, qrow, g);
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);
  auto blk_off = [&](int e) {
    const int cb = e < ne ? row[min(e, a.bpr - 1)] : -1;
    return cb >= 0 ? (uint32_t)(64 * cb) * tb : kOob;
  };

  typename P::Slot nxt;
  P::load_slot(nxt, Kr, Vr, blk_off(0), tid, tb);
  P::store_slot(nxt, ring, tid);
  __syncthreads();

  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int e = 0; e < ne; ++e) {
    P::load_slot(nxt, Kr, Vr, blk_off(e + 1), tid, tb);
    const uint8_t* slot = ring + (e & 1) * P::kSlot;
    const int key0 = 64 * row[e];
    f32x4 sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      f32x4 z = P::qk(slot + P::k_sub(u) + kl, q);
      if (key0 + 16 * u + 15 >= N) {  // ragged last block: keys past the end
        const int km = key0 + 16 * u + 4 * g;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) z[rr] = km + rr < N ? z[rr] : -INFINITY;
      }
      sc[u] = z;
      mx = fmaxf(mx, fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3])));
    }
    const float m_new = fmaxf(m_run, col_max(mx));
    const float m_use = m_new == -INFINITY ? 0.0f : m_new * a.scale_log2;
    const float corr = __builtin_amdgcn_exp2f(m_run * a.scale_log2 - m_use);  // 0 on the first block
    l_run *= corr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] *= corr;
    m_run = m_new;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float p[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        p[rr] = __builtin_amdgcn_exp2f(fmaf(sc[u][rr], a.scale_log2, -m_use));
        l_run += p[rr];
      }
      P::pv(slot + P::v_sub(u) + vl, p, acc);
    }
    // block e+1 goes into the slot block e-1 used (all waves passed the
    // barrier that ended iteration e-1)
    if (e + 1 < ne) P::store_slot(nxt, ring + ((e + 1) & 1) * P::kSlot, tid);
    __syncthreads();
  }
  const float l_tot = col_sum(l_run);
  P::store_o(acc, l_tot > 0.0f ? __builtin_amdgcn_rcpf(l_tot) : 0.0f, Or, qrow, g);
}

}  // namespace ma_dev
