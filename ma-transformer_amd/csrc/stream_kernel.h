// stream_kernel.h -- the sliding-window forward kernel (head_dim 64, any
// dilation, any left/right >= 0) for bf16, fp16 and fp32.
//
// One workgroup (4 waves) streams a chunk of consecutive 64-query tiles of one
// (batch, head, residue class).  A residue class rho of a dilated window is
// the subsequence i = rho + dil*m; on it the window is the contiguous band
// m-left .. m+right, so every dilation is the same banded problem on strided
// rows.  K/V live in an LDS ring of slots of P::kRows keys; tile t reads slots
// floor((64t-left)/rows) .. floor((64t+63+right)/rows), so moving to tile t+1
// needs exactly 64/rows new slots.  While tile t computes, tile t+1's Q rows
// and tile t+2's new K/V rows are in flight into registers; after the tile,
// tile t+1's rows are written over the slots no later tile reads.  Every
// Q/K/V/O row crosses HBM once, except the ring warm-up at chunk start.
//
// All global traffic uses buffer instructions on a per-workgroup resource
// whose range ends at the residue class's last row: rows past the end read as
// zero and their stores are dropped by the hardware range check, so loads and
// stores are issued unconditionally (exact memory counters, no exec-masked
// branches) and the ragged last tile needs no separate path.
//
// Per wave: 16 queries (one MFMA column each) against the 16-key sub-tiles
// that intersect their windows.  S^T = K Q^T lands as lane (query c, group g)
// holding keys 4g..4g+3 of a sub-tile, which is exactly the B operand layout
// P^T of O^T = V^T P^T, so probabilities never leave registers.  All control
// flow is wave-uniform (scalar).
#pragma once

#include "device_common.h"

namespace ma_dev {

constexpr int kHeadDim = 64;

struct StreamArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t N, H;
  int32_t left, right, dil;
  int32_t tiles;      // query tiles of the longest residue class
  int32_t chunk;      // tiles per workgroup
  int32_t chunks;     // ceil(tiles / chunk)
  int32_t tok_bytes;  // bytes between consecutive rows of a residue class (dil * H * 64 * elt)
  float scale_log2;   // softmax scale * log2(e)
  int32_t num_global;  // Longformer: global tokens 0..G-1 (G <= 16)
  float* partials;     // Longformer: [B*H][chunks][16][kPartial] per-chunk softmax partials of the global rows
  float* lse;          // Longformer, optional: each query row's softmax statistic (store_lse), [B*N*H]
  int32_t pairs;       // 1: chunks 2p and 2p+1 share an XCD (grid a multiple of 16, chunks even)
  const void* dout;    // Longformer delta mode (delta != null): the output gradient dO
  float* delta;        // Longformer delta mode: each row's sum_j P_ij dP_ij (= dO . O) in fp32, [B*N*H]; O not written
};

// One partial of a global query row: unnormalised O (64), running max of the
// log2-scaled scores, the softmax denominator, and (delta mode) the
// unnormalised sum of p dP, padded to 16 bytes.
constexpr int kPartial = kHeadDim + 4;

// A query row's softmax statistic for a backward from saved statistics:
// log2 of its softmax denominator sum_j 2^(s_j * sl2) over the raw scores
// s_j, i.e. m * sl2 + log2(l) for the running max m and the sum l taken
// against it (0 for a row with no key).  One lane group (g == 0) writes it.
__device__ __forceinline__ void store_lse(float* lse, int64_t row, bool valid, float m_raw, float l_tot, float sl2,
                                          int g) {
  if (lse && g == 0 && valid) lse[row] = l_tot > 0.0f ? m_raw * sl2 + __log2f(l_tot) : 0.0f;
}

// ---------------------------------------------------------------- 16-bit path
//
// Q.K^T on 16x16x32 MFMA (K rows row-major in LDS).  P.V on MFMA with the
// V^T operand read from row-major V rows through the LDS transpose read
// (tr_read): interior tiles pair sub-tiles on 16x16x32 MFMA (pv2), edge tiles
// take one sub-tile per 16x16x16 MFMA (pv; pairing there spilled registers at
// the 128-register budget and was measured slower).  O^T tile dt row m is
// head_dim d(dt, m) = 32*(dt>>1) + 8*(m>>2) + 4*(dt&1) + (m&3), so lane
// (query c, group g) ends with O[c][8g..8g+7] in acc[0..1] and
// O[c][32+8g..32+8g+7] in acc[2..3]: two 16 B stores per lane.  For that
// order lane l of a transpose read addresses V row l>>2 at head_dim
// 32*(dt>>1) + 8*(l&3) + 4*(dt&1): v_lane + v_tr(dt).
//
// KROW: bytes per K or V row in LDS (128 + pad).  160 puts the four rows of a
// transpose read's 16-lane group on disjoint LDS banks; 144 keeps the 16-byte
// row reads conflict-free instead.  160 measured faster (A/B on one box:
// dense causal bf16 forward 417 -> 388 us, backward 1783 -> 1645 us, cfg3
// backward from saved statistics 130 -> 125 us, the fused backward 0.2-0.9 %).
template <typename T, int KROW = 160>
struct HalfPath {
  using Elt = T;
  static constexpr int kRows = 64;                 // keys per ring slot
  static constexpr int kKRow = KROW;               // bytes per K or V row in LDS
  static constexpr int kSlotK = kRows * kKRow;     // 10240 at 160 B rows
  static constexpr int kSlot = 2 * kSlotK;         // K rows, then V rows
  static constexpr int kMinBlocks = 4;             // launch bound (workgroups per CU)
  static constexpr bool kTrRows = true;            // transposed operands read from rows (tr_read)
  struct Q {
    uint4 r[2];  // query c, head_dim 8g..8g+7 and 32+8g..32+8g+7
  };
  struct Slot {
    uint4 r[4];  // K then V rows tid>>3 and (tid>>3)+32 at 16-byte column tid&7
  };

  static __device__ __forceinline__ void load_q(Q& q, __amdgpu_buffer_rsrc_t Qr, uint32_t row, int g) {
    q.r[0] = bload16(Qr, row + 16 * g);
    q.r[1] = bload16(Qr, row + 16 * g + 64);
  }

  static __device__ __forceinline__ void load_slot(Slot& s, __amdgpu_buffer_rsrc_t Kr, __amdgpu_buffer_rsrc_t Vr,
                                                   uint32_t row_off, int tid, uint32_t tb) {
    const uint32_t k = row_off + (tid >> 3) * tb + (tid & 7) * 16;
    s.r[0] = bload16(Kr, k);
    s.r[1] = bload16(Kr, k + 32 * tb);
    s.r[2] = bload16(Vr, k);
    s.r[3] = bload16(Vr, k + 32 * tb);
  }

  static __device__ __forceinline__ void store_slot(const Slot& s, uint8_t* slot, int tid) {
    uint8_t* p = slot + (tid >> 3) * kKRow + 16 * (tid & 7);
    *reinterpret_cast<uint4*>(p) = s.r[0];
    *reinterpret_cast<uint4*>(p + 32 * kKRow) = s.r[1];
    *reinterpret_cast<uint4*>(p + kSlotK) = s.r[2];
    *reinterpret_cast<uint4*>(p + kSlotK + 32 * kKRow) = s.r[3];
  }

  // First matrix only (a slot whose second part is never read).
  struct Rows {
    uint4 r[2];  // rows tid>>3 and (tid>>3)+32 at column tid&7
  };
  static __device__ __forceinline__ void load_rows(Rows& s, __amdgpu_buffer_rsrc_t Kr, uint32_t row_off, int tid,
                                                   uint32_t tb) {
    const uint32_t k = row_off + (tid >> 3) * tb + (tid & 7) * 16;
    s.r[0] = bload16(Kr, k);
    s.r[1] = bload16(Kr, k + 32 * tb);
  }
  static __device__ __forceinline__ void store_rows(const Rows& s, uint8_t* slot, int tid) {
    const int chk = tid & 7;
    *reinterpret_cast<uint4*>(slot + (tid >> 3) * kKRow + 16 * chk) = s.r[0];
    *reinterpret_cast<uint4*>(slot + ((tid >> 3) + 32) * kKRow + 16 * chk) = s.r[1];
  }

  // Lane byte offsets inside a slot, and of sub-tile u (16 keys) of a slot.
  static __device__ __forceinline__ uint32_t k_lane(int c, int g) { return c * kKRow + 16 * g; }
  static __device__ __forceinline__ uint32_t v_lane(int c, int g) {
    return kSlotK + (4 * g + (c >> 2)) * kKRow + 16 * (c & 3);  // lane 16g + c: row l>>2, piece l&3
  }
  static constexpr uint32_t v_tr(int dt) { return 64 * (dt >> 1) + 8 * (dt & 1); }
  static constexpr uint32_t k_sub(int u) { return u * 16 * kKRow; }
  static constexpr uint32_t v_sub(int u) { return u * 16 * kKRow; }
  // 64-row blocks (the backward's unit) are one slot; sub-tile u (0..3) of a
  // block: rows at blk_k(u), the second matrix's transpose reads at blk_v(u)
  // (from v_lane).
  static constexpr int kSPB = 1;
  static constexpr int kBlk = kSlot;
  static constexpr uint32_t blk_k(int u) { return k_sub(u); }
  static constexpr uint32_t blk_v(int u) { return v_sub(u); }

  // S^T of 16 keys x this wave's 16 queries (raw dot products).
  static __device__ __forceinline__ f32x4 qk(const uint8_t* kp, const Q& q) {
    const uint4 a0 = *reinterpret_cast<const uint4*>(kp);
    const uint4 a1 = *reinterpret_cast<const uint4*>(kp + 64);
    f32x4 z = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    z = Mma<T>::x32(a0, q.r[0], z);
    return Mma<T>::x32(a1, q.r[1], z);
  }

  // O^T += V^T P^T over the 16 keys whose probabilities this lane holds in p.
  static __device__ __forceinline__ void pv(const uint8_t* vp, const float (&p)[4], f32x4 (&acc)[4]) {
    uint2 pb;
    pb.x = Mma<T>::pack2(p[0], p[1]);
    pb.y = Mma<T>::pack2(p[2], p[3]);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] = Mma<T>::x16(tr_read(vp + v_tr(dt)), pb, acc[dt]);
  }

  // The same over two sub-tiles (any two, e.g. from different slots) on one
  // 16x16x32 MFMA per head_dim tile, twice the keys per instruction of the
  // 16x16x16 form.  Contraction element 4h + r of lane group g is key 4g + r
  // of sub-tile h, in both operands: A = the lane's V^T words of the two
  // sub-tiles side by side, B = p0 then p1.
  static __device__ __forceinline__ void pv2(const uint8_t* vp0, const uint8_t* vp1, const float (&p0)[4],
                                             const float (&p1)[4], f32x4 (&acc)[4]) {
    uint4 pb;
    pb.x = Mma<T>::pack2(p0[0], p0[1]);
    pb.y = Mma<T>::pack2(p0[2], p0[3]);
    pb.z = Mma<T>::pack2(p1[0], p1[1]);
    pb.w = Mma<T>::pack2(p1[2], p1[3]);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const uint2 a0 = tr_read(vp0 + v_tr(dt));
      const uint2 a1 = tr_read(vp1 + v_tr(dt));
      acc[dt] = Mma<T>::x32(make_uint4(a0.x, a0.y, a1.x, a1.y), pb, acc[dt]);
    }
  }

  // Unnormalised accumulators of query c as floats into its 64-float row.
  static __device__ __forceinline__ void store_acc(const f32x4 (&acc)[4], float* row, int g) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      *reinterpret_cast<f32x4*>(row + 32 * half + 8 * g) = acc[2 * half];
      *reinterpret_cast<f32x4*>(row + 32 * half + 8 * g + 4) = acc[2 * half + 1];
    }
  }

  static __device__ __forceinline__ void store_o(const f32x4 (&acc)[4], float inv, __amdgpu_buffer_rsrc_t Or,
                                                 uint32_t row, int g) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const f32x4 a0 = acc[2 * half], a1 = acc[2 * half + 1];
      uint4 ov;
      ov.x = Mma<T>::pack2(a0[0] * inv, a0[1] * inv);
      ov.y = Mma<T>::pack2(a0[2] * inv, a0[3] * inv);
      ov.z = Mma<T>::pack2(a1[0] * inv, a1[1] * inv);
      ov.w = Mma<T>::pack2(a1[2] * inv, a1[3] * inv);
      bstore16(Or, row + 16 * g + 64 * half, ov);
    }
  }
};

// ---------------------------------------------------------------- fp32 path
//
// Both contractions on 16x16x4 fp32 MFMA, one contraction element per lane,
// so neither operand needs a transpose.  Q.K^T: lane (c, g) holds head_dim
// chunks g, g+4, g+8, g+12 (4 floats each) of key/query c.  P.V: the A operand
// of MFMA (r, dt) is V[key 4g+r][16dt+c], and V rows are stored in LDS with
// columns permuted to position 4*(d%16) + d/16 so that one 16 B read gives
// dt = 0..3.  O^T tile dt row 4g+rr is O[c][16dt+4g+rr]: four 16 B stores.
// Slots hold 32 keys (17 KB) so that a causal-64 ring is 4 slots = 68 KB.
// (The backward's layout, F32BwdPath below, permutes both matrices.)
struct F32Path {
  using Elt = float;
  static constexpr int kRows = 32;
  static constexpr int kKRow = 272;              // 256 + 16 pad
  static constexpr int kVRow = 272;
  static constexpr int kSlotK = kRows * kKRow;   // 8704
  static constexpr int kSlot = 2 * kSlotK;       // 17408
  static constexpr int kMinBlocks = 2;
  static constexpr bool kTrRows = false;  // no LDS transpose read: transposed operands from permuted rows
  struct Q {
    uint4 r[4];  // query c, head_dim chunk g + 4j (j = 0..3)
  };
  struct Slot {
    uint4 r[4];  // K row tid>>3 chunks tid&7 and (tid&7)+8; V row tid>>3, head_dim 32dp+4cb (+16)
  };

  static __device__ __forceinline__ void load_q(Q& q, __amdgpu_buffer_rsrc_t Qr, uint32_t row, int g) {
#pragma unroll
    for (int j = 0; j < 4; ++j) q.r[j] = bload16(Qr, row + 16 * (g + 4 * j));
  }

  static __device__ __forceinline__ void load_slot(Slot& s, __amdgpu_buffer_rsrc_t Kr, __amdgpu_buffer_rsrc_t Vr,
                                                   uint32_t row_off, int tid, uint32_t tb) {
    const uint32_t row = row_off + (tid >> 3) * tb;
    s.r[0] = bload16(Kr, row + 16 * (tid & 7));
    s.r[1] = bload16(Kr, row + 16 * (tid & 7) + 128);
    const int cb = (tid >> 1) & 3, dp = tid & 1;
    s.r[2] = bload16(Vr, row + 128 * dp + 16 * cb);       // head_dim 32dp + 4cb .. +3
    s.r[3] = bload16(Vr, row + 128 * dp + 64 + 16 * cb);  // head_dim 32dp + 16 + 4cb .. +3
  }

  static __device__ __forceinline__ void store_slot(const Slot& s, uint8_t* slot, int tid) {
    uint8_t* krow = slot + (tid >> 3) * kKRow;
    *reinterpret_cast<uint4*>(krow + 16 * (tid & 7)) = s.r[0];
    *reinterpret_cast<uint4*>(krow + 16 * (tid & 7) + 128) = s.r[1];
    store_perm(s.r[2], s.r[3], slot + kSlotK, tid);
  }

  // Row tid>>3 of a matrix whose head_dim 32dp + 4cb .. +3 (x) and 32dp + 16 +
  // 4cb .. +3 (y) this thread holds (cb = (tid>>1)&3, dp = tid&1), written with
  // columns permuted: head_dim 32dp + 4cb + cc and 32dp + 16 + 4cb + cc sit
  // side by side at position 4(4cb + cc) + 2dp.
  static __device__ __forceinline__ void store_perm(uint4 x, uint4 y, uint8_t* part, int tid) {
    const int cb = (tid >> 1) & 3, dp = tid & 1;
    uint8_t* row = part + (tid >> 3) * kKRow + 8 * dp;
    const uint32_t a[4] = {x.x, x.y, x.z, x.w};
    const uint32_t b[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) *reinterpret_cast<uint2*>(row + 16 * (4 * cb + cc)) = make_uint2(a[cc], b[cc]);
  }

  static __device__ __forceinline__ uint32_t k_lane(int c, int g) { return c * kKRow + 16 * g; }
  static __device__ __forceinline__ uint32_t v_lane(int c, int g) { return kSlotK + 4 * g * kVRow + 16 * c; }
  static constexpr uint32_t k_sub(int u) { return u * 16 * kKRow; }
  static constexpr uint32_t v_sub(int u) { return u * 16 * kVRow; }
  // 64-row blocks are two slots; sub-tile u (0..3) of a block: the first
  // matrix at blk_k(u) (from k_lane), the second at blk_v(u) (from v_lane).
  static constexpr int kSPB = 2;
  static constexpr int kBlk = 2 * kSlot;
  static constexpr uint32_t blk_k(int u) { return (u >> 1) * kSlot + k_sub(u & 1); }
  static constexpr uint32_t blk_v(int u) { return (u >> 1) * kSlot + v_sub(u & 1); }

  // A sub-tile's operands as registers, for a caller that reads the next
  // sub-tile's operands from LDS while this one computes: K rows (QK^T) and
  // permuted V rows (P.V), four 16 B reads each.  (qk / pv below read as they
  // go; issuing all four reads first measured slower in the block kernel.)
  using Ops = f32x4[4];
  static __device__ __forceinline__ void ld_k(const uint8_t* kp, Ops& a) {
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = __builtin_bit_cast(f32x4, *reinterpret_cast<const uint4*>(kp + 64 * j));
  }
  static __device__ __forceinline__ void ld_v(const uint8_t* vp, Ops& va) {
#pragma unroll
    for (int r = 0; r < 4; ++r) va[r] = __builtin_bit_cast(f32x4, *reinterpret_cast<const uint4*>(vp + r * kVRow));
  }
  static __device__ __forceinline__ f32x4 qk_ops(const Ops& a, const Q& q) {
    f32x4 z = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 b = __builtin_bit_cast(f32x4, q.r[j]);
#pragma unroll
      for (int r = 0; r < 4; ++r) z = mfma_f32(a[j][r], b[r], z);
    }
    return z;
  }
  static __device__ __forceinline__ void pv_ops(const Ops& va, const float (&p)[4], f32x4 (&acc)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] = mfma_f32(va[r][dt], p[r], acc[dt]);
  }

  static __device__ __forceinline__ f32x4 qk(const uint8_t* kp, const Q& q) {
    f32x4 z = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 a = __builtin_bit_cast(f32x4, *reinterpret_cast<const uint4*>(kp + 64 * j));
      const f32x4 b = __builtin_bit_cast(f32x4, q.r[j]);
#pragma unroll
      for (int r = 0; r < 4; ++r) z = mfma_f32(a[r], b[r], z);
    }
    return z;
  }

  static __device__ __forceinline__ void pv(const uint8_t* vp, const float (&p)[4], f32x4 (&acc)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const f32x4 va = __builtin_bit_cast(f32x4, *reinterpret_cast<const uint4*>(vp + r * kVRow));
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] = mfma_f32(va[dt], p[r], acc[dt]);
    }
  }

  // fp32 MFMA has no wider contraction: two sub-tiles are two updates.
  static __device__ __forceinline__ void pv2(const uint8_t* vp0, const uint8_t* vp1, const float (&p0)[4],
                                             const float (&p1)[4], f32x4 (&acc)[4]) {
    pv(vp0, p0, acc);
    pv(vp1, p1, acc);
  }

  static __device__ __forceinline__ void store_acc(const f32x4 (&acc)[4], float* row, int g) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) *reinterpret_cast<f32x4*>(row + 16 * dt + 4 * g) = acc[dt];
  }

  static __device__ __forceinline__ void store_o(const f32x4 (&acc)[4], float inv, __amdgpu_buffer_rsrc_t Or,
                                                 uint32_t row, int g) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) bstore16(Or, row + 16 * g + 64 * dt, __builtin_bit_cast(uint4, acc[dt] * inv));
  }
};

// The fp32 layout of the backward passes.  Each of them reads one matrix of a
// block both as a row operand and transposed (K for dQ; Q and dO for dK/dV),
// so both matrices of a slot are stored with permuted columns, once, and the
// row operand is read from the permuted copy too: lane (c, g) reads row c at
// positions 16g + 4e .. +3, i.e. head_dim 16j + 4g + e for j = 0..3, and
// MFMA (e, j) takes element j of that read and element e of the register
// operand's chunk g + 4j (head_dim 16j + 4g .. +3), so lane group g supplies
// head_dim 16j + 4g + e to both.  A block buffer is then one 64-row block
// (35 KB) instead of two, and the backward kernels fit two workgroups per CU.
// The forward keeps F32Path's plain K rows: its ring stores are 16 B wide
// there, and the permuted K rows measured 1.2 % slower on a dilated fp32
// window.
struct F32BwdPath : F32Path {
  struct Slot {
    uint4 r[4];  // first then second matrix, row tid>>3, head_dim 32dp+4cb and 32dp+16+4cb (+0..3)
  };
  static __device__ __forceinline__ void load_slot(Slot& s, __amdgpu_buffer_rsrc_t Kr, __amdgpu_buffer_rsrc_t Vr,
                                                   uint32_t row_off, int tid, uint32_t tb) {
    const uint32_t row = row_off + (tid >> 3) * tb;
    const int cb = (tid >> 1) & 3, dp = tid & 1;
    s.r[0] = bload16(Kr, row + 128 * dp + 16 * cb);
    s.r[1] = bload16(Kr, row + 128 * dp + 64 + 16 * cb);
    s.r[2] = bload16(Vr, row + 128 * dp + 16 * cb);
    s.r[3] = bload16(Vr, row + 128 * dp + 64 + 16 * cb);
  }
  static __device__ __forceinline__ void store_slot(const Slot& s, uint8_t* slot, int tid) {
    store_perm(s.r[0], s.r[1], slot, tid);
    store_perm(s.r[2], s.r[3], slot + kSlotK, tid);
  }
  static __device__ __forceinline__ uint32_t k_lane(int c, int g) { return c * kKRow + 64 * g; }
  static __device__ __forceinline__ f32x4 qk(const uint8_t* kp, const Q& q) {
    f32x4 b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = __builtin_bit_cast(f32x4, q.r[j]);
    f32x4 z = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const f32x4 a = __builtin_bit_cast(f32x4, *reinterpret_cast<const uint4*>(kp + 16 * e));
#pragma unroll
      for (int j = 0; j < 4; ++j) z = mfma_f32(a[j], b[j][e], z);
    }
    return z;
  }
};

// ---------------------------------------------------------------- 64-row blocks

// One 64-row block of an operand: P::kSPB slots of P::kRows rows (one for
// the 16-bit path, two for fp32), loaded into registers and written to
// consecutive slots of a block buffer.  Blocks whose offset is out of range
// (kOob) read nothing.
template <class P>
struct BlkSlots {
  typename P::Slot s[P::kSPB];
};
template <class P>
__device__ __forceinline__ void load_blk(BlkSlots<P>& b, __amdgpu_buffer_rsrc_t A, __amdgpu_buffer_rsrc_t B,
                                         uint32_t off, int tid, uint32_t tb) {
#pragma unroll
  for (int i = 0; i < P::kSPB; ++i) P::load_slot(b.s[i], A, B, off + (uint32_t)(i * P::kRows) * tb, tid, tb);
}
template <class P>
__device__ __forceinline__ void store_blk(const BlkSlots<P>& b, uint8_t* buf, int tid) {
#pragma unroll
  for (int i = 0; i < P::kSPB; ++i) P::store_slot(b.s[i], buf + i * P::kSlot, tid);
}

// ---------------------------------------------------------------- tiles

// Ring location of sub-tile s (16 keys): slot s / (rows/16), sub-tile within it.
template <class P, int NSLOT>
__device__ __forceinline__ uint32_t ring_slot_bytes(int s) {
  constexpr int kSubs = P::kRows / 16;
  return (uint32_t)(((s / kSubs) % NSLOT) * P::kSlot);
}

// Longformer delta mode: d + sum_r p[r] dp[r] (probabilities before their
// 16-bit rounding, dP = dO . V in fp32 from exact 16-bit products).
__device__ __forceinline__ float p_dp(const float (&p)[4], const f32x4& dp, float d) {
#pragma unroll
  for (int r = 0; r < 4; ++r) d = fmaf(p[r], dp[r], d);
  return d;
}

// One wave's 16 queries qa..qa+15 (qa wave-uniform) against the ring, any
// window (runtime left/right): scores on MFMA, softmax in registers (online
// across groups of SG sub-tiles), P.V on MFMA, one store per O row.  Used for
// tiles at the sequence edges and for windows without a fixed instantiation.
// Rows >= Nr compute on zero Q rows and their stores fall outside the buffer.
// Both tile forms return the lane's query row's softmax statistic (log2 of its
// denominator in units of the scaled scores), which only the Longformer
// instantiation stores.
template <class P, int NSLOT, int SG, bool LG>
__device__ __forceinline__ float stream_tile(const uint8_t* ring, uint32_t kl, uint32_t vl, const typename P::Q& q,
                                            int qa, int Nr, int L, int R, float sl2, __amdgpu_buffer_rsrc_t Or,
                                            uint32_t orow, int g, int dl, int G, const typename P::Q& gq, bool dm,
                                            float& dlt) {
  constexpr int kSubs = P::kRows / 16;
  int sub_lo = max(floordiv32(qa - L, 16), 0);
  const int sub_hi = min(floordiv32(qa + 15 + R, 16), (Nr - 1) >> 4);
  const uint32_t span = (uint32_t)(L + R);
  float m_run = -INFINITY, l_run = 0.0f, d_run = 0.0f;  // d_run: delta mode, sum of p dP
  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (LG) {
    // Longformer global keys 0..G-1: sub-tile 0 of the slot after the ring
    f32x4 z = P::qk(ring + NSLOT * P::kSlot + kl, q);
#pragma unroll
    for (int r = 0; r < 4; ++r) z[r] = 4 * g + r < G ? z[r] : -INFINITY;
    m_run = col_max(fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3])));
    const float m_use = m_run * sl2;  // finite: G >= 1
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = __builtin_amdgcn_exp2f(fmaf(z[r], sl2, -m_use));
      l_run += p[r];
    }
    if (dm) d_run = p_dp(p, P::qk(ring + NSLOT * P::kSlot + P::kSlotK + kl, gq), d_run);
    P::pv(ring + NSLOT * P::kSlot + vl, p, acc);
  }
  for (int s0 = sub_lo; s0 <= sub_hi; s0 += SG) {
    f32x4 sc[SG];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < SG; ++j) {
      const int s = s0 + j;
      if (s > sub_hi) break;
      f32x4 z = P::qk(ring + ring_slot_bytes<P, NSLOT>(s) + P::k_sub(s % kSubs) + kl, q);
      // key - query offsets of this sub-tile span [16s-qa-15, 16s-qa+15]
      const int rel = 16 * s - qa;
      if (rel - 15 < -L || rel + 15 > R) {
        // element r: key - query + L = dl + rel + r, inside the window iff in [0, L+R]
        const int x = dl + rel;
#pragma unroll
        for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(x + r) <= span ? z[r] : -INFINITY;
      }
      if (16 * s + 15 >= Nr) {
        const int km = 16 * s + 4 * g;
#pragma unroll
        for (int r = 0; r < 4; ++r) z[r] = km + r < Nr ? z[r] : -INFINITY;
      }
      if (LG && 16 * s < G) {  // window keys below G are already counted as global keys
        const int km = 16 * s + 4 * g;
#pragma unroll
        for (int r = 0; r < 4; ++r) z[r] = km + r >= G ? z[r] : -INFINITY;
      }
      sc[j] = z;
      mx = fmaxf(mx, fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3])));
    }
    const float m_new = fmaxf(m_run, col_max(mx));
    // scores are raw dot products; the softmax scale is folded into exp2's argument
    const float m_use = m_new == -INFINITY ? 0.0f : m_new * sl2;
    if (LG || s0 != sub_lo) {  // rescale what earlier groups accumulated
      const float corr = __builtin_amdgcn_exp2f(m_run * sl2 - m_use);
      l_run *= corr;
      d_run *= corr;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) acc[dt] *= corr;
    }
    m_run = m_new;
#pragma unroll
    for (int j = 0; j < SG; ++j) {
      const int s = s0 + j;
      if (s > sub_hi) break;
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = __builtin_amdgcn_exp2f(fmaf(sc[j][r], sl2, -m_use));
        l_run += p[r];
      }
      if (LG && dm)
        d_run = p_dp(p, P::qk(ring + ring_slot_bytes<P, NSLOT>(s) + P::kSlotK + P::v_sub(s % kSubs) + kl, gq),
                     d_run);
      P::pv(ring + ring_slot_bytes<P, NSLOT>(s) + P::v_sub(s % kSubs) + vl, p, acc);
    }
  }
  const float l_tot = col_sum(l_run);
  const float inv = l_tot > 0.0f ? __builtin_amdgcn_rcpf(l_tot) : 0.0f;
  if constexpr (LG) {  // delta mode: sum_j P_ij dP_ij instead of O
    if (dm)
      dlt = l_tot > 0.0f ? col_sum(d_run) / l_tot : 0.0f;
    else
      P::store_o(acc, inv, Or, orow, g);
  } else {
    P::store_o(acc, inv, Or, orow, g);
  }
  return l_tot > 0.0f ? m_run * sl2 + __log2f(l_tot) : 0.0f;
}

// Compile-time geometry of a fixed window [i-L, i+R]: a wave's 16 queries at
// qa = 16*(4t + wv) read sub-tiles s = 4t + wv - CL + j, j < NSUB, whose key -
// query offsets 16*(j-CL) + [-15, 15] are the same for every interior tile.
template <int L, int R, int RS>
struct WinGeom {
  static constexpr int CL = (L + 15) / 16;
  static constexpr int NSUB = (15 + R) / 16 + CL + 1;
  static constexpr int NSLOT = (63 + R) / RS + (L + RS - 1) / RS + 1;
};

// Interior tile of a fixed window: every sub-tile exists and lies before the
// sequence end, so the whole tile is straight-line code: the sub-tile count,
// which sub-tiles need a mask and the ring offsets are compile-time (up to the
// tile's slot rotation), the per-lane mask compares are loop-invariant, and
// the softmax is two-pass.
template <class P, int L, int R, bool LG>
__device__ __forceinline__ float window_tile(const uint8_t* ring, uint32_t kl, uint32_t vl, const typename P::Q& q,
                                            int t, int wv, float sl2, __amdgpu_buffer_rsrc_t Or, uint32_t orow,
                                            int g, int dl, int ng, const typename P::Q& gq, bool dm, float& dlt) {
  using G = WinGeom<L, R, P::kRows>;
  constexpr int kSubs = P::kRows / 16;
  f32x4 sc[G::NSUB];
  uint32_t vaddr[G::NSUB];
  if constexpr (!P::kTrRows && !LG) {
    // fp32: each sub-tile's 16 MFMAs run while the next sub-tile's operands
    // are read from LDS into the other register buffer; the scheduling
    // barriers keep the compiler from sinking those reads to their use.
    uint32_t kaddr[G::NSUB];
#pragma unroll
    for (int j = 0; j < G::NSUB; ++j) {
      const int u = wv + 3 * G::CL + j;
      const uint32_t sb = (uint32_t)((((t - G::CL) * (4 / kSubs) + u / kSubs) % G::NSLOT) * P::kSlot);
      kaddr[j] = sb + P::k_sub(u % kSubs) + kl;
      vaddr[j] = sb + P::v_sub(u % kSubs) + vl;
    }
    typename P::Ops ob[2];
    P::ld_k(ring + kaddr[0], ob[0]);
#pragma unroll
    for (int j = 0; j < G::NSUB; ++j) {
      if (j + 1 < G::NSUB) P::ld_k(ring + kaddr[j + 1], ob[(j + 1) & 1]);
      else P::ld_v(ring + vaddr[0], ob[(j + 1) & 1]);  // the first P.V operand
      __builtin_amdgcn_sched_barrier(0);
      f32x4 z = P::qk_ops(ob[j & 1], q);
      __builtin_amdgcn_sched_barrier(0);
      const int rel = 16 * (j - G::CL);
      if (rel - 15 < -L || rel + 15 > R) {  // resolved at compile time
#pragma unroll
        for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(dl + rel + r) <= (uint32_t)(L + R) ? z[r] : -INFINITY;
      }
      sc[j] = z;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < G::NSUB; ++j) mx = fmaxf(mx, fmaxf(fmaxf(sc[j][0], sc[j][1]), fmaxf(sc[j][2], sc[j][3])));
    const float m_use = col_max(mx) * sl2;  // finite: every query sees its own key
    float l_run = 0.0f;
    f32x4 acc[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int kV0 = G::NSUB & 1;  // buffer holding the first P.V operand
#pragma unroll
    for (int j = 0; j < G::NSUB; ++j) {
      if (j + 1 < G::NSUB) P::ld_v(ring + vaddr[j + 1], ob[(kV0 + j + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = __builtin_amdgcn_exp2f(fmaf(sc[j][r], sl2, -m_use));
        l_run += p[r];
      }
      P::pv_ops(ob[(kV0 + j) & 1], p, acc);
      __builtin_amdgcn_sched_barrier(0);
    }
    const float l_tot = col_sum(l_run);
    P::store_o(acc, __builtin_amdgcn_rcpf(l_tot), Or, orow, g);
    return m_use + __log2f(l_tot);
  }
  f32x4 zg = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float mx = -INFINITY;
  if (LG) {  // Longformer global keys 0..ng-1 (interior tiles: no window key is below ng)
    zg = P::qk(ring + G::NSLOT * P::kSlot + kl, q);
#pragma unroll
    for (int r = 0; r < 4; ++r) zg[r] = 4 * g + r < ng ? zg[r] : -INFINITY;
    mx = fmaxf(fmaxf(zg[0], zg[1]), fmaxf(zg[2], zg[3]));
  }
#pragma unroll
  for (int j = 0; j < G::NSUB; ++j) {
    const int u = wv + 3 * G::CL + j;  // s = 4(t - CL) + u, u >= 0
    const int slot = ((t - G::CL) * (4 / kSubs) + u / kSubs) % G::NSLOT;
    const uint32_t sb = (uint32_t)(slot * P::kSlot);
    vaddr[j] = sb + P::v_sub(u % kSubs) + vl;
    f32x4 z = P::qk(ring + sb + P::k_sub(u % kSubs) + kl, q);
    const int rel = 16 * (j - G::CL);
    if (rel - 15 < -L || rel + 15 > R) {  // resolved at compile time
#pragma unroll
      for (int r = 0; r < 4; ++r) z[r] = (uint32_t)(dl + rel + r) <= (uint32_t)(L + R) ? z[r] : -INFINITY;
    }
    sc[j] = z;
  }
#pragma unroll
  for (int j = 0; j < G::NSUB; ++j) mx = fmaxf(mx, fmaxf(fmaxf(sc[j][0], sc[j][1]), fmaxf(sc[j][2], sc[j][3])));
  const float m_use = col_max(mx) * sl2;  // finite: every query sees its own key
  float l_run = 0.0f;
  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) acc[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // P.V two sub-tiles per MFMA; the Longformer global sub-tile is element 0
  constexpr int kN = G::NSUB + (LG ? 1 : 0);
  auto score = [&](int j) -> const f32x4& { return LG ? (j == 0 ? zg : sc[j - 1]) : sc[j]; };
  auto vaddr_of = [&](int j) { return LG ? (j == 0 ? (uint32_t)(G::NSLOT * P::kSlot) + vl : vaddr[j - 1]) : vaddr[j]; };
  // delta mode: the V rows of sub-tile j as the row operand (dP = dO V^T)
  auto vrow_of = [&](int j) { return vaddr_of(j) - vl + (uint32_t)P::kSlotK + kl; };
  float d_run = 0.0f;
#pragma unroll
  for (int j = 0; j < kN; j += 2) {
    float p0[4], p1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p0[r] = __builtin_amdgcn_exp2f(fmaf(score(j)[r], sl2, -m_use));
      l_run += p0[r];
    }
    if (LG && dm) d_run = p_dp(p0, P::qk(ring + vrow_of(j), gq), d_run);
    if (j + 1 < kN) {  // resolved at compile time
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p1[r] = __builtin_amdgcn_exp2f(fmaf(score(j + 1)[r], sl2, -m_use));
        l_run += p1[r];
      }
      if (LG && dm) d_run = p_dp(p1, P::qk(ring + vrow_of(j + 1), gq), d_run);
      P::pv2(ring + vaddr_of(j), ring + vaddr_of(j + 1), p0, p1, acc);
    } else {
      P::pv(ring + vaddr_of(j), p0, acc);
    }
  }
  const float l_tot = col_sum(l_run);
  if constexpr (LG) {  // delta mode: sum_j P_ij dP_ij instead of O
    if (dm)
      dlt = col_sum(d_run) / l_tot;  // l_tot > 0: every query sees its own key
    else
      P::store_o(acc, __builtin_amdgcn_rcpf(l_tot), Or, orow, g);
  } else {
    P::store_o(acc, __builtin_amdgcn_rcpf(l_tot), Or, orow, g);
  }
  return m_use + __log2f(l_tot);
}

// ---------------------------------------------------------------- kernel

//
// FL/FR >= 0: specialised for window [i-FL, i+FR] (interior tiles take
// window_tile); FL < 0: any window, every tile takes stream_tile.
//
// LG: Longformer (dilation 1): every query also attends the global keys
// 0..G-1 (G <= 16, held in the slot after the ring, window keys below G
// masked so no key counts twice), and each wave folds one 16-key sub-tile of
// every tile into an online softmax for the global query rows 0..G-1, written
// as one partial per wave for longformer_combine.
//
// DM (with LG, delta mode: the first half of a Longformer backward without
// saved statistics): also reads each tile's dO rows, sums p dP beside the
// softmax (dP = dO V^T on the same MFMA form as the scores) and writes each
// row's delta = sum_j P_ij dP_ij with its statistic instead of O.  Its own
// instantiation, so the plain forward keeps its registers.
template <class P, int NSLOT, int SG, int FL, int FR, bool LG, bool DM>
__global__ __launch_bounds__(256, LG ? 2 : P::kMinBlocks) void stream_kernel(StreamArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t ring[];  // (NSLOT + LG) * P::kSlot bytes
  using Elt = typename P::Elt;
  constexpr bool kFixed = FL >= 0;
  constexpr int FLc = FL < 0 ? 0 : FL, FRc = FR < 0 ? 0 : FR;
  constexpr int RS = P::kRows;    // keys per slot
  constexpr int SPS = 64 / RS;    // slots per 64-row step

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, kept in an SGPR
  const int c = lane & 15;
  const int g = lane >> 4;

  // Workgroup order: chunk fastest.  The dispatcher deals ids to the 8 XCDs
  // round-robin, so every XCD holds every head and chunks spread over the
  // whole sequence.  Orders that give an XCD one head, or one contiguous token
  // range, measured 17-30 % slower on the target (HBM channel locality);
  // hashed orders measured the same as this one.  With `pairs`, chunks 2p and
  // 2p+1 run on one XCD (pairs still dealt round-robin) and walk towards each
  // other's boundary, so the halo block they share is fetched once into that
  // XCD's L2.
  int lin = blockIdx.x;
  if (a.pairs) {  // ids 8i + x (XCD x): pair 8(i/2) + x, member i&1
    const int x = lin & 7, i = lin >> 3;
    lin = 16 * (i >> 1) + 2 * x + (i & 1);
  }
  const int chunk_id = lin % a.chunks;
  lin /= a.chunks;
  const int rho = lin % a.dil;
  lin /= a.dil;
  const int h = lin % (int)a.H;
  const int b = lin / (int)a.H;

  const int Nr = (int)((a.N - rho + a.dil - 1) / a.dil);
  const int tiles_r = (Nr + 63) >> 6;
  const int t0 = chunk_id * a.chunk;
  const int t1 = min(t0 + a.chunk, tiles_r);
  if (t0 >= t1) return;  // uniform per workgroup, before any barrier
  const int nblk = (Nr + RS - 1) / RS;  // ring slots' worth of keys in this residue class
  const int L = kFixed ? FL : a.left;
  const int R = kFixed ? FR : a.right;
  const uint32_t tb = (uint32_t)a.tok_bytes;

  // Buffer resources start at the first row this workgroup reads; their
  // range ends with the residue class's last row.  Offsets below are bytes
  // relative to base_row (the host checks they stay below 2^31).
  const int blo0 = max(floordiv32(t0 * 64 - L, RS), 0);
  const int base_row = LG ? 0 : blo0 * RS;  // Longformer also reads rows 0..G-1
  const int64_t base = (((int64_t)b * a.N + rho) * a.H + h) * kHeadDim + (int64_t)base_row * (tb / sizeof(Elt));
  const int64_t range = (int64_t)(Nr - 1 - base_row) * tb + kHeadDim * sizeof(Elt);
  const uint32_t nrec = (uint32_t)(range < 0x7FFFFFFF ? range : 0x7FFFFFFF);
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const Elt*>(a.q) + base, nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const Elt*>(a.k) + base, nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const Elt*>(a.v) + base, nrec);
  const __amdgpu_buffer_rsrc_t Or = make_rsrc(static_cast<const Elt*>(a.o) + base, nrec);
  // Longformer delta mode: dO rows read where O rows would be written
  constexpr bool dm = LG && DM;
  const __amdgpu_buffer_rsrc_t Gr = make_rsrc(static_cast<const Elt*>(dm ? a.dout : a.o) + base, nrec);

  auto row_off = [&](int row) { return (uint32_t)(row - base_row) * tb; };
  const uint32_t q_lane = (16 * wv + c) * tb;  // this lane's query row within a tile
  const uint32_t kl = P::k_lane(c, g), vl = P::v_lane(c, g);
  const int dl = 4 * g - c + L;  // key - query + L of accumulator element 0
  // Interior tiles: wave 0's first sub-tile 4t - CL >= 0, and wave 3's last
  // sub-tile 4t + 2 - CL + NSUB ends before Nr.
  constexpr int kCL = kFixed ? WinGeom<FLc, FRc, RS>::CL : 0;
  constexpr int kNSUB = kFixed ? WinGeom<FLc, FRc, RS>::NSUB : 0;
  const int t_int_lo = (kCL + (LG ? 4 : 3)) >> 2;  // Longformer: no window sub-tile below key 16
  const int t_int_hi = floordiv32(floordiv32(Nr - 16, 16) + kCL - 2 - kNSUB, 4) + 1;

  // Tile order: with a right halo (R > 0) even chunks ascend and odd chunks
  // descend, so two neighbouring chunks read the K/V blocks on their common
  // boundary at the same moment (both at their first tiles or both at their
  // last) and the second read can be served from cache (cfg2 window: 40.5 ->
  // 38.3 us); causal windows measured faster all ascending (58.5 vs 59.9 us)
  // in the plain order.  With pairs and no right halo the even chunk of a
  // pair descends, so it reads its last block (the odd chunk's halo) first.
  // The ring works either way: a step down needs the 64/rows slots below the
  // current band, and they replace the slots at its top.
  const int dir = R > 0 ? ((chunk_id & 1) ? -1 : 1) : (a.pairs && !(chunk_id & 1) ? -1 : 1);
  const int tfirst = dir > 0 ? t0 : t1 - 1;
  auto blo_of = [&](int t) { return floordiv32(t * 64 - L, RS); };
  auto bhi_of = [&](int t) { return floordiv32(t * 64 + 63 + R, RS); };
  // first of the 64/rows slots tile t adds when reached from t - dir
  auto new_of = [&](int t) { return dir > 0 ? bhi_of(t) - SPS + 1 : blo_of(t); };
  auto tile_ok = [&](int t) { return t >= t0 && t < t1; };

  // ---- prologue: Q rows of the first tile, the slots it reads, and the
  // second tile's new rows
  typename P::Q qc;
  P::load_q(qc, Qr, row_off(tfirst * 64) + q_lane, g);
  typename P::Q gc{};  // delta mode: the tile's dO rows
  if (LG && dm) P::load_q(gc, Gr, row_off(tfirst * 64) + q_lane, g);
  const int blo_f = max(blo_of(tfirst), 0);
  const int top_f = min(bhi_of(tfirst), nblk - 1);
  typename P::Slot X[SPS], Y[SPS];
  {
    typename P::Slot pre[NSLOT];
#pragma unroll
    for (int s = 0; s < NSLOT; ++s)
      P::load_slot(pre[s], Kr, Vr, blo_f + s <= top_f ? row_off((blo_f + s) * RS) : kOob, tid, tb);
#pragma unroll
    for (int i = 0; i < SPS; ++i) {
      const int blk = new_of(tfirst + dir) + i;
      P::load_slot(X[i], Kr, Vr, tile_ok(tfirst + dir) && blk >= 0 && blk < nblk ? row_off(blk * RS) : kOob, tid,
                   tb);
    }
#pragma unroll
    for (int s = 0; s < NSLOT; ++s)
      if (blo_f + s <= top_f) P::store_slot(pre[s], ring + ((blo_f + s) % NSLOT) * P::kSlot, tid);
  }
  typename P::Q qg, gqg{};  // Longformer: Q (and, delta mode, dO) rows of the global queries (query c of every wave)
  if (LG) {
    typename P::Slot gs;
    P::load_slot(gs, Kr, Vr, row_off(0), tid, tb);
    P::store_slot(gs, ring + NSLOT * P::kSlot, tid);
    P::load_q(qg, Qr, row_off(0) + c * tb, g);
    if (dm) P::load_q(gqg, Gr, row_off(0) + c * tb, g);
  }
  __syncthreads();
  const int G = LG ? a.num_global : 0;
  float mg = -INFINITY, lg = 0.0f, dg = 0.0f;  // Longformer global rows: this wave's softmax partial
  f32x4 accg[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) accg[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // One pipeline step: tile t computes while the next tile's Q rows and the
  // tile after's new K/V rows (into `nxt`) are in flight; the next tile's
  // rows (`cur`, loaded one step earlier) then replace the ring slots tile t
  // was the last to read.
  auto step = [&](int t, typename P::Slot(&cur)[SPS], typename P::Slot(&nxt)[SPS]) {
    const int tn = t + dir, tnn = t + 2 * dir;
    typename P::Q qn, gn{};
    P::load_q(qn, Qr, (tile_ok(tn) ? row_off(tn * 64) : kOob) + q_lane, g);
    if (LG && dm) P::load_q(gn, Gr, (tile_ok(tn) ? row_off(tn * 64) : kOob) + q_lane, g);
#pragma unroll
    for (int i = 0; i < SPS; ++i) {
      const int blk = new_of(tnn) + i;
      P::load_slot(nxt[i], Kr, Vr, tile_ok(tnn) && blk >= 0 && blk < nblk ? row_off(blk * RS) : kOob, tid, tb);
    }

    const uint32_t orow = row_off(t * 64) + q_lane;
    float lse2, dlt = 0.0f;
    if (kFixed && t >= t_int_lo && t < t_int_hi)
      lse2 = window_tile<P, FLc, FRc, LG>(ring, kl, vl, qc, t, wv, a.scale_log2, Or, orow, g, dl, G, gc, dm, dlt);
    else
      lse2 = stream_tile<P, NSLOT, SG, LG>(ring, kl, vl, qc, t * 64 + 16 * wv, Nr, L, R, a.scale_log2, Or, orow,
                                           g, dl, G, gc, dm, dlt);
    if constexpr (LG) {  // dilation 1: query m is token m (rows 0..G-1 are rewritten by the combine)
      const int m = t * 64 + 16 * wv + c;
      const int64_t row = ((int64_t)b * a.N + m) * a.H + h;
      if (a.lse && g == 0 && m < Nr) a.lse[row] = lse2;
      if (dm && g == 0 && m < Nr) a.delta[row] = dlt;
    }
    if (LG) {  // global query rows against keys 64t + 16wv .. +15 (in the ring at tile t)
      const int key0 = t * 64 + 16 * wv;
      constexpr int kSubs = RS / 16;
      f32x4 z = P::qk(ring + ring_slot_bytes<P, NSLOT>(key0 / 16) + P::k_sub((key0 / 16) % kSubs) + kl, qg);
      if (key0 + 15 >= Nr) {
#pragma unroll
        for (int r = 0; r < 4; ++r) z[r] = key0 + 4 * g + r < Nr ? z[r] : -INFINITY;
      }
      const float m_new = fmaxf(mg, col_max(fmaxf(fmaxf(z[0], z[1]), fmaxf(z[2], z[3]))));
      const float m_use = m_new == -INFINITY ? 0.0f : m_new * a.scale_log2;
      const float corr = __builtin_amdgcn_exp2f(mg * a.scale_log2 - m_use);
      lg *= corr;
      dg *= corr;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) accg[dt] *= corr;
      mg = m_new;
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = __builtin_amdgcn_exp2f(fmaf(z[r], a.scale_log2, -m_use));
        lg += p[r];
      }
      const uint32_t vsub = ring_slot_bytes<P, NSLOT>(key0 / 16) + P::v_sub((key0 / 16) % kSubs);
      if (dm) dg = p_dp(p, P::qk(ring + vsub + P::kSlotK + kl, gqg), dg);
      P::pv(ring + vsub + vl, p, accg);
    }

    __syncthreads();
#pragma unroll
    for (int i = 0; i < SPS; ++i) {
      const int blk = new_of(tn) + i;
      if (tile_ok(tn) && blk >= 0 && blk < nblk) P::store_slot(cur[i], ring + (blk % NSLOT) * P::kSlot, tid);
    }
    __syncthreads();
    qc = qn;
    gc = gn;
  };

  const int cnt = t1 - t0;
  for (int n = 0; n < cnt; n += 2) {
    step(tfirst + n * dir, X, Y);
    if (n + 1 >= cnt) break;
    step(tfirst + (n + 1) * dir, Y, X);
  }

  if (LG) {
    // Each wave's partial for global query c ([64 unnormalised O][log2-scaled
    // max][denominator][delta mode: sum of p dP]) goes to LDS (the ring is
    // free after the last tile's barrier; rows of 68 floats keep the 16 B
    // stores aligned); the 4 waves' partials of a query then merge
    // (log-sum-exp) into one per chunk, so the combine reads a quarter as many.
    constexpr int kRowF = 68;
    const float l_tot = col_sum(lg);
    const float d_tot = dm ? col_sum(dg) : 0.0f;
    float* shp = reinterpret_cast<float*>(ring) + (wv * 16 + c) * kRowF;
    P::store_acc(accg, shp, g);
    if (g == 0) {
      shp[kHeadDim] = mg == -INFINITY ? -INFINITY : mg * a.scale_log2;
      shp[kHeadDim + 1] = l_tot;
      shp[kHeadDim + 2] = d_tot;
    }
    __syncthreads();
    const int qq = tid >> 4, d0 = 4 * (tid & 15);  // global query qq, head_dim d0..d0+3
    const float* sp = reinterpret_cast<const float*>(ring) + qq * kRowF;
    float mw[4], mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = sp[w * 16 * kRowF + kHeadDim];
      mt = fmaxf(mt, mw[w]);
    }
    float lt = 0.0f, dtt = 0.0f;
    f32x4 at = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    if (mt != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float cw = __builtin_amdgcn_exp2f(mw[w] - mt);  // 0 for a wave that saw no key
        lt = fmaf(sp[w * 16 * kRowF + kHeadDim + 1], cw, lt);
        dtt = fmaf(sp[w * 16 * kRowF + kHeadDim + 2], cw, dtt);
        at += *reinterpret_cast<const f32x4*>(sp + w * 16 * kRowF + d0) * cw;
      }
    }
    float* dst = a.partials + ((((int64_t)b * a.H + h) * a.chunks + chunk_id) * 16 + qq) * kPartial;
    *reinterpret_cast<f32x4*>(dst + d0) = at;  // rows of 68 floats: 16 B aligned
    if ((tid & 15) == 0) *reinterpret_cast<f32x4*>(dst + kHeadDim) = f32x4{mt, lt, dtt, 0.0f};
  }
}

// Global query rows of Longformer: merge the per-wave partials of every chunk
// (log-sum-exp combine) into O rows 0..G-1.  One workgroup of 4 waves per
// (batch, head, global row), over one partial per chunk; thread (wave w,
// lane d) owns head_dim element d of the partials p = w, w+4, ...  A wave
// loads 8 of its partials (maximum, denominator, element d) at once, then
// merges them, so a row of up to 32 partials costs one load round trip; the 4
// wave results merge in LDS.  (A single wave folding the partials one by one
// waited out one round trip per partial: 42 us at cfg 4; a maximum pass
// before the weighted sums, two round trips: 5.2 us.)
template <typename Elt>
__global__ __launch_bounds__(256) void longformer_combine(const float* __restrict__ partials, Elt* __restrict__ o,
                                                          int nparts, int G, int H, int64_t N, float* lse,
                                                          float* delta) {
  __shared__ float sh[4][kPartial];
  const int d = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int gq = blockIdx.x % G;
  const int bh = blockIdx.x / G;  // b * H + h
  const int h = bh % H;
  const int b = bh / H;
  // partial p of this global row: base + p * 16 * kPartial
  const float* base = partials + ((int64_t)bh * nparts * 16 + gq) * kPartial;
  constexpr int64_t kStride = 16 * kPartial;
  // Batches of 8 partials per wave, all loads of a batch issued together:
  // one load round trip per 32 partials of the row.  Delta mode also merges
  // the partials' sums of p dP, with the denominators' weights.
  const bool dm = delta != nullptr;
  float m = -INFINITY, l = 0.0f, acc = 0.0f, dsum = 0.0f;
  for (int p0 = wv; p0 < nparts; p0 += 32) {
    float mk[8], lk[8], ak[8], dk[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int p = p0 + 4 * k;
      const float* src = base + (int64_t)min(p, nparts - 1) * kStride;
      mk[k] = src[kHeadDim];
      lk[k] = src[kHeadDim + 1];
      dk[k] = dm ? src[kHeadDim + 2] : 0.0f;
      ak[k] = src[d];
      if (p >= nparts) mk[k] = -INFINITY;
    }
    float mb = m;
#pragma unroll
    for (int k = 0; k < 8; ++k) mb = fmaxf(mb, mk[k]);
    if (mb != -INFINITY) {
      const float c = __builtin_amdgcn_exp2f(m - mb);  // 0 while m is -inf
      l *= c;
      acc *= c;
      dsum *= c;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float w = __builtin_amdgcn_exp2f(mk[k] - mb);  // 0 for a partial that saw no key
        l = fmaf(lk[k], w, l);
        acc = fmaf(ak[k], w, acc);
        dsum = fmaf(dk[k], w, dsum);
      }
      m = mb;
    }
  }
  sh[wv][d] = acc;
  if (d == 0) {
    sh[wv][kHeadDim] = m;
    sh[wv][kHeadDim + 1] = l;
    sh[wv][kHeadDim + 2] = dsum;
  }
  __syncthreads();
  if (wv == 0) {
    float mt = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mt = fmaxf(mt, sh[w][kHeadDim]);
    float lt = 0.0f, at = 0.0f, dt = 0.0f;
    if (mt != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float c = __builtin_amdgcn_exp2f(sh[w][kHeadDim] - mt);
        lt = fmaf(sh[w][kHeadDim + 1], c, lt);
        at = fmaf(sh[w][d], c, at);
        dt = fmaf(sh[w][kHeadDim + 2], c, dt);
      }
    }
    const int64_t row = ((int64_t)b * N + gq) * H + h;
    if (dm) {  // delta mode: the row's sum_j P_ij dP_ij; O not written
      if (d == 0) delta[row] = lt > 0.0f ? dt / lt : 0.0f;
    } else {
      o[row * kHeadDim + d] = static_cast<Elt>(lt > 0.0f ? at / lt : 0.0f);
    }
    // the global row's statistic (mt is in log2 units of the scaled scores)
    if (lse && d == 0) lse[row] = lt > 0.0f ? mt + __log2f(lt) : 0.0f;
  }
}

}  // namespace ma_dev

namespace ma_dev {

// ---------------------------------------------------------------- copy probe
//
// The stream kernel's memory traffic without its arithmetic: the same
// workgroups, chunks and 64-row tiles of one (batch, head, residue class),
// the same halo blocks before (and, with a right window, after) each chunk,
// O = Q xor K xor V bitwise.  It measures what this access pattern can move
// on the device -- the ceiling a bandwidth-bound stream kernel runs against.
// EB: bytes per head row (128 for 16-bit, 256 for fp32).
template <int EB>
__global__ __launch_bounds__(256) void copy_probe_kernel(StreamArgs a) {
  constexpr int CPR = EB / 16;              // 16-byte chunks per row
  constexpr int NU = 64 * CPR / 256;        // uint4 per thread per tile and tensor
  const int tid = threadIdx.x;
  int lin = blockIdx.x;
  if (a.pairs) {
    const int x = lin & 7, i = lin >> 3;
    lin = 16 * (i >> 1) + 2 * x + (i & 1);
  }
  const int chunk_id = lin % a.chunks;
  lin /= a.chunks;
  const int rho = lin % a.dil;
  lin /= a.dil;
  const int h = lin % (int)a.H;
  const int b = lin / (int)a.H;
  const int Nr = (int)((a.N - rho + a.dil - 1) / a.dil);
  const int tiles_r = (Nr + 63) >> 6;
  const int t0 = chunk_id * a.chunk;
  const int t1 = min(t0 + a.chunk, tiles_r);
  if (t0 >= t1) return;
  const uint32_t tb = (uint32_t)a.tok_bytes;
  const int nblk = (Nr + 63) >> 6;
  const int hlo = max(floordiv32(t0 * 64 - a.left, 64), 0);               // first halo block before the chunk
  const int hhi = min(floordiv32((t1 - 1) * 64 + 63 + a.right, 64), nblk - 1);  // last block after it
  const int base_row = hlo * 64;
  const int64_t base = (((int64_t)b * a.N + rho) * a.H + h) * EB + (int64_t)base_row * tb;  // bytes
  const int64_t range = (int64_t)(Nr - 1 - base_row) * tb + EB;
  const uint32_t nrec = (uint32_t)(range < 0x7FFFFFFF ? range : 0x7FFFFFFF);
  const __amdgpu_buffer_rsrc_t Qr = make_rsrc(static_cast<const uint8_t*>(a.q) + base, nrec);
  const __amdgpu_buffer_rsrc_t Kr = make_rsrc(static_cast<const uint8_t*>(a.k) + base, nrec);
  const __amdgpu_buffer_rsrc_t Vr = make_rsrc(static_cast<const uint8_t*>(a.v) + base, nrec);
  const __amdgpu_buffer_rsrc_t Or = make_rsrc(static_cast<uint8_t*>(a.o) + base, nrec);
  auto off = [&](int blk, int j) {
    const int e = tid + 256 * j;
    return (uint32_t)(blk * 64 + e / CPR - base_row) * tb + (uint32_t)(e % CPR) * 16;
  };
  // halo blocks: K and V rows the window reads outside the chunk's own tiles
  uint4 hx = make_uint4(0u, 0u, 0u, 0u);
  for (int blk = hlo; blk <= hhi; ++blk) {
    if (blk >= t0 && blk < t1) continue;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      const uint4 x = bload16(Kr, off(blk, j)), y = bload16(Vr, off(blk, j));
      hx.x ^= x.x ^ y.x;
      hx.y ^= x.y ^ y.y;
    }
  }
  uint4 x[3][NU];
#pragma unroll
  for (int j = 0; j < NU; ++j) {
    x[0][j] = bload16(Qr, off(t0, j));
    x[1][j] = bload16(Kr, off(t0, j));
    x[2][j] = bload16(Vr, off(t0, j));
  }
  for (int t = t0; t < t1; ++t) {
    uint4 y[NU];
#pragma unroll
    for (int j = 0; j < NU; ++j)
      y[j] = make_uint4(x[0][j].x ^ x[1][j].x ^ x[2][j].x ^ hx.x, x[0][j].y ^ x[1][j].y ^ x[2][j].y ^ hx.y,
                        x[0][j].z ^ x[1][j].z ^ x[2][j].z, x[0][j].w ^ x[1][j].w ^ x[2][j].w);
    const uint32_t nx = t + 1 < t1 ? 0u : kOob;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
      x[0][j] = bload16(Qr, nx + off(t + 1, j));
      x[1][j] = bload16(Kr, nx + off(t + 1, j));
      x[2][j] = bload16(Vr, nx + off(t + 1, j));
    }
#pragma unroll
    for (int j = 0; j < NU; ++j) bstore16(Or, off(t, j), y[j]);
  }
}

}  // namespace ma_dev
