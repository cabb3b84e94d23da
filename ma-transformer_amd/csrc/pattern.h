// pattern.h -- closed-form key sets S_i of the sparse-attention patterns.
//
// Shared by the host index enumerator (ma_attn_row_keys) and the device
// kernels, so host and GPU agree on every index by construction.  Each row's
// key set is ascending and is described by a short list of segments; the
// t-th key of the row is found by walking them.
//
//   SLIDING      {i + dil*t : -left <= t <= right} n [0,N)
//                reference window w (src/csrc/ma_core.cpp:197-198,
//                src/cuda/sparse_attention_kernel.cu:232-233) is left=right=w,
//                dil=1; dilation per doc/sparse_attention_whitepaper.md:98-104
//   DENSE        [0,N) or [0,i] (ma_core.cpp:66-157; the causal -1e9 fill of
//                :114-120 contributes exactly zero weight)
//   BLOCK_SPARSE union of [c*bs, min((c+1)*bs, N)) over the row block's table
//                entries c >= 0 (ascending), cf. sparse_attention.cpp:203-231
//   LONGFORMER   i < G: [0,N); else [0,G) U [max(i-left,G), min(i+right,N-1)]
//                (sparse_attention.cpp:234-259 without its duplicate entries)
//   INDEX_SET    keys[offsets[i] .. offsets[i+1]) (CSR, one pattern for all
//                (batch, head), as the generic COO attention of
//                sparse_attention.cpp:11-152); the row range is clamped into
//                [0, nnz], so any offsets array reads inside the key array
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MA_HD __host__ __device__ inline
#else
#define MA_HD inline
#endif

namespace ma {

enum Pattern : int32_t { kSliding = 0, kDense = 1, kBlockSparse = 2, kLongformer = 3, kIndexSet = 4 };

struct PatternParams {
  int64_t n;         // sequence length
  int32_t pattern;
  int32_t causal;
  int64_t left, right, dilation;
  int64_t block_size;
  const int32_t* table;  // host or device pointer, matching the caller
  int64_t bpr;           // table width
  int64_t num_global;
  const int64_t* offsets;  // INDEX_SET: [n + 1] row offsets into keys
  const int32_t* keys;     // INDEX_SET: [nnz] key positions
  int64_t nnz;
};

MA_HD int64_t imin64(int64_t a, int64_t b) { return a < b ? a : b; }
MA_HD int64_t imax64(int64_t a, int64_t b) { return a > b ? a : b; }

// floor(a / d) for d > 0 and any sign of a
MA_HD int64_t floordiv64(int64_t a, int64_t d) {
  int64_t q = a / d;
  return (a % d != 0 && a < 0) ? q - 1 : q;
}

// A row's key set as up to two arithmetic segments (SLIDING, DENSE,
// LONGFORMER), a table walk (BLOCK_SPARSE) or a slice of the key array
// (INDEX_SET: keys[start0 + t]).
struct RowKeys {
  int64_t count;
  // segment 0: keys start0 + step0 * t for t < len0
  int64_t start0, step0, len0;
  // segment 1 (contiguous): keys start1 + t for t < count - len0
  int64_t start1;
};

MA_HD RowKeys row_keys(const PatternParams& p, int64_t i) {
  RowKeys r{0, 0, 1, 0, 0};
  const int64_t N = p.n;
  if (i < 0 || i >= N) return r;
  switch (p.pattern) {
    case kSliding: {
      const int64_t dl = p.dilation;
      const int64_t tlo = imax64(-p.left, -floordiv64(i, dl));
      const int64_t thi = imin64(p.right, floordiv64(N - 1 - i, dl));
      const int64_t len = thi >= tlo ? thi - tlo + 1 : 0;
      r.count = len;
      r.start0 = i + dl * tlo;
      r.step0 = dl;
      r.len0 = len;
      break;
    }
    case kDense: {
      const int64_t len = p.causal ? i + 1 : N;
      r.count = len;
      r.len0 = len;
      break;
    }
    case kBlockSparse: {
      // count only; keys come from block_key()
      const int64_t bs = p.block_size, row = i / bs;
      int64_t cnt = 0;
      for (int64_t e = 0; e < p.bpr; ++e) {
        const int32_t c = p.table[row * p.bpr + e];
        if (c < 0) continue;
        cnt += imin64(bs, N - (int64_t)c * bs);
      }
      r.count = cnt;
      r.len0 = cnt;
      break;
    }
    case kLongformer: {
      const int64_t G = imin64(p.num_global, N);
      if (i < G) {
        r.count = N;
        r.len0 = N;
      } else {
        const int64_t lo = imax64(imax64(i - p.left, 0), G);
        const int64_t hi = imin64(i + p.right, N - 1);
        const int64_t loc = hi >= lo ? hi - lo + 1 : 0;
        r.len0 = G;
        r.start1 = lo;
        r.count = G + loc;
      }
      break;
    }
    case kIndexSet: {
      const int64_t lo = imin64(imax64(p.offsets[i], 0), p.nnz);
      const int64_t hi = imin64(imax64(p.offsets[i + 1], lo), p.nnz);
      r.count = hi - lo;
      r.start0 = lo;
      r.len0 = r.count;
      break;
    }
    default:
      r.count = -1;
  }
  return r;
}

// t-th key (0 <= t < count) of BLOCK_SPARSE row i.
MA_HD int64_t block_key(const PatternParams& p, int64_t i, int64_t t) {
  const int64_t bs = p.block_size, row = i / bs;
  for (int64_t e = 0; e < p.bpr; ++e) {
    const int32_t c = p.table[row * p.bpr + e];
    if (c < 0) continue;
    const int64_t len = imin64(bs, p.n - (int64_t)c * bs);
    if (t < len) return (int64_t)c * bs + t;
    t -= len;
  }
  return -1;
}

// t-th key (0 <= t < rk.count) of row i.
MA_HD int64_t key_at(const PatternParams& p, const RowKeys& rk, int64_t i, int64_t t) {
  if (p.pattern == kBlockSparse) return block_key(p, i, t);
  if (p.pattern == kIndexSet) return p.keys[rk.start0 + t];
  return t < rk.len0 ? rk.start0 + rk.step0 * t : rk.start1 + (t - rk.len0);
}

// Membership of key j in S_i for the banded patterns (SLIDING with dilation 1
// in the residue-class index space, LONGFORMER local rows); used as the
// per-element mask of the tiled kernels.
MA_HD bool in_window(int64_t qm, int64_t km, int64_t left, int64_t right) {
  return km >= qm - left && km <= qm + right;
}

}  // namespace ma
