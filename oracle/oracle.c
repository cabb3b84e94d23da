/*
 * oracle.c -- CPU restatement of the reference sparse-attention forward and
 * backward.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * engine and the CPU baseline timed by bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product path never does.
 *
 * Arithmetic follows ma_core::compute_sparse_attention
 * (/root/reference src/csrc/ma_core.cpp:160-246) operation for operation:
 *   scores[t] = (sum_d q[d]*k[j_t][d]) * scale     sequential fp32 (:202-209)
 *   m = max_t scores[t]                             (:214-217)
 *   e_t = expf(scores[t] - m); sum += e_t            (:220-224)
 *   p_t = e_t / sum                                  (:227-229)
 *   o[d] = sum_t p_t * v[j_t][d]                     sequential (:232-239)
 *   empty key set => zero row                        (:185, :212)
 * with scale = 1.0f / sqrtf((float)D) (:188).  The only generalisation is the
 * key list: the reference's window [max(0,i-w), min(N,i+w+1)) (:197-198)
 * becomes an explicit ascending list j_0 < j_1 < ... produced by
 * oracle_row_keys() for each pattern below.  Layout is [B,N,H,D]
 * (src/csrc/tensor.cpp:108).
 *
 * Build with -ffp-contract=off so products and sums round separately, as the
 * reference's -O3 x86-64 build does (setup.py:55; no FMA in the baseline ISA).
 *
 * Patterns (the frozen index-set specification):
 *   0 SLIDING      {i + dil*t : -left <= t <= right} n [0,N)
 *                  (reference window w: left = right = w, dil = 1,
 *                   ma_core.cpp:197-198; dilation from
 *                   doc/sparse_attention_whitepaper.md:98-104)
 *   1 DENSE        [0,N) or [0,i] if causal (ma_core.cpp:66-157: the -1e9
 *                  causal fill of :114-120 gives expf(...)=0 exactly, so it
 *                  equals dropping those keys)
 *   2 BLOCK_SPARSE union of table blocks of row-block i/bs
 *                  (intent of src/csrc/sparse_attention.cpp:203-231)
 *   3 LONGFORMER   i < G: [0,N); else [i-left, i+right] U [0,G), no duplicates
 *                  (intent of sparse_attention.cpp:234-259 and
 *                   whitepaper :109-124)
 *   4 INDEX_SET    keys[offsets[i] .. offsets[i+1]) given by the caller (CSR),
 *                  every key once and ascending: the generic COO attention of
 *                  sparse_attention.cpp:11-152 over a set.  That path scales
 *                  Q before the dot product (:25-26) where ma_core scales the
 *                  dot (:209); with D a power of 4 the scale is a power of two
 *                  and the two orders give the same bits.  Its one-pattern-
 *                  for-all-heads rule is kept; its double exponentiation of a
 *                  repeated entry (:98-108) is not: repeated or unsorted keys
 *                  are rejected (-1).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef struct oracle_spec {
  int64_t B, N, H, D;
  int32_t pattern;
  int32_t causal;
  int64_t left, right, dilation;
  int64_t block_size;
  const int32_t* table; /* host, [ceil(N/bs), bpr] */
  int64_t bpr;
  int64_t num_global;
  const int64_t* offsets; /* INDEX_SET: host [N+1] */
  const int32_t* keys;    /* INDEX_SET: host [nnz] */
  int64_t nnz;
} oracle_spec;

static int64_t imax(int64_t a, int64_t b) { return a > b ? a : b; }
static int64_t imin(int64_t a, int64_t b) { return a < b ? a : b; }

/* floor division for possibly negative numerators, positive d */
static int64_t fdiv(int64_t a, int64_t d) {
  int64_t q = a / d;
  if ((a % d != 0) && (a < 0)) q -= 1;
  return q;
}

/* Ascending key list of row i.  Returns the count; writes at most cap keys. */
int64_t oracle_row_keys(const oracle_spec* s, int64_t i, int64_t* out, int64_t cap) {
  int64_t n = 0;
  const int64_t N = s->N;
#define PUSH(j)                  \
  do {                           \
    if (n < cap) out[n] = (j);   \
    n++;                         \
  } while (0)
  if (i < 0 || i >= N) return 0;
  switch (s->pattern) {
    case 0: { /* SLIDING: t from -left to right, key i + dil*t inside [0,N) */
      const int64_t dl = s->dilation;
      if (dl < 1) return -1;
      /* smallest t with i + dl*t >= 0 : t >= ceil(-i/dl) */
      int64_t tlo = imax(-s->left, -fdiv(i, dl));
      /* largest t with i + dl*t <= N-1 : t <= floor((N-1-i)/dl) */
      int64_t thi = imin(s->right, fdiv(N - 1 - i, dl));
      for (int64_t t = tlo; t <= thi; ++t) PUSH(i + dl * t);
      break;
    }
    case 1: { /* DENSE */
      int64_t hi = s->causal ? i : N - 1;
      for (int64_t j = 0; j <= hi; ++j) PUSH(j);
      break;
    }
    case 2: { /* BLOCK_SPARSE: table entries are ascending, -1 padded */
      const int64_t bs = s->block_size;
      if (bs < 1) return -1;
      const int64_t r = i / bs;
      for (int64_t e = 0; e < s->bpr; ++e) {
        int32_t c = s->table[r * s->bpr + e];
        if (c < 0) continue;
        int64_t lo = (int64_t)c * bs, hi = imin((int64_t)(c + 1) * bs, N);
        for (int64_t j = lo; j < hi; ++j) PUSH(j);
      }
      break;
    }
    case 3: { /* LONGFORMER */
      const int64_t G = imin(s->num_global, N);
      if (i < G) {
        for (int64_t j = 0; j < N; ++j) PUSH(j);
      } else {
        int64_t lo = imax(i - s->left, 0), hi = imin(i + s->right, N - 1);
        for (int64_t j = 0; j < G; ++j) PUSH(j);
        for (int64_t j = imax(lo, G); j <= hi; ++j) PUSH(j);
      }
      break;
    }
    case 4: { /* INDEX_SET */
      const int64_t a = s->offsets[i], b = s->offsets[i + 1];
      if (a < 0 || b < a || b > s->nnz) return -1;
      for (int64_t t = a; t < b; ++t) {
        const int64_t j = s->keys[t];
        if (j < 0 || j >= N || (t > a && j <= s->keys[t - 1])) return -1;
        PUSH(j);
      }
      break;
    }
    default:
      return -1;
  }
#undef PUSH
  return n;
}

/* INDEX_SET well-formed: offsets from 0 to nnz, non-decreasing; each row's
 * keys strictly ascending inside [0,N).  Other patterns: always 1. */
static int index_set_ok(const oracle_spec* s) {
  if (s->pattern != 4) return 1;
  if (s->N > 0 && (!s->offsets || s->offsets[0] != 0 || s->offsets[s->N] != s->nnz)) return 0;
  if (s->nnz > 0 && !s->keys) return 0;
  for (int64_t i = 0; i < s->N; ++i) {
    const int64_t a = s->offsets[i], b = s->offsets[i + 1];
    if (b < a) return 0;
    for (int64_t t = a; t < b; ++t)
      if (s->keys[t] < 0 || s->keys[t] >= s->N || (t > a && s->keys[t] <= s->keys[t - 1])) return 0;
  }
  return 1;
}

/*
 * fp32 forward over rows b in [0,B), heads [h_lo,h_hi), queries [i_lo,i_hi).
 * Rows outside the ranges are left untouched.  Returns 0, or -1 on bad input.
 */
int oracle_forward_f32(const oracle_spec* s, const float* q, const float* k,
                       const float* v, float* o, int64_t h_lo, int64_t h_hi,
                       int64_t i_lo, int64_t i_hi) {
  const int64_t N = s->N, H = s->H, D = s->D;
  if (N < 0 || H < 0 || D <= 0 || !index_set_ok(s)) return -1;
  const float scale = 1.0f / sqrtf((float)D);
  int64_t cap = N > 0 ? N : 1;
  int64_t* keys = (int64_t*)malloc(sizeof(int64_t) * (size_t)cap);
  float* scores = (float*)malloc(sizeof(float) * (size_t)cap);
  if (!keys || !scores) {
    free(keys);
    free(scores);
    return -1;
  }
  for (int64_t b = 0; b < s->B; ++b) {
    for (int64_t h = h_lo; h < h_hi; ++h) {
      for (int64_t i = i_lo; i < i_hi; ++i) {
        const float* qi = q + ((b * N + i) * H + h) * D;
        float* oi = o + ((b * N + i) * H + h) * D;
        int64_t n = oracle_row_keys(s, i, keys, cap);
        if (n <= 0) {
          for (int64_t d = 0; d < D; ++d) oi[d] = 0.0f;
          continue;
        }
        for (int64_t t = 0; t < n; ++t) {
          const float* kj = k + ((b * N + keys[t]) * H + h) * D;
          float score = 0.0f;
          for (int64_t d = 0; d < D; ++d) score += qi[d] * kj[d];
          scores[t] = score * scale;
        }
        float m = scores[0];
        for (int64_t t = 1; t < n; ++t) m = (m < scores[t]) ? scores[t] : m;
        float sum = 0.0f;
        for (int64_t t = 0; t < n; ++t) {
          scores[t] = expf(scores[t] - m);
          sum += scores[t];
        }
        for (int64_t t = 0; t < n; ++t) scores[t] /= sum;
        for (int64_t d = 0; d < D; ++d) {
          float acc = 0.0f;
          for (int64_t t = 0; t < n; ++t) {
            const float* vj = v + ((b * N + keys[t]) * H + h) * D;
            acc += scores[t] * vj[d];
          }
          oi[d] = acc;
        }
      }
    }
  }
  free(keys);
  free(scores);
  return 0;
}

/*
 * fp32 backward: dq, dk, dv (each [B,N,H,D], zero-filled here) for
 * dout = dL/dO, restating sparse_attention_backward_kernel
 * (/root/reference src/cuda/sparse_attention_kernel.cu:265-346; the dense
 * twin :104-175 is the same with keys [0,N) or [0,i]) per query row i:
 *   1) s_t = (sum_d q[d]*k[j_t][d]) * scale; m = max_t s_t;
 *      sum = sum_t expf(s_t - m), 1 if 0                      (:285-304)
 *   2) p_t = expf(s_t - m) / sum; dp_t = sum_d dout[d]*v[j_t][d];
 *      sdot += dp_t * p_t; dv[j_t] += p_t * dout              (:306-323)
 *   3) ds_t = (dp_t - sdot) * p_t; dq += ds_t*scale*k[j_t];
 *      dk[j_t] += ds_t*scale*q                                (:325-345)
 * over the pattern's ascending key list (oracle_row_keys).  The reference's
 * atomicAdd order across rows is unspecified; here rows accumulate in
 * ascending (b, h, i) order.
 */
int oracle_backward_f32(const oracle_spec* s, const float* q, const float* k,
                        const float* v, const float* dout, float* dq, float* dk,
                        float* dv) {
  const int64_t N = s->N, H = s->H, D = s->D, B = s->B;
  if (N < 0 || H < 0 || D <= 0 || B < 0 || !index_set_ok(s)) return -1;
  const float scale = 1.0f / sqrtf((float)D);
  const int64_t total = B * N * H * D;
  for (int64_t x = 0; x < total; ++x) dq[x] = dk[x] = dv[x] = 0.0f;
  int64_t cap = N > 0 ? N : 1;
  int64_t* keys = (int64_t*)malloc(sizeof(int64_t) * (size_t)cap);
  float* sc = (float*)malloc(sizeof(float) * (size_t)cap);
  float* dp = (float*)malloc(sizeof(float) * (size_t)cap);
  if (!keys || !sc || !dp) {
    free(keys);
    free(sc);
    free(dp);
    return -1;
  }
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      for (int64_t i = 0; i < N; ++i) {
        const int64_t ri = ((b * N + i) * H + h) * D;
        const int64_t n = oracle_row_keys(s, i, keys, cap);
        if (n <= 0) continue;
        float m = -INFINITY;
        for (int64_t t = 0; t < n; ++t) {
          const float* kj = k + ((b * N + keys[t]) * H + h) * D;
          float dot = 0.0f;
          for (int64_t d = 0; d < D; ++d) dot += q[ri + d] * kj[d];
          sc[t] = dot * scale;
          if (sc[t] > m) m = sc[t];
        }
        float sum = 0.0f;
        for (int64_t t = 0; t < n; ++t) sum += expf(sc[t] - m);
        if (sum == 0.0f) sum = 1.0f;
        float sdot = 0.0f;
        for (int64_t t = 0; t < n; ++t) {
          const int64_t rj = ((b * N + keys[t]) * H + h) * D;
          sc[t] = expf(sc[t] - m) / sum; /* p_t from here on */
          float acc = 0.0f;
          for (int64_t d = 0; d < D; ++d) acc += dout[ri + d] * v[rj + d];
          dp[t] = acc;
          sdot += acc * sc[t];
          for (int64_t d = 0; d < D; ++d) dv[rj + d] += sc[t] * dout[ri + d];
        }
        for (int64_t t = 0; t < n; ++t) {
          const int64_t rj = ((b * N + keys[t]) * H + h) * D;
          const float ds = (dp[t] - sdot) * sc[t];
          for (int64_t d = 0; d < D; ++d) {
            dq[ri + d] += ds * scale * k[rj + d];
            dk[rj + d] += ds * scale * q[ri + d];
          }
        }
      }
    }
  }
  free(keys);
  free(sc);
  free(dp);
  return 0;
}

/* SplitMix64 step (Steele, Lea, Flood 2014). */
static uint64_t splitmix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/*
 * Seeded block table: row r = sorted({r} U {r-1 if r>=1} U extra distinct
 * uniform picks from the other blocks), -1 padded to width 2 + extra.
 * Stream for row r starts at state = seed ^ (golden * (r + 1)); candidates are
 * z % nb with z rejected when z >= nb * floor(2^64 / nb) (no modulo bias),
 * and rejected again when already in the row.
 */
int oracle_block_table(uint64_t seed, int64_t nb, int64_t extra, int32_t* out) {
  if (nb < 0 || extra < 0) return -1;
  const int64_t w = 2 + extra;
  const uint64_t limit = nb > 0 ? (UINT64_MAX / (uint64_t)nb) * (uint64_t)nb : 0;
  for (int64_t r = 0; r < nb; ++r) {
    int32_t row[64];
    int64_t cnt = 0;
    if (w > 64) return -1;
    row[cnt++] = (int32_t)r;
    if (r >= 1) row[cnt++] = (int32_t)(r - 1);
    int64_t avail = nb - cnt;
    int64_t want = extra < avail ? extra : avail;
    uint64_t st = seed ^ (0x9E3779B97F4A7C15ull * (uint64_t)(r + 1));
    int64_t got = 0;
    while (got < want) {
      uint64_t z = splitmix64(&st);
      if (z >= limit) continue;
      int32_t c = (int32_t)(z % (uint64_t)nb);
      int dup = 0;
      for (int64_t e = 0; e < cnt; ++e) dup |= (row[e] == c);
      if (dup) continue;
      row[cnt++] = c;
      got++;
    }
    /* insertion sort ascending */
    for (int64_t a = 1; a < cnt; ++a) {
      int32_t x = row[a];
      int64_t b = a - 1;
      while (b >= 0 && row[b] > x) {
        row[b + 1] = row[b];
        b--;
      }
      row[b + 1] = x;
    }
    for (int64_t e = 0; e < w; ++e) out[r * w + e] = e < cnt ? row[e] : -1;
  }
  return 0;
}
