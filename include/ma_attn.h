/*
 * ma_attn.h -- C-ABI of the MI355X sparse-attention forward engine (gfx950).
 *
 * Plain C: integer sizes, raw device pointers and a hipStream_t passed as
 * void*.  No torch or HIP types appear in these signatures, so any host
 * language (ctypes, cffi, a C++ extension) can bind them.
 *
 * Layout of every Q/K/V/O buffer: [batch, seq_len, num_heads, head_dim],
 * head_dim fastest, contiguous (the reference's NWHD layout,
 * src/csrc/tensor.cpp:108 and src/cuda/sparse_attention_kernel.cu:28-32).
 * Q, K, V and O share one dtype.  O is written exactly once per row.
 *
 * Index sets S_i (key positions query i attends, ascending, clipped to [0,N)):
 *   SLIDING      { i + dilation*t : -left <= t <= right }
 *                (reference window_size=w  <=>  left = right = w, dilation 1)
 *   DENSE        [0, N), or [0, i] when causal
 *   BLOCK_SPARSE union over c in block_table[i / block_size][*] (c >= 0)
 *                of [c*block_size, min((c+1)*block_size, N))
 *   LONGFORMER   i <  num_global: [0, N)
 *                i >= num_global: { i - left .. i + right } U [0, num_global)
 *                (set union, every key once)
 *   INDEX_SET    index_keys[index_offsets[i] .. index_offsets[i+1]): an
 *                explicit key set per query row (CSR), shared by every
 *                (batch, head), as the reference's generic COO attention
 *                (src/csrc/sparse_attention.cpp:11-152) takes one pattern for
 *                all of them.  Keys ascending and distinct within a row: the
 *                reference path exponentiates a repeated entry twice
 *                (:98-108); here a key set is a set.
 * An empty S_i gives an all-zero output row (src/csrc/ma_core.cpp:212).
 *
 * Return codes: 0 on success, non-zero on invalid input or launch failure;
 * ma_attn_last_error() then holds a message.  Nothing is launched on invalid
 * input.  All calls are asynchronous on the given stream and never allocate.
 */
#ifndef MA_ATTN_H
#define MA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum ma_attn_dtype {
  MA_ATTN_F32 = 0,
  MA_ATTN_BF16 = 1,
  MA_ATTN_F16 = 2
};

enum ma_attn_pattern {
  MA_ATTN_SLIDING = 0,
  MA_ATTN_DENSE = 1,
  MA_ATTN_BLOCK_SPARSE = 2,
  MA_ATTN_LONGFORMER = 3,
  MA_ATTN_INDEX_SET = 4
};

/*
 * The 64x64-tile form of an INDEX_SET key set (ma_attn_tile_plan builds it
 * on the host; the caller copies the blob to the device).  Entries are the
 * (query tile t, key block c) pairs that hold at least one key of the set,
 * ordered by tile, then block.  All offsets are bytes into the blob.
 */
typedef struct ma_attn_tile_header {
  int64_t seq_len;        /* N of the set */
  int64_t num_tiles;      /* ceil(N / 64): query tiles, and key blocks */
  int64_t num_entries;
  int64_t seg;            /* entries per work item: longer tile rows (and key-block
                             columns) are split over several items, merged after */
  int64_t num_q_items;    /* query-side work items (forward, statistics, dQ) */
  int64_t num_q_split;    /* query tiles split over more than one item */
  int64_t num_q_partials; /* items of split query tiles: one partial result each */
  int64_t num_k_items;    /* key-side work items (dK, dV) */
  int64_t num_k_split;
  int64_t num_k_partials;
  int64_t off_blk;        /* int32 [num_entries]: key block, bit 30 set when all 64x64 pairs are in the set */
  int64_t off_mask;       /* uint64 [num_entries][64]: bit k of word r <=> key 64*blk + k in S_(64*tile + r) */
  int64_t off_kmask;      /* uint64 [num_entries][64]: the transpose, bit r of word k (same condition) */
  int64_t off_tile;       /* int32 [num_entries]: query tile of the entry */
  int64_t off_kentry;     /* int32 [num_entries]: entry ids ordered by key block, then tile */
  int64_t off_q_items;    /* int32 [num_q_items][4]: tile, first entry, end entry, partial slot or -1 */
  int64_t off_q_split;    /* int32 [num_q_split][4]: tile, first slot, slot count, 0 */
  int64_t off_k_items;    /* int32 [num_k_items][4]: key block, first and end position in kentry, slot or -1 */
  int64_t off_k_split;    /* int32 [num_k_split][4]: key block, first slot, slot count, 0 */
  int64_t total_bytes;
  int64_t num_masked;     /* entries without bit 30 (not every pair in the set); -1 after the
                             sizes-only call (plan NULL).  0 lets the kernels skip all mask work */
} ma_attn_tile_header;

typedef struct ma_attn_desc {
  int64_t batch;
  int64_t seq_len;
  int64_t num_heads;
  int64_t head_dim;
  int32_t dtype;    /* enum ma_attn_dtype */
  int32_t pattern;  /* enum ma_attn_pattern */
  int64_t left;     /* SLIDING / LONGFORMER: taps before i */
  int64_t right;    /* SLIDING / LONGFORMER: taps after i */
  int64_t dilation; /* SLIDING: stride between taps, >= 1 */
  int32_t causal;   /* DENSE: 1 => keys [0, i] */
  int32_t reserved0;
  int64_t block_size;         /* BLOCK_SPARSE: rows per block, >= 1 */
  const int32_t* block_table; /* BLOCK_SPARSE: device int32 [ceil(N/bs), blocks_per_row],
                                 ascending, -1 padded */
  int64_t blocks_per_row;     /* BLOCK_SPARSE: table width */
  int64_t num_global;         /* LONGFORMER: global tokens at positions 0..G-1 */
  float scale;                /* softmax scale; 0 => 1.0f / sqrtf((float)head_dim) */
  int32_t reserved1;
  const int64_t* index_offsets; /* INDEX_SET: device int64 [seq_len + 1], non-decreasing,
                                   index_offsets[0] = 0, index_offsets[seq_len] = num_indices */
  const int32_t* index_keys;    /* INDEX_SET: device int32 [num_indices], each row's keys
                                   ascending and distinct, in [0, seq_len) */
  int64_t num_indices;          /* INDEX_SET: length of index_keys */
  const int64_t* index_t_offsets; /* INDEX_SET backward only: the transposed set, device int64
                                     [seq_len + 1]: key j is listed by the queries
                                     index_t_queries[index_t_offsets[j] .. index_t_offsets[j+1]) */
  const int32_t* index_t_queries; /* INDEX_SET backward only: device int32 [num_indices], ascending
                                     per key */
  const ma_attn_tile_header* tile_header; /* INDEX_SET, optional: HOST copy of the set's tile plan
                                             header; with tile_plan, head_dim 64 runs the tiled
                                             MFMA kernels (forward and backward) */
  const void* tile_plan;                  /* INDEX_SET, optional: DEVICE copy of the whole plan */
} ma_attn_desc;

/*
 * Sparse-attention forward: O = softmax_j(<Q_i, K_j> * scale) V over j in S_i.
 * Replaces the reference's extension entry points
 *   sparse_forward_cuda   src/cuda/sparse_attention_kernel.cu:423-458 (SLIDING, left=right=w)
 *   dense_forward_cuda    src/cuda/sparse_attention_kernel.cu:348-382 (DENSE)
 * and the CPU engine it is checked against,
 *   ma_core::compute_sparse_attention  src/csrc/ma_core.cpp:160-246
 *   ma_core::compute_dense_attention   src/csrc/ma_core.cpp:66-157,
 * and gives the block-sparse / Longformer patterns of
 *   src/csrc/sparse_attention.cpp:203-259 and the generic index-set attention
 *   of :11-152 (INDEX_SET) a working forward.  INDEX_SET reads its offsets
 *   and keys as given, with every access kept inside them: a row's offsets
 *   are clamped into [0, num_indices] and keys outside [0, seq_len) are
 *   skipped, so malformed sets give wrong rows, never a fault.
 * workspace: device memory of ma_attn_workspace_size(desc) bytes (may be NULL
 * when that size is 0).  stream: a hipStream_t (NULL = default stream).
 */
int ma_attn_forward(const ma_attn_desc* desc, const void* q, const void* k,
                    const void* v, void* o, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Bytes of device workspace ma_attn_forward needs for desc (0 for most
 * patterns).  No reference counterpart: the reference allocates inside its
 * extension (sparse_attention_kernel.cu:440); this engine never allocates. */
size_t ma_attn_workspace_size(const ma_attn_desc* desc);

/*
 * Sparse-attention backward: given dout = dL/dO, writes dq, dk, dv (each
 * [B,N,H,D] in desc->dtype, every row written) for the SLIDING and DENSE
 * patterns, recomputing the softmax from q, k, v (no saved forward state),
 * as the reference's backward entry points do:
 *   sparse_backward_cuda  src/cuda/sparse_attention_kernel.cu:459-497 (SLIDING, left=right=w;
 *                         kernel :265-346)
 *   dense_backward_cuda   src/cuda/sparse_attention_kernel.cu:383-418 (DENSE; kernel :104-175)
 * generalised to any left/right/dilation and to bf16/fp16 (fp32 arithmetic),
 * for INDEX_SET, which also needs the transposed set (index_t_offsets,
 * index_t_queries: for each key, the queries that list it), and for
 * LONGFORMER in 16 bits at head_dim 64 with right = 0, 0 <= left < 128 and 1
 * to 16 global tokens (a forward that writes each row's lse and
 * delta_i = sum_j P_ij dP_ij, dP_ij = dout_i . v_j, in fp32, then the
 * one-pass backward of ma_attn_backward_saved from them).  Other patterns
 * return non-zero.  workspace: device memory of
 * ma_attn_backward_workspace_size(desc) bytes (per-row softmax statistics;
 * LONGFORMER also the per-segment partial sums of the global rows and keys).
 */
int ma_attn_backward(const ma_attn_desc* desc, const void* q, const void* k,
                     const void* v, const void* dout, void* dq, void* dk,
                     void* dv, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Bytes of device workspace ma_attn_backward needs (8 per (b, i, h) row;
 * LONGFORMER adds the forward's and the backward's partial sums).
 * No reference counterpart: the reference keeps no statistics (it recomputes
 * them per gradient pass, sparse_attention_kernel.cu:285-304). */
size_t ma_attn_backward_workspace_size(const ma_attn_desc* desc);

/*
 * ma_attn_forward / ma_attn_backward with the call's kernels bracketed by two
 * caller-created HIP events (hipEvent_t, either may be NULL): start_event
 * records when the call's first kernel starts and stop_event when its last
 * kernel ends, stamped on the kernels' own dispatches (hipExtLaunchKernel), so
 * their difference is the kernels' execution time without the gaps between
 * launches.  For timing; no counterpart in the reference.
 */
int ma_attn_forward_timed(const ma_attn_desc* desc, const void* q, const void* k,
                          const void* v, void* o, void* workspace,
                          size_t workspace_bytes, void* stream,
                          void* start_event, void* stop_event);
int ma_attn_backward_timed(const ma_attn_desc* desc, const void* q, const void* k,
                           const void* v, const void* dout, void* dq, void* dk,
                           void* dv, void* workspace, size_t workspace_bytes,
                           void* stream, void* start_event, void* stop_event);

/*
 * Training pair with saved statistics.  No reference counterpart: the
 * reference's backward recomputes every softmax from q, k, v
 * (src/cuda/sparse_attention_kernel.cu:265-346, its autograd path
 * src/layers/ma_core_bridge.py:116-154); a forward that also keeps each
 * row's statistic lets the backward skip that.
 *
 * ma_attn_forward_lse: ma_attn_forward (same o, same workspace) that also
 * writes lse[(b*N + i)*H + h] (float32, B*N*H entries): log2 of row i's
 * softmax denominator sum_j 2^(scale*log2(e)*q_i.k_j) (0 for a row with no
 * key).  Taken by the kernels that produce it at head_dim 64: BLOCK_SPARSE
 * (block size 64) and DENSE on the block-row kernel, LONGFORMER with 1 to
 * 16 global tokens on the stream kernel (any dtype), INDEX_SET with a tile
 * plan; otherwise non-zero with an error.
 *
 * ma_attn_backward_saved: the gradients of ma_attn_backward from the
 * forward's o and lse (delta_i = dout_i . o_i), for an INDEX_SET with a tile
 * plan, which may hold the key sets of a BLOCK_SPARSE or LONGFORMER forward
 * (ma_attn_pattern_csr enumerates them), for DENSE (head_dim 64), and for
 * LONGFORMER itself in 16 bits at head_dim 64 with right = 0, 0 <= left < 128
 * and 1 to 16 global tokens (one pass over the sequence; per-segment sums of
 * the global rows' and keys' gradients in the workspace).
 * Workspace: ma_attn_backward_workspace_size(desc).  The _timed forms stamp
 * their kernels as ma_attn_forward_timed / ma_attn_backward_timed do (either
 * event may be NULL, so a forward_lse + backward_saved pair can be stamped
 * as one span).
 */
int ma_attn_forward_lse(const ma_attn_desc* desc, const void* q, const void* k,
                        const void* v, void* o, float* lse, void* workspace,
                        size_t workspace_bytes, void* stream);
int ma_attn_forward_lse_timed(const ma_attn_desc* desc, const void* q, const void* k,
                              const void* v, void* o, float* lse, void* workspace,
                              size_t workspace_bytes, void* stream, void* start_event,
                              void* stop_event);
int ma_attn_backward_saved(const ma_attn_desc* desc, const void* q, const void* k,
                           const void* v, const void* o, const float* lse,
                           const void* dout, void* dq, void* dk, void* dv,
                           void* workspace, size_t workspace_bytes, void* stream);
int ma_attn_backward_saved_timed(const ma_attn_desc* desc, const void* q, const void* k,
                                 const void* v, const void* o, const float* lse,
                                 const void* dout, void* dq, void* dk, void* dv,
                                 void* workspace, size_t workspace_bytes, void* stream,
                                 void* start_event, void* stop_event);

/* Validates desc without launching; 0 when ma_attn_forward would accept it.
 * Mirrors the checks of sparse_attention_kernel.cu:427-432. */
int ma_attn_validate(const ma_attn_desc* desc);

/* Message for the last non-zero return on this thread ("" if none). */
const char* ma_attn_last_error(void);

/*
 * Host: seeded block table for BLOCK_SPARSE.  Row r holds {r} U {r-1 if r>=1}
 * U `random_per_row` distinct blocks drawn uniformly (SplitMix64 keyed by
 * (seed, r), rejection sampling) from the remaining blocks, sorted ascending,
 * -1 padded to width 2 + random_per_row.  Replaces the unseeded
 * BlockSparseAttention / create_random_sparse_pattern generators
 * (src/csrc/sparse_attention.cpp:203-231, :287-310).
 * table_out: host int32 [num_blocks, 2 + random_per_row].
 */
int ma_attn_block_table(uint64_t seed, int64_t num_blocks,
                        int64_t random_per_row, int32_t* table_out);

/*
 * Host: the ascending key list S_i of query row i for desc (block_table, if
 * used, is a HOST pointer here).  Writes min(|S_i|, cap) keys to keys_out and
 * returns |S_i|, or -1 on invalid input (INDEX_SET included: its sets are
 * the caller's own input).  The same closed forms drive the kernels; this
 * exposes them for bit-exact index checks.  Replaces the COO
 * generators create_sliding_window_pattern (src/csrc/ma_core.cpp:34-48) and
 * SlidingWindow/Longformer generate_sparse_pattern
 * (src/csrc/sparse_attention.cpp:181-259).
 */
int64_t ma_attn_row_keys(const ma_attn_desc* desc, const int32_t* host_block_table,
                         int64_t i, int64_t* keys_out, int64_t cap);

/*
 * Host: every row's key list of desc at once, as CSR.  offsets_out (host
 * int64 [seq_len + 1], may be NULL) receives the row offsets; keys_out (host
 * int32 [keys_cap], may be NULL) the keys, row after row, each row ascending.
 * Returns the total key count (nnz), or -1 on invalid input or when keys_out
 * is given and keys_cap < nnz.  Call once with keys_out = NULL for the count.
 * The same closed forms as ma_attn_row_keys, one call instead of one per row.
 * Replaces the reference's whole-pattern COO generators
 * create_sliding_window_pattern (src/csrc/ma_core.cpp:34-48) and
 * generate_sparse_pattern (src/csrc/sparse_attention.cpp:181-259), which emit
 * (row, col) lists of the same entries.
 */
int64_t ma_attn_pattern_csr(const ma_attn_desc* desc, const int32_t* host_block_table,
                            int64_t* offsets_out, int32_t* keys_out, int64_t keys_cap);

/*
 * ma_attn_forward for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  It takes no workspace and allocates
 * nothing: the two forward kernels that need scratch, the Longformer stream
 * kernel (its per-chunk partials of the global rows) and the tiled index-set
 * kernel (the partial results of a tile plan's split rows), take their
 * ma_attn_workspace_size(desc) bytes from a static device array of
 * MA_ATTN_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs
 * on until the process ends.  A call needing more is rejected with a
 * message and launches nothing.  Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (concurrent streams or threads) race.
 * Outputs are identical to ma_attn_forward's on the same inputs.
 */
int ma_attn_forward_noalloc(const ma_attn_desc* desc, const void* q, const void* k,
                            const void* v, void* o, void* stream);

#define MA_ATTN_NOALLOC_SCRATCH_BYTES (8u << 20)

/* Re-reads the kernel-selection switches (MA_ATTN_KERNEL, MA_ATTN_NO_FIXED,
 * MA_ATTN_BWD_NO_FIXED) from the environment; the library reads them once when
 * it loads.  For tests and A/B timing; no reference counterpart. */
void ma_attn_reload_options(void);

/*
 * Host: the tile plan of a CSR key set (host offsets [seq_len + 1], keys
 * [offsets[seq_len]], each row ascending, keys in [0, seq_len)).  seg: entries
 * per work item (0: the library's default).  With plan NULL, fills header
 * only (sizes and offsets); then, given plan of header->total_bytes bytes,
 * writes the whole plan (the header first).  Returns 0, or -1 on invalid
 * input.  No reference counterpart: the reference's generic COO attention
 * (src/csrc/sparse_attention.cpp:11-152) scans an N x N score matrix per
 * (batch, head); the plan is what lets this engine run an explicit set on
 * 64x64 MFMA tiles with per-row bit masks.
 */
int ma_attn_tile_plan(int64_t seq_len, const int64_t* offsets, const int32_t* keys, int64_t seg,
                      ma_attn_tile_header* header, void* plan, size_t plan_bytes);

/*
 * Measurement: a forward kernel's memory traffic for desc without its
 * arithmetic.  SLIDING (head_dim 64): the stream kernel's workgroups, chunks,
 * 64-row tiles of one (batch, head) and halo blocks, writing o = q xor k xor v
 * bitwise.  BLOCK_SPARSE (block_size 64, head_dim 64, blocks_per_row <= 4, a
 * device table as ma_attn_forward takes): the block-row kernel's workgroups,
 * each reading its row's Q tile and listed K/V blocks and writing
 * o[i] = q[i] xor (xor over the row's blocks c of k[64c + i%64] xor
 * v[64c + i%64]).  Gives the copy speed of that kernel's access pattern on the
 * device, the ceiling it runs against.  Returns non-zero when the kernel would
 * not take desc.  The _timed form stamps the kernel's start and stop on two
 * caller-created events, as ma_attn_forward_timed.  No reference counterpart.
 */
int ma_attn_copy_probe(const ma_attn_desc* desc, const void* q, const void* k, const void* v,
                       void* o, void* stream);
int ma_attn_copy_probe_timed(const ma_attn_desc* desc, const void* q, const void* k,
                             const void* v, void* o, void* stream, void* start_event,
                             void* stop_event);

/*
 * Measurement: the fused backward's memory traffic for desc without its
 * arithmetic (SLIDING, bf16/fp16, head_dim 64, windows [i-63, i] and
 * [i-32, i+31] of any dilation: the descriptors ma_attn_backward runs as one
 * fused launch).  The same workgroups, chunks and steps read the K, V, Q and
 * dO rows the kernel reads and write dq = q xor dout, dk = k, dv = v
 * bitwise, each row once, at the kernel's positions.  Gives the copy speed of
 * that access pattern on the device.  Returns non-zero when the fused kernel
 * would not take desc.  The _timed form stamps the kernel's start and stop on
 * two caller-created events.  No reference counterpart.
 */
int ma_attn_backward_copy_probe(const ma_attn_desc* desc, const void* q, const void* k,
                                const void* v, const void* dout, void* dq, void* dk, void* dv,
                                void* stream);
int ma_attn_backward_copy_probe_timed(const ma_attn_desc* desc, const void* q, const void* k,
                                      const void* v, const void* dout, void* dq, void* dk,
                                      void* dv, void* stream, void* start_event,
                                      void* stop_event);

/* ABI version of this header (bumped on incompatible change, and when an
 * entry point takes descriptors it refused before: 10, ma_attn_backward on
 * LONGFORMER). */
int ma_attn_abi_version(void);

#define MA_ATTN_ABI_VERSION 10

#ifdef __cplusplus
}
#endif

#endif /* MA_ATTN_H */
