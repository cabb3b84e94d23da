/*
 * ma_encoder.h -- C-ABI of the fused encoder layer (gfx950): the eval-mode
 * forward of the reference's CustomTransformerEncoderLayer
 * (src/model.py:28-53) in one kernel launch.
 *
 *   attn = SparseAttention(src, src, src)      single head, head_dim = d_model,
 *                                              keys [i - window, i + window] of
 *                                              the token's own sequence, scale
 *                                              1/sqrtf(d_model)
 *                                              (src/layers/sparse_attention.py:49-86,
 *                                              src/csrc/ma_core.cpp:160-246)
 *   h    = LayerNorm1(src + attn)              (dropout1 is the identity in eval)
 *   out  = LayerNorm2(h + linear2(relu(linear1(h))))
 *
 * The reference runs this as separate PyTorch operations (attention, add,
 * LayerNorm, Linear, ReLU, Linear, add, LayerNorm).  Here every intermediate
 * stays on chip: a workgroup takes 16 tokens, reads their rows (plus the
 * window's neighbour rows) once, and writes the 16 output rows once; both
 * Linear layers run on fp32 MFMA.  Everything is float32.
 *
 * Layout: src, attn, out are [batch, seq_len, d_model] contiguous; Linear
 * weights are torch.nn.Linear's [out_features, in_features] row-major.  All
 * pointers are device pointers, 16-byte aligned; out must not overlap src or
 * attn.  d_model in {16, 32, 64, 128}; d_ff = 4 * d_model (the reference's).
 *
 * Return codes as include/ma_attn.h: 0 on success, non-zero with a message
 * in ma_attn_last_error() on invalid input (nothing launched) or launch
 * failure.  Asynchronous on `stream`; no allocation, no synchronisation.
 */
#ifndef MA_ENCODER_H
#define MA_ENCODER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ma_encoder_layer {
  int64_t batch;
  int64_t seq_len;
  int64_t d_model;
  int64_t d_ff;         /* must be 4 * d_model */
  int64_t window;       /* attention keys [i - window, i + window] (clipped to the sequence) */
  float ln_eps;         /* LayerNorm eps of both norms (torch default 1e-5) */
  int32_t reserved;
  const float* norm1_weight;   /* [d_model] */
  const float* norm1_bias;     /* [d_model] */
  const float* linear1_weight; /* [d_ff, d_model] */
  const float* linear1_bias;   /* [d_ff] */
  const float* linear2_weight; /* [d_model, d_ff] */
  const float* linear2_bias;   /* [d_model] */
  const float* norm2_weight;   /* [d_model] */
  const float* norm2_bias;     /* [d_model] */
} ma_encoder_layer;

/*
 * One encoder layer, eval mode.  attn = NULL: the kernel computes the layer's
 * sliding-window self-attention itself (one launch per layer).  attn given
 * ([batch, seq_len, d_model], e.g. from ma_attn_forward): only the block
 * after the attention runs (residual, LayerNorm1, linear1, ReLU, linear2,
 * residual, LayerNorm2).
 * Replaces CustomTransformerEncoderLayer.forward (src/model.py:42-53) with
 * model.eval().
 */
int ma_encoder_layer_forward(const ma_encoder_layer* layer, const float* src, const float* attn,
                             float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MA_ENCODER_H */
