// ref_driver.cpp -- a C entry layer over the reference's own CPU engine.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile together with the
// reference's untouched sources /root/reference/src/csrc/ma_core.cpp and
// tensor.cpp (the two files the reference's setup.py:49-51 builds beside its
// pybind layer) into oracle/_ref/libma_core_ref.so.  Nothing of the reference
// is copied here: this file only marshals raw float buffers into
// ma_core::Tensor (shape order (b, s, head_dim, heads), attention_types.hpp:67-68,
// as ma_core.cpp:19 builds it) and calls
//   ma_core::compute_sparse_attention   ma_core.cpp:160-246
//   ma_core::compute_dense_attention    ma_core.cpp:66-157
//   ma_core::create_sliding_window_pattern  ma_core.cpp:34-48
//   ma_core::get_pattern_statistics         ma_core.cpp:51-63
// so tests can hold the oracle restatement against the reference's own bits.
#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

#include "ma_core.hpp"

namespace {
ma_core::Tensor make(int64_t B, int64_t N, int64_t H, int64_t D, const float* src) {
  ma_core::Tensor t = ma_core::create_tensor({B, N, H, D});
  t.copy_from(src, static_cast<size_t>(B * N * H * D) * sizeof(float));
  return t;
}
}  // namespace

extern "C" int ref_sparse_forward(int64_t B, int64_t N, int64_t H, int64_t D, int64_t w,
                                  const float* q, const float* k, const float* v, float* o) {
  try {
    ma_core::Tensor tq = make(B, N, H, D, q), tk = make(B, N, H, D, k), tv = make(B, N, H, D, v);
    ma_core::Tensor out = ma_core::compute_sparse_attention(tq, tk, tv, w);
    out.copy_to(o, static_cast<size_t>(B * N * H * D) * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

extern "C" int ref_dense_forward(int64_t B, int64_t N, int64_t H, int64_t D, int causal,
                                 const float* q, const float* k, const float* v, float* o) {
  try {
    ma_core::Tensor tq = make(B, N, H, D, q), tk = make(B, N, H, D, k), tv = make(B, N, H, D, v);
    ma_core::Tensor out = ma_core::compute_dense_attention(tq, tk, tv, causal != 0);
    out.copy_to(o, static_cast<size_t>(B * N * H * D) * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// The same two calls with a value head_dim Dv of its own (the reference sizes
// O by the value's head_dim, ma_core.cpp:84-90, :178-183): q, k are
// [B, N, H, D], v and o [B, N, H, Dv].
extern "C" int ref_sparse_forward_v(int64_t B, int64_t N, int64_t H, int64_t D, int64_t Dv, int64_t w,
                                    const float* q, const float* k, const float* v, float* o) {
  try {
    ma_core::Tensor tq = make(B, N, H, D, q), tk = make(B, N, H, D, k), tv = make(B, N, H, Dv, v);
    ma_core::Tensor out = ma_core::compute_sparse_attention(tq, tk, tv, w);
    out.copy_to(o, static_cast<size_t>(B * N * H * Dv) * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

extern "C" int ref_dense_forward_v(int64_t B, int64_t N, int64_t H, int64_t D, int64_t Dv, int causal,
                                   const float* q, const float* k, const float* v, float* o) {
  try {
    ma_core::Tensor tq = make(B, N, H, D, q), tk = make(B, N, H, D, k), tv = make(B, N, H, Dv, v);
    ma_core::Tensor out = ma_core::compute_dense_attention(tq, tk, tv, causal != 0);
    out.copy_to(o, static_cast<size_t>(B * N * H * Dv) * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}

// COO entries of create_sliding_window_pattern(N, w); returns nnz, writes up to cap.
extern "C" int64_t ref_sliding_pattern(int64_t N, int64_t w, int64_t* rows, int64_t* cols,
                                       int64_t cap) {
  try {
    ma_core::SparseTensor p = ma_core::create_sliding_window_pattern(N, w);
    int64_t n = p.nnz();
    for (int64_t e = 0; e < n && e < cap; ++e) {
      rows[e] = p.row_indices[e];
      cols[e] = p.col_indices[e];
    }
    return n;
  } catch (const std::exception&) {
    return -1;
  }
}

// get_pattern_statistics(create_sliding_window_pattern(N, w)) as a C string;
// returns its length (written up to cap - 1 bytes plus a NUL), -1 on error.
extern "C" int64_t ref_pattern_statistics(int64_t N, int64_t w, char* out, int64_t cap) {
  try {
    const std::string s = ma_core::get_pattern_statistics(ma_core::create_sliding_window_pattern(N, w));
    const int64_t n = static_cast<int64_t>(s.size());
    if (cap > 0) {
      const int64_t m = n < cap - 1 ? n : cap - 1;
      std::memcpy(out, s.data(), static_cast<size_t>(m));
      out[m] = 0;
    }
    return n;
  } catch (const std::exception&) {
    return -1;
  }
}
