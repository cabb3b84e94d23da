// device_common.h -- gfx950 device helpers shared by the attention kernels:
// vector types, MFMA selection per element type, buffer-resource loads and
// stores with hardware range checking, and the cross-lane reductions that
// combine the four lane groups sharing one MFMA column.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ma_dev {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// MFMA operand handling per 16-bit element type.
//   x32 : 16x16x32 (8 elements of the contraction per lane)
//   x16 : 16x16x16 (4 elements per lane)
template <typename T>
struct Mma;

template <>
struct Mma<__bf16> {
  static __device__ __forceinline__ f32x4 x32(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 x16(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b),
                                                     c, 0, 0, 0);
  }
  // x in the low half, y in the high half, each rounded to nearest even: one
  // v_cvt_pk_bf16_f32 (converting the two separately and shifting them
  // together costs four instructions)
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x, y}, bf16x2));
  }
};

template <>
struct Mma<_Float16> {
  static __device__ __forceinline__ f32x4 x32(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 x16(uint2 a, uint2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0,
                                                 0, 0);
  }
  // one v_cvt_pk_f16_f32 (round to nearest even)
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){x, y}, f16x2));
  }
};

// fp32 MFMA: 16x16x4, one contraction element per lane.
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- buffer resources
//
// A raw buffer resource (stride 0) covers [base, base + bytes).  Loads past
// the range return zero and stores past it are dropped, by the hardware range
// check, so both can be issued unconditionally.
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit dwords (gfx9 family)

// Base offset for a load that must be issued (to keep the memory counters
// exact) but whose data is not needed: every lane offset added to it stays in
// [2^31, 2^32), past any buffer range, so the hardware returns zeros without
// a memory access.
constexpr uint32_t kOob = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// Default cache policy.  Marking the streaming traffic non-temporal was
// measured slower on the target workload (58.4 us default, 64.3 us nt stores,
// 69.1 us nt loads): a 128 B row is read by two half-row instructions, and the
// second must still find the line in cache.
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

__device__ __forceinline__ uint2 bload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

__device__ __forceinline__ void bstore8(__amdgpu_buffer_rsrc_t r, uint32_t off, uint2 x) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, x), r, (int)off, 0, 0);
}

__device__ __forceinline__ void bstore16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 x) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, x), r, (int)off, 0, 0);
}

// ---------------------------------------------------------------- LDS transpose read
//
// gfx950's ds_read_b64_tr_b16 on row-major 16-bit rows: within each 16-lane
// group, lane i receives element i%4 of the 8-byte piece addressed by lane
// 4e + i/4, for e = 0..3 (checked on the device).  With lane l addressing
// row l>>2, a lane group reads 4 rows and each lane ends with one column of
// them: the MFMA operand layout of the transposed matrix.
__device__ __forceinline__ uint2 tr_read(const uint8_t* p) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)(p));
  return __builtin_bit_cast(uint2, r);
}

// ---------------------------------------------------------------- reductions
//
// Over the 4 lanes {l, l^16, l^32, l^48} (the lane groups that share one MFMA
// column) with the gfx950 row/half swaps: each swap returns a lane's own value
// and its partner's, so op(pair) is the xor-exchange result.
__device__ __forceinline__ float col_max(float x) {
  const i32x2 p = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  x = fmaxf(__int_as_float(p[0]), __int_as_float(p[1]));
  const i32x2 q = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float(q[0]), __int_as_float(q[1]));
}

__device__ __forceinline__ float col_sum(float x) {
  const i32x2 p = __builtin_amdgcn_permlane16_swap(__float_as_int(x), __float_as_int(x), false, false);
  x = __int_as_float(p[0]) + __int_as_float(p[1]);
  const i32x2 q = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float(q[0]) + __int_as_float(q[1]);
}

__device__ __forceinline__ int floordiv32(int a, int d) {
  const int q = a / d;
  return (a % d != 0 && a < 0) ? q - 1 : q;
}

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own
// L2.  This renumbering gives XCD x the contiguous run of ids [x*G/8,
// (x+1)*G/8) in order, so work items with neighbouring ids (a head's rows or
// tiles) share one L2.  Bijective: the first 8*(G/8) ids are permuted, the
// rest keep their number.
__device__ __forceinline__ int xcd_row_order(int bid, int G) {
  const int per = G >> 3;
  return bid < (per << 3) ? (bid & 7) * per + (bid >> 3) : bid;
}

}  // namespace ma_dev
