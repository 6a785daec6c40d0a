// Shared device helpers for the gfx950 kernels: vector types, the MFMA
// wrapper, and the thread-local error channel of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gpa_mi355x.h"

namespace gpa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// D = A(32x16) * B(16x32) + C, bf16 operands, fp32 accumulate.
// Operand layout (wave64): lane l supplies A[l%32][8*(l/32) .. +8] and
// B[8*(l/32) .. +8][l%32].  Result: lane l holds column l%32, register r
// holds row 8*(r/4) + 4*(l/32) + (r%4).
__device__ __forceinline__ f32x16 mfma32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row of the 32x32 MFMA result held by register r of a lane in half `hi`.
__device__ __forceinline__ constexpr int mfma_row(int r, int hi) {
  return 8 * (r >> 2) + 4 * hi + (r & 3);
}

// D = A(16x32) * B(32x16) + C, bf16 operands, fp32 accumulate.
// Operand layout (wave64): lane l supplies A[l%16][8*(l/16) .. +8] and
// B[8*(l/16) .. +8][l%16].  Result: lane l holds column l%16, register r
// holds row 4*(l/16) + r.
__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 16 independent 4x4x4 blocks, bf16 operands, fp32 accumulate.  With an
// all-ones A operand every lane receives the sum of its own four B values
// (in all four result registers).
__device__ __forceinline__ f32x4 mfma4x4x4(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0);
}

// The same three MFMA shapes on 16-bit operands of either format: the
// operands travel as bf16x8 / bf16x4 bit patterns, and F16 selects the fp16
// instruction (identical operand and result layouts).
template <bool F16>
__device__ __forceinline__ f32x16 mfma32x32x16_t(bf16x8 a, bf16x8 b, f32x16 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <bool F16>
__device__ __forceinline__ f32x4 mfma16x16x32_t(bf16x8 a, bf16x8 b, f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
template <bool F16>
__device__ __forceinline__ f32x4 mfma4x4x4_t(bf16x4 a, bf16x4 b, f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4, a),
                                              __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(a, b, c, 0, 0, 0);
}

// A 16-bit element of either format to fp32, and fp32 to its bit pattern
// (round to nearest even).
template <bool F16>
__device__ __forceinline__ float half_to_f32(__bf16 x) {
  if constexpr (F16)
    return (float)__builtin_bit_cast(_Float16, x);
  else
    return (float)x;
}
template <bool F16>
__device__ __forceinline__ __bf16 f32_to_half(float x) {
  if constexpr (F16)
    return __builtin_bit_cast(__bf16, (_Float16)x);
  else
    return (__bf16)x;
}

// Two fp32 values to a packed pair of 16-bit values (round to nearest even),
// one v_cvt_pk_{bf16,f16}_f32.  (Element-wise fp16 casts through bit casts
// defeat the pairing; the vector conversion does not.)
template <bool F16>
__device__ __forceinline__ bf16x2 pack2(float a, float b) {
  if constexpr (F16) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(bf16x2, __builtin_convertvector(f32x2{a, b}, f16x2));
  } else {
    return bf16x2{(__bf16)a, (__bf16)b};
  }
}

// Raw buffer resource over `bytes` bytes at `base`.  Loads through it are
// range-checked by the hardware: an access at or past `bytes` returns zeros,
// so tile prefetches need neither branches nor index clamps.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// Loads at byte offset voff + soff: voff per lane, soff wave-uniform (SGPR),
// so a per-tile advance costs no vector ALU work.
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                            uint32_t soff = 0) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

__device__ __forceinline__ u32x2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                           uint32_t soff = 0) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
}

// v_permlane32_swap on one value: lanes l and l^32 exchange.  The builtin
// returns {lanes 0-31 of x in both halves, lanes 32-63 of x in both halves},
// so combining the pair with a symmetric op yields (x[l] op x[l^32]) in
// every lane, with no LDS round trip.
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace gpa

// Error channel (defined in abi.hip).
void gpa_set_error(const char* fmt, ...);
void gpa_clear_error();
