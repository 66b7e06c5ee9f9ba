// mfma_ops.h -- gfx950 MFMA operand helpers shared by the small-M GEMM and
// the expert-grouped MoE: exact fp8 e4m3 -> 16-bit operand decode and the
// 16x16x32 bf16 / f16 MFMA with f32 accumulation.
#pragma once
#include "dev_common.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

enum { GW_F16 = 0, GW_BF16 = 1, GW_FP8 = 2 };   // weight storage
enum { GX_BF16 = 0, GX_F16 = 1 };               // x storage = MFMA operand type

// four e4m3 bytes -> four 16-bit operand values (two u32), exact
template <int XT>
__device__ __forceinline__ void fp8x4_op(uint32_t w, uint32_t &lo, uint32_t &hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  if (XT == GX_BF16) {
    // straight to packed bf16, two values per v_cvt_scalef32_pk_bf16_fp8
    // (scale 1): an e4m3 value has <= 4 significant bits and its exponent
    // range fits bf16's, so the conversion is exact
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
    hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
  } else {               // via f32; exact in fp16 too (normal range 2^-14..2^15)
    f2_t a = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
    f2_t b = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a[0], a[1]));
    hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(b[0], b[1]));
  }
}

template <int XT>
__device__ __forceinline__ f32x4_t mfma16(const uint4 &A, const uint4 &B, f32x4_t c) {
  if (XT == GX_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, A),
                                                   __builtin_bit_cast(bf16x8_t, B), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, A),
                                                __builtin_bit_cast(f16x8_t, B), c, 0, 0, 0);
}

// two f32 -> a packed fp16 pair, round to nearest even; element 0 in the low half
__device__ __forceinline__ uint32_t pk_f16(float a, float b) {
  return (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
}

// v_mfma_f32_16x16x16_{bf16,f16}: A and B as two u32 each (4 16-bit values,
// element 0 in the low half of the first); lane l holds A[m = l%16][k = 4
// (l/16) + j] and B[k = 4 (l/16) + j][n = l%16], and gets D[4 (l/16) + i][l%16]
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
template <int XT>
__device__ __forceinline__ f32x4_t mfma16x16(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4_t c) {
  typedef uint32_t u2_t __attribute__((ext_vector_type(2)));
  const u2_t A = {a0, a1}, B = {b0, b1};
  if (XT == GX_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, A),
                                                     __builtin_bit_cast(s16x4_t, B), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, A), __builtin_bit_cast(f16x4_t, B),
                                               c, 0, 0, 0);
}
