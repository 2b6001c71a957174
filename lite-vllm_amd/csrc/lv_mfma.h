// MFMA operand types and the 32x32x16 bf16/fp16 matrix instruction used by
// the chunk-attention and linear kernels.
//
// v_mfma_f32_32x32x16_{bf16,f16} (wave64), operand layouts:
//   A[i][k] (32 x 16): lane i % 32 + 32 * (k / 8), element k % 8
//   B[k][j] (16 x 32): lane j % 32 + 32 * (k / 8), element k % 8
//   D[i][j] (32 x 32, fp32): lane j + 32 * ((i / 4) % 2), element 4 * (i / 8) + i % 4
// so a lane's A or B operand is 8 consecutive k of one row: one 16-byte load
// from a k-contiguous matrix.
#pragma once
#include "lv_common.h"

namespace lv {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

template <typename T> struct Mfma32;
template <> struct Mfma32<bf16> {
  using v8 = bf16x8_t;
  __device__ __forceinline__ static f32x16_t run(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // Two fp32 values -> packed pair, round to nearest even (v_cvt_pk_bf16_f32).
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
  }
};
template <> struct Mfma32<f16> {
  using v8 = f16x8_t;
  __device__ __forceinline__ static f32x16_t run(v8 a, v8 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    return (uint32_t)float_to_f16_bits(a) | ((uint32_t)float_to_f16_bits(b) << 16);
  }
};


// 16 bytes per lane from global memory straight into LDS at wave base + 16 lane.
__device__ __forceinline__ void load_lds16(const void* g, uint16_t* lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_wave_base, 16,
                                   0, 0);
}

}  // namespace lv
