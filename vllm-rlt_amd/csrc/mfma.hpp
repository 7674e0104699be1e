// MFMA attention building blocks for gfx950 shared by the prefill and decode
// kernels: 32x32x16 bf16/fp16 MFMA operands, the transposing LDS read that
// feeds V^T, and the cross-half maximum of a wave.
#pragma once

#include "common.hpp"

namespace rlt {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(1))) void global_void;

// max(x[l], x[l ^ 32]) in every lane: v_permlane32_swap exchanges one
// register's upper 32 lanes with another's lower 32, so two copies of x end
// up holding the two halves' values in swapped order, whichever way round.
// The waits cover the VALU->permlane and permlane->VALU hazards, which the
// compiler does not see inside assembly.
__device__ __forceinline__ float max_across_halves(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return fmaxf(a, b);
}

template <typename T> struct MfmaOps;
template <> struct MfmaOps<bf16> {
  using V8 = bf16x8;
  __device__ static f32x16 mma(V8 a, V8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0); }
  __device__ static uint32_t pack2(float x, float y) {
    const bf16x2 r = {static_cast<__bf16>(x), static_cast<__bf16>(y)};  // v_cvt_pk_bf16_f32, RNE
    return __builtin_bit_cast(uint32_t, r);
  }
  // acc + lo + hi of a packed pair, exactly the rounded values the MFMA reads
  // (v_dot2c_f32_bf16 against ones).
  __device__ static float sum2(uint32_t pair, float acc) {
    const bf16x2 one = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), one, acc, false);
  }
};
template <> struct MfmaOps<f16> {
  using V8 = f16x8;
  __device__ static f32x16 mma(V8 a, V8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }
  __device__ static uint32_t pack2(float x, float y) {
    const f16x2 r = {static_cast<_Float16>(x), static_cast<_Float16>(y)};
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ static float sum2(uint32_t pair, float acc) {
    const f16x2 one = {static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), one, acc, false);
  }
};

template <typename V8>
__device__ __forceinline__ V8 as_v8(u32x4 x) {
  return __builtin_bit_cast(V8, x);
}

// Transposing LDS read (ds_read_b64_tr_b16).  In each 16-lane group, lane L
// supplies the address of 4 consecutive 16-bit elements; lane j receives
// element j%4 of the chunks supplied by lanes j/4, j/4+4, j/4+8, j/4+12.  With
// lane L addressing row L/4, column 4(L%4) of a row-major tile, lane j gets
// rows 0..3 of column j -- four consecutive keys of one V column.
__device__ __forceinline__ u32x2 lds_read_tr(const uint16_t* p) {
  const i16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(u32x2, x);
}

}  // namespace rlt
