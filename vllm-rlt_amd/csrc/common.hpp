// Shared device helpers for the rlt_kv gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rlt_kv.h"

namespace rlt {

// ---------------------------------------------------------------------------
// Host-side status reporting (status.hip).
int fail(int code, const char* fmt, ...);
int check_launch(const char* kernel);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int dtype_size(int dtype) {
  switch (dtype) {
    case RLT_FLOAT32: return 4;
    case RLT_FLOAT16: return 2;
    case RLT_BFLOAT16: return 2;
    default: return 0;
  }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Storage element types.  bf16 travels as raw 16-bit words; fp16 uses the
// native _Float16 conversions (v_cvt_f32_f16 / v_cvt_f16_f32, round to
// nearest even).
struct bf16 {
  uint16_t bits;
};
using f16 = _Float16;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 with round-to-nearest-even; NaN becomes the canonical quiet
// NaN 0x7FC0, the same bits torch's float->bfloat16 cast produces.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ uint32_t f16_bits(float f) {
  f16 h = static_cast<f16>(f);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
}

// Number of elements in a 16-byte packet.
template <typename T> struct Packet;
template <> struct Packet<bf16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const u32x4& p, float* x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = bf16_lo(p[i]);
      x[2 * i + 1] = bf16_hi(p[i]);
    }
  }
  __device__ __forceinline__ static u32x4 pack(const float* x) {
    u32x4 p;
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = f32_to_bf16_bits(x[2 * i]) | (f32_to_bf16_bits(x[2 * i + 1]) << 16);
    return p;
  }
};
template <> struct Packet<f16> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void unpack(const u32x4& p, float* x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(p[i] & 0xffffu)));
      x[2 * i + 1] = static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(p[i] >> 16)));
    }
  }
  __device__ __forceinline__ static u32x4 pack(const float* x) {
    u32x4 p;
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = f16_bits(x[2 * i]) | (f16_bits(x[2 * i + 1]) << 16);
    return p;
  }
};
template <> struct Packet<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void unpack(const u32x4& p, float* x) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(p[i]);
  }
  __device__ __forceinline__ static u32x4 pack(const float* x) {
    u32x4 p;
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __float_as_uint(x[i]);
    return p;
  }
};

// Scalar element <-> fp32 (generic, strided paths).
__device__ __forceinline__ float load_elem(const bf16* p) { return __uint_as_float(static_cast<uint32_t>(p->bits) << 16); }
__device__ __forceinline__ float load_elem(const f16* p) { return static_cast<float>(*p); }
__device__ __forceinline__ float load_elem(const float* p) { return *p; }
__device__ __forceinline__ void store_elem(bf16* p, float x) { p->bits = static_cast<uint16_t>(f32_to_bf16_bits(x)); }
__device__ __forceinline__ void store_elem(f16* p, float x) { *p = static_cast<f16>(x); }
__device__ __forceinline__ void store_elem(float* p, float x) { *p = x; }

// ---------------------------------------------------------------------------
// Lane exchange.  Every reduction below is a butterfly over an involution of
// the lanes (lane l meets partner p(l), p(p(l)) == l), so a lane and its
// partner add the same two operands and -- fp32 addition being commutative --
// every lane of a group ends with bit-identical sums.  Within a 16-lane DPP
// row the involutions are quad_perm [1,0,3,2] (xor 1), quad_perm [2,3,0,1]
// (xor 2), row_half_mirror (j <-> 7-j) and row_mirror (j <-> 15-j); after the
// first two steps every quad holds its quad sum, so the mirrors join quads
// 0+1, 2+3 and then halves.  Wider groups continue with xor 16 / xor 32.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // row_half_mirror
constexpr int kDppMirror = 0x140;     // row_mirror

__device__ __forceinline__ float xor_lane(float x, int mask) { return __shfl_xor(x, mask, 64); }

// Sum over aligned groups of W lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (W >= 2) x += dpp<kDppXor1>(x);
  if constexpr (W >= 4) x += dpp<kDppXor2>(x);
  if constexpr (W >= 8) x += dpp<kDppHalfMirror>(x);
  if constexpr (W >= 16) x += dpp<kDppMirror>(x);
  if constexpr (W >= 32) x += xor_lane(x, 16);
  if constexpr (W >= 64) x += xor_lane(x, 32);
  return x;
}

// Butterfly over the lanes that share (lane % STRIDE): partners at xor STRIDE,
// 2*STRIDE, ... < 64.  Used to join per-token-group partials.
template <int STRIDE>
__device__ __forceinline__ float strided_sum(float x) {
#pragma unroll
  for (int m = STRIDE; m < 64; m <<= 1) x += xor_lane(x, m);
  return x;
}
template <int STRIDE>
__device__ __forceinline__ float strided_max(float x) {
#pragma unroll
  for (int m = STRIDE; m < 64; m <<= 1) x = fmaxf(x, xor_lane(x, m));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uniform64(int64_t x) {
  uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
  uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

}  // namespace rlt
