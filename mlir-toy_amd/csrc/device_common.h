// device_common.h — gfx950 building blocks shared by the HIP kernels:
// vector types for MFMA operands, 16-bit conversions, exp2, cross-lane
// helpers and the E4M3FN codec.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace neptune {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegFltMax = -3.40282347e+38f;  // HTile:23

// 16-bit storage types. Values move as raw uint16_t; the MFMA operand type
// is chosen by the Elem tag.
struct Bf16Tag {
  typedef bf16x8 vec8;
  __device__ static inline float to_f32(uint16_t h) {
    return __uint_as_float(uint32_t(h) << 16);
  }
  // round to nearest even (v_cvt_pk_bf16_f32)
  __device__ static inline uint16_t from_f32(float f) {
    __bf16 b = (__bf16)f;
    return __builtin_bit_cast(uint16_t, b);
  }
  // two values, round to nearest even, in one v_cvt_pk_bf16_f32
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
  }
  __device__ static inline f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

struct F16Tag {
  typedef f16x8 vec8;
  __device__ static inline float to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
  __device__ static inline uint16_t from_f32(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
  }
  // two values, round to nearest even, in one v_cvt_pk_f16_f32
  __device__ static inline uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, f16x2));
  }
  __device__ static inline f32x16 mfma32(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline f32x4 mfma16(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <class V>
__device__ inline V as_vec8(u32x4 u) {
  return __builtin_bit_cast(V, u);
}

// f(std::integral_constant<int, 0>{}) .. f(std::integral_constant<int, N - 1>{}),
// in order: a loop whose index is a constant expression in the body
template <class F, int... I>
__device__ inline void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ inline void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// v_exp_f32: 2^x, flushes denormal results; exp2(-inf) = 0.
__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// value of lane (l ^ 32)
__device__ inline float swap_halves(float x) {
  return __shfl_xor(x, 32, 64);
}

// max(x, x of lane l ^ 16) and max(x, x of lane l ^ 32), in registers: with
// both operands x, v_permlane16_swap exchanges rows 0 <-> 1 and 2 <-> 3 (16
// lanes each) and v_permlane32_swap the two 32-lane halves, so one of the
// two results is x and the other its partner, with no LDS round trip (what
// __shfl_xor's ds_bpermute costs)
__device__ inline float max_xor16(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float max_xor32(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// OCP E4M3FN -> f32 for two codes (hardware, exact): bytes 0,1 (HI=false)
// or bytes 2,3 (HI=true) of `packed`.
template <bool HI>
__device__ inline f32x2 e4m3x2_to_f32(uint32_t packed) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(packed, HI);
}

// OCP E4M3FN encode, round to nearest even, saturate to +-448. Integer
// restatement so the codes are bit-identical to the host codec.
__device__ inline uint8_t f32_to_e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return uint8_t(sign | 0x7fu);
  float af = __uint_as_float(a);
  if (af >= 448.0f) return uint8_t(sign | 0x7eu);
  if (af < 0.015625f) {
    // af * 512 is exact in fp32 (power-of-two scale of a value < 8)
    float scaled = af * 512.0f;
    float fl = floorf(scaled);
    float rem = scaled - fl;
    uint32_t m = uint32_t(fl);
    if (rem > 0.5f || (rem == 0.5f && (m & 1u))) m++;
    return uint8_t(sign | m);
  }
  int32_t e = int32_t(a >> 23) - 127;
  uint32_t mant = a & 0x7fffffu;
  uint32_t r = (uint32_t(e + 7) << 3) | (mant >> 20);
  uint32_t rem = mant & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) r++;
  if (r > 0x7eu) r = 0x7eu;
  return uint8_t(sign | r);
}

__device__ inline int64_t cdiv64(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace neptune
