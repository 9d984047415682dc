// Shared device helpers for the SmolVLA gfx950 kernels.
//
// Storage type for activations and weights is IEEE bfloat16 (`__bf16`);
// arithmetic is fp32.  float -> bf16 uses the hardware round-to-nearest-even
// conversion (v_cvt_pk_bf16_f32 on gfx950), which is the rounding torch uses
// for `.to(torch.bfloat16)`, so every kernel's rounding points can mirror the
// reference torch modules one for one.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/svla.h"

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// LDS pointer type for __builtin_amdgcn_global_load_lds destinations
typedef __attribute__((address_space(3))) void* lds_ptr_t;

#define SVLA_WAVE 64

__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }
__device__ __forceinline__ bf16 f2bf(float x) { return (bf16)x; }
// round an fp32 value through bf16 (models a bf16 tensor boundary in torch)
__device__ __forceinline__ float rbf(float x) { return (float)(bf16)x; }

// A value combined with the one of lane l ^ 16 (l ^ 32) of the wave:
// v_permlane16_swap / v_permlane32_swap with both operands the value return
// it and its partner in the two results (a VALU exchange, where a shuffle
// would be an LDS permute).  Sums and maxima are commutative, so the result
// equals v + partner bit for bit.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = xor16_sum(xor32_sum(v));
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v += __shfl_xor(v, o, SVLA_WAVE);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  v = xor16_max(xor32_max(v));
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, SVLA_WAVE));
  return v;
}

// 16-byte global load/store of 8 bf16 values.
__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ void st8(bf16* p, bf16x8 v) { *reinterpret_cast<bf16x8*>(p) = v; }

// x * sigmoid(x) as x / (1 + 2^(-x log2 e)) with the hardware exp2 and
// reciprocal (1 ulp each): the result is rounded to bf16 by every caller, so
// the IEEE division's extra accuracy is invisible.  exp2 -> inf for very
// negative x gives x * 0 = -0, the correctly rounded limit.
__device__ __forceinline__ float fast_sigmoid_scaled(float z_log2e) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-z_log2e));
}
__device__ __forceinline__ float silu_f(float x) {
  return x * fast_sigmoid_scaled(x * 1.4426950408889634f);
}

// tanh-approximated GELU (torch approximate='tanh'):
//   0.5 x (1 + tanh(u)),  u = sqrt(2/pi) (x + 0.044715 x^3)
// evaluated through the identity 0.5 (1 + tanh(u)) = sigmoid(2u), i.e.
//   x / (1 + exp(-2u)),
// which needs one exp2 and one reciprocal instead of a tanh (the tanh form
// also loses all relative accuracy for x < -3 where 1 + tanh(u) cancels).
__device__ __forceinline__ float gelu_tanh_f(float x) {
  // 2 * sqrt(2/pi) * log2(e) and 2 * sqrt(2/pi) * 0.044715 * log2(e)
  const float c0 = 2.3022082f, c1 = 0.10294324f;
  // -z with the sign folded into the constants (exact)
  const float nz = x * __builtin_fmaf(-c1, x * x, -c0);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(nz));
}

// exact-erf GELU (the reference's nn.GELU() default)
__device__ __forceinline__ float gelu_erf_f(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f));
}

#define SVLA_CHECK_LAUNCH()                        \
  do {                                             \
    hipError_t e__ = hipGetLastError();            \
    if (e__ != hipSuccess) return (int)e__;        \
  } while (0)

static inline bool svla_aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
