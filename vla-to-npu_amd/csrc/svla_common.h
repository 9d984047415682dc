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
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define SVLA_WAVE 64

__device__ __forceinline__ float bf2f(bf16 x) { return (float)x; }
__device__ __forceinline__ bf16 f2bf(float x) { return (bf16)x; }
// round an fp32 value through bf16 (models a bf16 tensor boundary in torch)
__device__ __forceinline__ float rbf(float x) { return (float)(bf16)x; }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, SVLA_WAVE);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, SVLA_WAVE));
  return v;
}

// 16-byte global load/store of 8 bf16 values.
__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ void st8(bf16* p, bf16x8 v) { *reinterpret_cast<bf16x8*>(p) = v; }

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }

// tanh-approximated GELU, computed as torch does for approximate='tanh':
// 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))).
__device__ __forceinline__ float gelu_tanh_f(float x) {
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  float inner = k0 * (x + k1 * x * x * x);
  return 0.5f * x * (1.0f + tanhf(inner));
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
