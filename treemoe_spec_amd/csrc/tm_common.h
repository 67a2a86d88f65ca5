// Shared device helpers for the gfx950 kernels of libtreemoe_amd.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/treemoe_amd.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

#define TM_HIP_CHECK_LAUNCH()                                   \
  do {                                                          \
    hipError_t err__ = hipGetLastError();                       \
    if (err__ != hipSuccess) return TM_ERR_HIP_BASE + (int)err__; \
  } while (0)

__device__ __forceinline__ float tm_bf16_to_f32(uint16_t u) {
  return __uint_as_float(((uint32_t)u) << 16);
}

// fp32 -> bf16 with round-to-nearest-even; NaN maps to a quiet NaN.  Same
// rounding as torch's float->bfloat16 conversion.
__device__ __forceinline__ uint16_t tm_f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float tm_f16_to_f32(uint16_t u) {
  return (float)__builtin_bit_cast(_Float16, u);
}

// fp32 -> fp16, round to nearest even (the hardware conversion: subnormals
// kept, overflow to infinity, NaN stays NaN), as torch's float->half.
__device__ __forceinline__ uint16_t tm_f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// 16-bit element type of op1's activations and weights: TM_DTYPE_BF16 or
// TM_DTYPE_F16.  to_f32 widens one element exactly; round narrows an fp32
// value to the type with round-to-nearest-even.
template <int DT>
struct Half16 {
  static __device__ __forceinline__ float to_f32(uint16_t u) {
    return DT == TM_DTYPE_F16 ? tm_f16_to_f32(u) : tm_bf16_to_f32(u);
  }
  static __device__ __forceinline__ uint16_t round(float f) {
    return DT == TM_DTYPE_F16 ? tm_f32_to_f16(f) : tm_f32_to_bf16(f);
  }
};

// Store at device scope (relaxed; 2, 4 or 8 bytes): written through this
// XCD's L2 rather than left dirty in it.  For data a later kernel reads, this
// spares the end-of-kernel release, which has to write every dirty L2 line
// back before the next kernel starts (the 8 XCD L2s are not coherent with
// each other).
template <typename T>
__device__ __forceinline__ void tm_store_through(T* ptr, T v) {
  static_assert(sizeof(T) == 2 || sizeof(T) == 4 || sizeof(T) == 8, "2, 4 or 8 bytes");
  if constexpr (sizeof(T) == 2) {
    __hip_atomic_store(reinterpret_cast<uint16_t*>(ptr), __builtin_bit_cast(uint16_t, v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else if constexpr (sizeof(T) == 4) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>(ptr), __builtin_bit_cast(uint32_t, v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(ptr), __builtin_bit_cast(uint64_t, v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Wait for this wave's LDS operations, then a plain workgroup barrier.  Unlike
// __syncthreads() this does not drain outstanding global loads, so weight
// prefetches stay in flight across the barrier.
__device__ __forceinline__ void tm_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// e^x for x <= 0 (softmax arguments), IEEE single precision, evaluated with a
// fixed sequence of correctly rounded operations so that a host restatement
// reproduces it bit for bit.  Method: Cody & Waite argument reduction
// x = k*ln2 + r with ln2 split into a 16-bit head and a tail, degree-7 Taylor
// polynomial of e^r on |r| <= ln2/2 (truncation error < 2^-27 relative), and
// an exact scale by 2^k.  Arguments below -80 return 0 (e^-80 ~ 1.8e-35), which
// keeps every intermediate and the result away from subnormals.
__device__ __forceinline__ float tm_expf_det(float x) {
  if (!(x > -80.0f)) return 0.0f;
  if (x > 0.0f) x = 0.0f;
  const float kf = rintf(x * 1.44269504088896341f);
  float r = fmaf(kf, -0.693145751953125f, x);
  r = fmaf(kf, -1.42860676533018704e-06f, r);
  float p = 1.98412698412698413e-04f;
  p = fmaf(p, r, 1.38888888888888889e-03f);
  p = fmaf(p, r, 8.33333333333333333e-03f);
  p = fmaf(p, r, 4.16666666666666667e-02f);
  p = fmaf(p, r, 1.66666666666666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int k = (int)kf;
  return p * __int_as_float((k + 127) << 23);
}
