// Shared helpers for the gfx950 kernels of libshard_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/shard_hip.h"

namespace shard {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));

// Records the text of a failed HIP call for shard_last_error().
void set_last_error(const char* what, hipError_t err);

#define SHARD_LAUNCH_CHECK(what)                       \
  do {                                                 \
    hipError_t _e = hipGetLastError();                 \
    if (_e != hipSuccess) {                            \
      ::shard::set_last_error(what, _e);               \
      return SHARD_ERR_HIP;                            \
    }                                                  \
  } while (0)

__device__ __forceinline__ float h2f(uint16_t bits) {
  return (float)__builtin_bit_cast(half_t, bits);
}

__device__ __forceinline__ uint16_t f2h(float x) {
  return __builtin_bit_cast(uint16_t, (half_t)x);  // round-to-nearest-even
}

__device__ __forceinline__ unsigned lane_id() { return threadIdx.x & 63u; }

// Order-preserving map of fp32 to uint32 (for atomicMin/Max on floats).
__device__ __forceinline__ uint32_t f2ord(float f) {
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float ord2f(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// x * s for s = +-1 as a sign-bit flip: exact, and keeps the sign of zero
// (-1 * +0 = -0), which a multiply lowered to fma(x, s, +0) would lose.
__device__ __forceinline__ float mul_sign(float x, float s) {
  return __uint_as_float(__float_as_uint(x) ^ (__float_as_uint(s) & 0x80000000u));
}

// fp16(x) of an fp32 value that must be rounded exactly once from this very
// register: the empty asm keeps the compiler from folding the producing
// multiply into a mixed-precision fma with a +0 addend (which turns -0 into +0).
__device__ __forceinline__ uint16_t f2h_opaque(float x) {
  asm volatile("" : "+v"(x));
  return f2h(x);
}

// IEEE fp32 ops with explicit rounding (no contraction into FMA).
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float sub_rn(float a, float b) { return __fsub_rn(a, b); }
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float div_rn(float a, float b) { return __fdiv_rn(a, b); }

inline int grid_cap(int64_t blocks, int cap = 65535 * 8) {
  return (int)(blocks < cap ? blocks : cap);
}

}  // namespace shard
