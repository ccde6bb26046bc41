// Shared helpers for the gfx950 kernels of libshard_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/shard_hip.h"

namespace shard {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));

// Records the text of a failed HIP call for shard_last_error().
void set_last_error(const char* what, hipError_t err);
// Records a plain message (a failed check that is not a HIP call).
void set_last_text(const char* text);

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
// a / b correctly rounded from y = div_rn(1, b) (Markstein's theorem: with y
// within half an ulp of 1/b and q within one ulp of a/b, the exact residual
// r = a - b q and RN(q + r y) give RN(a / b)), for quotients in the normal
// range: three full-rate operations instead of the division sequence.  The
// residual is formed as -(b q - a) so that a zero a keeps its sign.
__device__ __forceinline__ float div_by_rcp(float a, float b, float y) {
  const float q = a * y;
  const float r = -__builtin_fmaf(b, q, -a);
  return __builtin_fmaf(r, y, q);
}

// ---- cross-lane exchange without the LDS crossbar.
// DPP moves inside rows of 16 lanes; v_permlane16_swap / v_permlane32_swap
// (gfx950) across rows and halves.  A ds_bpermute costs an LDS round trip
// (~100+ cycles) per step of a reduction chain; these are VALU operations.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- 7 - i inside groups of 8
constexpr int kDppMirror = 0x140;      // lane i <- 15 - i inside rows of 16
constexpr int kDppRor4 = 0x124;        // row rotate right by 4
constexpr int kDppRor8 = 0x128;        // row rotate right by 8
constexpr int kDppRor12 = 0x12C;       // row rotate right by 12

// (value of row r^1, value of half h^1) pairs: returns both swap results; for
// a commutative reduction their combination is the same on every lane.
__device__ __forceinline__ void perm16_swap(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void perm32_swap(float v, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// Reductions whose result every lane of the group holds: over each row of 16,
// each half (32 lanes) and the whole wave.
template <class Op>
__device__ __forceinline__ float row16_reduce(float v, Op op) {
  v = op(v, dpp_mov<kDppXor1>(v));
  v = op(v, dpp_mov<kDppXor2>(v));
  v = op(v, dpp_mov<kDppHalfMirror>(v));
  return op(v, dpp_mov<kDppMirror>(v));
}
template <class Op>
__device__ __forceinline__ float half32_reduce(float v, Op op) {
  v = row16_reduce(v, op);
  float a, b;
  perm16_swap(v, a, b);
  return op(a, b);
}
template <class Op>
__device__ __forceinline__ float wave64_reduce(float v, Op op) {
  v = half32_reduce(v, op);
  float a, b;
  perm32_swap(v, a, b);
  return op(a, b);
}
struct OpMax { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct OpAdd { __device__ float operator()(float a, float b) const { return a + b; } };

// The value of lane (l ^ HL), HL a power of two below 64.
template <int HL>
__device__ __forceinline__ float xor_lane(float v) {
  const int l = (int)(threadIdx.x & 63u);
  if constexpr (HL == 1) {
    return dpp_mov<kDppXor1>(v);
  } else if constexpr (HL == 2) {
    return dpp_mov<kDppXor2>(v);
  } else if constexpr (HL == 4) {
    // rotate right by 4 brings lane i-4, by 12 brings lane i+4 (mod 16)
    const float lo = dpp_mov<kDppRor4>(v), hi = dpp_mov<kDppRor12>(v);
    return (l & 4) ? lo : hi;
  } else if constexpr (HL == 8) {
    return dpp_mov<kDppRor8>(v);
  } else if constexpr (HL == 16) {
    float a, b;
    perm16_swap(v, a, b);  // a: rows (0,0,2,2), b: rows (1,1,3,3)
    return (l & 16) ? a : b;
  } else {
    static_assert(HL == 32, "xor_lane: HL must be a power of two below 64");
    float a, b;
    perm32_swap(v, a, b);  // a: halves (0,0), b: halves (1,1)
    return (l & 32) ? a : b;
  }
}

// ---- fast Walsh-Hadamard transform of one row held by a wave.
// One butterfly stage across lanes l and l ^ H (element stride H): the lower
// lane of a pair gets x + p, the upper p - x.  Both are fma(s, ., .) with
// s = +-1: s * x is exact, so the fma rounds once, exactly as the add or
// subtract (signs of zeros included), and no select is needed.
template <int H, int E>
__device__ __forceinline__ void fwht_lane_stage(float (&x)[E], int l) {
  const float s = (l & H) ? -1.f : 1.f;
#pragma unroll
  for (int k = 0; k < E; ++k) {
    if constexpr (H == 16 || H == 32) {
      float a, b;  // the pair's lower-lane and upper-lane values, in both lanes
      if constexpr (H == 16) perm16_swap(x[k], a, b);
      else perm32_swap(x[k], a, b);
      x[k] = __builtin_fmaf(s, b, a);
    } else {
      x[k] = __builtin_fmaf(s, x[k], xor_lane<H>(x[k]));
    }
  }
}

template <int E>
__device__ __forceinline__ void wave_fwht(float (&x)[E], int d) {
  // d == 64 * E: element i = lane + 64 k; strides 1..32 cross lanes, 64.. cross registers
  const int l = (int)lane_id();
  fwht_lane_stage<1>(x, l);
  fwht_lane_stage<2>(x, l);
  fwht_lane_stage<4>(x, l);
  fwht_lane_stage<8>(x, l);
  fwht_lane_stage<16>(x, l);
  fwht_lane_stage<32>(x, l);
#pragma unroll
  for (int hk = 1; hk < E; hk <<= 1) {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      if ((k & hk) == 0) {
        const float a = x[k], b = x[k | hk];
        x[k] = add_rn(a, b);
        x[k | hk] = sub_rn(a, b);
      }
    }
  }
  // torch divides an fp32 tensor by the Python float sqrt(d): fp32(double sqrt)
  const float s = (float)sqrt((double)d);
#pragma unroll
  for (int k = 0; k < E; ++k) x[k] = div_rn(x[k], s);
}

// The same transform with a contiguous layout: lane l holds elements
// E l .. E l + E - 1 (so a row loads and stores as E-element vectors).  Stages
// still run in increasing stride h and pair the same elements: strides h < E
// inside the lane, then strides h >= E across lanes l and l ^ (h / E).
template <int E, bool SCALE = true>
__device__ __forceinline__ void wave_fwht_contig(float (&x)[E], int d) {
  const int l = (int)lane_id();
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int j = 0; j < E; ++j) {
      if ((j & h) == 0) {
        const float a = x[j], b = x[j | h];
        x[j] = add_rn(a, b);
        x[j | h] = sub_rn(a, b);
      }
    }
  }
  fwht_lane_stage<1>(x, l);
  fwht_lane_stage<2>(x, l);
  fwht_lane_stage<4>(x, l);
  fwht_lane_stage<8>(x, l);
  fwht_lane_stage<16>(x, l);
  fwht_lane_stage<32>(x, l);
  if constexpr (SCALE) {  // SCALE = false leaves the final division to the caller
    const float s = (float)sqrt((double)d);
#pragma unroll
    for (int k = 0; k < E; ++k) x[k] = div_rn(x[k], s);
  }
}

inline int grid_cap(int64_t blocks, int cap = 65535 * 8) {
  return (int)(blocks < cap ? blocks : cap);
}

}  // namespace shard
