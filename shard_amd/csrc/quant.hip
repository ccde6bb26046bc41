// Bit-exact integer chains of the compressed-KV path on gfx950:
//   * key coefficient group quantization -> dequantization -> int4 -> packing
//   * per-token 8-bit Lloyd-Max stream quantizer
//   * Walsh-Hadamard transform, VQ front half, nearest-centroid assignment,
//     deterministic k-means centroid update
// This file is compiled with -ffp-contract=off and uses explicitly rounded
// fp32 operations so every value follows the reference's per-op rounding.
#include <algorithm>
#include <cmath>

#include "common.h"

namespace shard {

// ---------------------------------------------------------------------------
// int4 chain (rope.py:95-161 values, cache.py:416-420, triton_kernels.py:648-682)
// ---------------------------------------------------------------------------

// Dequantized group value of one coefficient (quantize_group then
// dequantize_group): y = code/L*rng + lo, code = clamp(rint(clamp((x-lo)/rng,0,1)*L),0,L).
__device__ __forceinline__ int group_code(float x, int bits, float lo, float rng) {
  if (bits <= 0) return 0;
  const float L = (float)((1 << bits) - 1);
  float v = div_rn(sub_rn(x, lo), rng);
  v = fminf(fmaxf(v, 0.f), 1.f);
  v = mul_rn(v, L);
  const float code = rintf(v);  // round half to even, as torch.round
  return (int)fminf(fmaxf(code, 0.f), L);
}

__device__ __forceinline__ float group_deq(float x, int bits, float lo, float rng,
                                           uint8_t* code_out) {
  const int code = group_code(x, bits, lo, rng);
  *code_out = (uint8_t)code;
  if (bits <= 0) return 0.f;
  const float L = (float)((1 << bits) - 1);
  return add_rn(mul_rn(div_rn((float)code, L), rng), lo);
}

// The column reductions write one partial per (block, column) and a wave per
// column folds the partials: no global atomics (every block would otherwise
// hit the same keep addresses).  Column passes use blocks of (column, row
// group) threads; thread (c, g) takes rows r0 + g, r0 + g + RG, ...
constexpr int kI4Blocks = 256;  // partial slots per column

__device__ __forceinline__ uint32_t u32min(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t u32max(uint32_t a, uint32_t b) { return a < b ? b : a; }

// Column min/max (order-preserving keys) of one slab of rows.
__global__ __launch_bounds__(1024) void k_int4_minmax(const float* __restrict__ proj, int64_t n,
                                                      int keep, int64_t rows_per_block,
                                                      uint32_t* __restrict__ pmin,
                                                      uint32_t* __restrict__ pmax) {
  __shared__ float smn[1024], smx[1024];
  const int c = threadIdx.x, rg = threadIdx.y, RG = blockDim.y, w = blockDim.x;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < n ? r0 + rows_per_block : n;
  float mn = INFINITY, mx = -INFINITY;
  if (c < keep) {
    int64_t r = r0 + rg;
    for (; r + 3 * RG < r1; r += 4 * RG) {  // four rows in flight
      const float x0 = proj[r * keep + c], x1 = proj[(r + RG) * keep + c];
      const float x2 = proj[(r + 2 * RG) * keep + c], x3 = proj[(r + 3 * RG) * keep + c];
      mn = fminf(fminf(fminf(mn, x0), fminf(x1, x2)), x3);
      mx = fmaxf(fmaxf(fmaxf(mx, x0), fmaxf(x1, x2)), x3);
    }
    for (; r < r1; r += RG) {
      const float x = proj[r * keep + c];
      mn = fminf(mn, x);
      mx = fmaxf(mx, x);
    }
  }
  smn[rg * w + c] = mn;
  smx[rg * w + c] = mx;
  __syncthreads();
  if (rg == 0 && c < keep) {
    for (int q = 1; q < RG; ++q) {
      mn = fminf(mn, smn[q * w + c]);
      mx = fmaxf(mx, smx[q * w + c]);
    }
    pmin[(int64_t)blockIdx.x * keep + c] = f2ord(mn);
    pmax[(int64_t)blockIdx.x * keep + c] = f2ord(mx);
  }
}

// One wave per column: fold the block partials; lo = min, rng = max(max - lo, 1e-6).
__global__ void k_int4_fold_minmax(const uint32_t* __restrict__ pmin,
                                   const uint32_t* __restrict__ pmax, int nblk, int keep,
                                   float* __restrict__ lo, float* __restrict__ rng) {
  const int c = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6), l = (int)lane_id();
  if (c >= keep) return;  // whole waves
  uint32_t a = 0xFFFFFFFFu, b = 0u;
  for (int q = l; q < nblk; q += 64) {
    a = u32min(a, pmin[(int64_t)q * keep + c]);
    b = u32max(b, pmax[(int64_t)q * keep + c]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    a = u32min(a, __shfl_xor(a, o));
    b = u32max(b, __shfl_xor(b, o));
  }
  if (l == 0) {
    const float lv = ord2f(a);
    lo[c] = lv;
    rng[c] = fmaxf(sub_rn(ord2f(b), lv), 1e-6f);
  }
}

// One wave per column: the column's lo, rng, coefficient scale and int4
// table from its min and max alone.  The group code, and with it the
// dequantized value y, never decreases as x grows (every step of group_deq is
// a monotone rounding of a monotone function of x for rng > 0), so the
// column's largest |y| is |y| of its smallest or of its largest element, both
// computed here with the arithmetic the element pass uses: cs = max(max |y|,
// 1e-6) / 7 is the reference's (cache.py:417-418) without a pass over the
// elements (finite projections; a non-finite element breaks the order).
__global__ void k_int4_fold(const uint32_t* __restrict__ pmin, const uint32_t* __restrict__ pmax,
                            int nblk, int keep, const int32_t* __restrict__ bits,
                            float* __restrict__ clo, float* __restrict__ crng,
                            int8_t* __restrict__ qtab, float* coeff_scale, float* lo_out,
                            float* rng_out) {
  const int c = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6), l = (int)lane_id();
  if (c >= keep) return;  // whole waves
  uint32_t a = 0xFFFFFFFFu, bmax = 0u;
  for (int q = l; q < nblk; q += 64) {
    a = u32min(a, pmin[(int64_t)q * keep + c]);
    bmax = u32max(bmax, pmax[(int64_t)q * keep + c]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    a = u32min(a, __shfl_xor(a, o));
    bmax = u32max(bmax, __shfl_xor(bmax, o));
  }
  const float lv = ord2f(a), xmax = ord2f(bmax);
  const float rv = fmaxf(sub_rn(xmax, lv), 1e-6f);
  const int b = bits[c];
  uint8_t k0, k1;
  const float y0 = group_deq(lv, b, lv, rv, &k0), y1 = group_deq(xmax, b, lv, rv, &k1);
  const float cs = div_rn(fmaxf(fmaxf(fabsf(y0), fabsf(y1)), 1e-6f), 7.0f);
  for (int code = l; code < 256; code += 64) {
    float y = 0.f;  // columns without bits have y = 0 (code 0)
    if (b > 0 && code < (1 << b)) {
      const float L = (float)((1 << b) - 1);
      y = add_rn(mul_rn(div_rn((float)code, L), rv), lv);
    }
    qtab[c * 256 + code] = (int8_t)fminf(fmaxf(rintf(div_rn(y, cs)), -7.f), 7.f);
  }
  if (l == 0) {
    clo[c] = lv;
    crng[c] = rv;
    coeff_scale[c] = cs;
    if (lo_out) lo_out[c] = b > 0 ? lv : 0.f;
    if (rng_out) rng_out[c] = b > 0 ? rv : 0.f;
  }
}

// Group codes and packed int4 values of one slab of rows, straight from the
// projection (keep even: an element's nibble pair lies in its row).  Thread
// (c, g) takes column c of rows r0 + g, r0 + g + RG, ..., eight rows in
// flight; q = qtab[c][code] (k_int4_fold's table).  The waves hold 64
// consecutive columns of a row, so the nibbles of 8 columns meet in one lane
// by three DPP moves and go out as one 32-bit word (words: keep % 8 == 0 and
// a 4-byte aligned output; else each even column stores its byte).
template <bool WORDS, bool CODES>
__global__ __launch_bounds__(1024) void k_int4_pack_rows(const float* __restrict__ proj, int64_t n,
                                                         int keep, int64_t rows_per_block,
                                                         const int32_t* __restrict__ bits,
                                                         const float* __restrict__ clo,
                                                         const float* __restrict__ crng,
                                                         const int8_t* __restrict__ qtab,
                                                         uint8_t* __restrict__ codes,
                                                         uint8_t* __restrict__ packed) {
  const int c = threadIdx.x, rg = threadIdx.y, RG = blockDim.y;
  const int l = (int)lane_id();
  const bool col_ok = c < keep;
  const int cc = col_ok ? c : keep - 1;  // lanes past the last column read a valid column
  const int b = bits[cc];
  const float lv = clo[cc], rv = crng[cc];
  const int8_t* qt = qtab + cc * 256;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < n ? r0 + rows_per_block : n;
  const bool store = col_ok && (WORDS ? (l & 7) == 0 : (c & 1) == 0);
  const int64_t step = (int64_t)RG * keep;
  int64_t e = (r0 + rg) * keep + cc;  // element of this thread's next row
  auto emit = [&](float x) {  // all lanes of the wave (DPP moves)
    const int code = group_code(x, b, lv, rv);
    const uint32_t nib = col_ok ? (uint32_t)((qt[code] + 8) & 15) : 8u;
    if (CODES && col_ok) codes[e] = (uint8_t)code;
    // DPP moves within rows of 16 lanes: lane c takes lane c ^ 1, c ^ 2, c + 4
    uint32_t t = nib | ((uint32_t)__builtin_amdgcn_mov_dpp((int)nib, kDppXor1, 0xF, 0xF, false) << 4);
    if (WORDS) {
      t |= (uint32_t)__builtin_amdgcn_mov_dpp((int)t, kDppXor2, 0xF, 0xF, false) << 8;
      t |= (uint32_t)__builtin_amdgcn_mov_dpp((int)t, kDppRor12, 0xF, 0xF, false) << 16;
      if (store) *(uint32_t*)(packed + e / 2) = t;
    } else if (store) {
      packed[e / 2] = (uint8_t)t;  // even lanes: the byte of columns c, c + 1
    }
    e += step;
  };
  int64_t r = r0 + rg;
  for (; r + 7 * RG < r1; r += 8 * RG) {  // uniform per wave (one row group)
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = proj[e + i * step];
#pragma unroll
    for (int i = 0; i < 8; ++i) emit(x[i]);
  }
  for (; r < r1; r += RG) emit(proj[e]);
}

// Column max |y| of the dequantized values of one slab, and the group codes.
__global__ __launch_bounds__(1024) void k_int4_absmax(const float* __restrict__ proj, int64_t n,
                                                      int keep, int64_t rows_per_block,
                                                      const int32_t* __restrict__ bits,
                                                      const float* __restrict__ lo,
                                                      const float* __restrict__ rng,
                                                      uint32_t* __restrict__ pamax,
                                                      uint8_t* __restrict__ codes) {
  __shared__ float sam[1024];
  const int c = threadIdx.x, rg = threadIdx.y, RG = blockDim.y, w = blockDim.x;
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < n ? r0 + rows_per_block : n;
  float amax = 0.f;
  if (c < keep) {
    const int b = bits[c];
    const float l = lo[c], rn = rng[c];
    int64_t r = r0 + rg;
    for (; r + RG < r1; r += 2 * RG) {
      const float x0 = proj[r * keep + c], x1 = proj[(r + RG) * keep + c];
      uint8_t k0, k1;
      const float y0 = group_deq(x0, b, l, rn, &k0), y1 = group_deq(x1, b, l, rn, &k1);
      amax = fmaxf(amax, fmaxf(fabsf(y0), fabsf(y1)));
      codes[r * keep + c] = k0;
      codes[(r + RG) * keep + c] = k1;
    }
    for (; r < r1; r += RG) {
      uint8_t k0;
      const float y = group_deq(proj[r * keep + c], b, l, rn, &k0);
      amax = fmaxf(amax, fabsf(y));
      codes[r * keep + c] = k0;
    }
  }
  sam[rg * w + c] = amax;
  __syncthreads();
  if (rg == 0 && c < keep) {
    for (int q = 1; q < RG; ++q) amax = fmaxf(amax, sam[q * w + c]);
    pamax[(int64_t)blockIdx.x * keep + c] = __float_as_uint(amax);  // >= 0: bits order as values
  }
}

// One wave per column: cs = max(max |y|, 1e-6) / 7, the per-column outputs,
// and the column's int4 value of every group code (y and q depend on the
// element only through its code): qtab[c][code] = clamp(rint(y(code) / cs), -7, 7).
__global__ void k_int4_fold_absmax(const uint32_t* __restrict__ pamax, int nblk, int keep,
                                   const int32_t* __restrict__ bits, const float* __restrict__ lo,
                                   const float* __restrict__ rng, int8_t* __restrict__ qtab,
                                   float* coeff_scale, float* lo_out, float* rng_out) {
  const int c = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6), l = (int)lane_id();
  if (c >= keep) return;  // whole waves
  uint32_t a = 0u;
  for (int q = l; q < nblk; q += 64) a = u32max(a, pamax[(int64_t)q * keep + c]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) a = u32max(a, __shfl_xor(a, o));
  const float cs = div_rn(fmaxf(__uint_as_float(a), 1e-6f), 7.0f);
  const int b = bits[c];
  const float lv = lo[c], rv = rng[c];
  for (int code = l; code < 256; code += 64) {
    float y = 0.f;  // columns without bits have y = 0 (code 0)
    if (b > 0 && code < (1 << b)) {
      const float L = (float)((1 << b) - 1);
      y = add_rn(mul_rn(div_rn((float)code, L), rv), lv);
    }
    qtab[c * 256 + code] = (int8_t)fminf(fmaxf(rintf(div_rn(y, cs)), -7.f), 7.f);
  }
  if (l == 0) {
    coeff_scale[c] = cs;
    if (lo_out) lo_out[c] = b > 0 ? lv : 0.f;
    if (rng_out) rng_out[c] = b > 0 ? rv : 0.f;
  }
}

// Byte i packs elements 2i and 2i + 1 of the row-major matrix from their group
// codes; a thread takes 8 elements (4 bytes).  IT is 32-bit when the element
// count allows, so the column of an element is a 32-bit mod.
template <typename IT>
__global__ void k_int4_pack(const uint8_t* __restrict__ codes, IT total, int keep,
                            const int8_t* __restrict__ qtab, uint8_t* __restrict__ packed) {
  const IT nbytes = (total + 1) / 2;
  const IT nquads = (nbytes + 3) / 4;
  const IT stride = (IT)gridDim.x * blockDim.x;
  for (IT i = (IT)blockIdx.x * blockDim.x + threadIdx.x; i < nquads; i += stride) {
    const IT e0 = 8 * i;
    int c = (int)(e0 % (IT)keep);
    uint32_t word = 0;
    if (e0 + 8 <= total && ((uintptr_t)(codes + e0) & 7) == 0) {
      const uint2 cw = *(const uint2*)(codes + e0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint32_t code = ((j < 4 ? cw.x : cw.y) >> (8 * (j & 3))) & 255u;
        word |= (uint32_t)((qtab[c * 256 + code] + 8) & 15) << (4 * j);
        c = c + 1 == keep ? 0 : c + 1;
      }
    } else {
      for (int j = 0; j < 8; ++j) {
        // an odd count pairs the last element with a zero value (nibble 8), as
        // the reference appends a 0 before packing (triton_kernels.py:668-670)
        const int q = e0 + j < total ? qtab[c * 256 + codes[e0 + j]] : 0;
        word |= (uint32_t)((q + 8) & 15) << (4 * j);
        c = c + 1 == keep ? 0 : c + 1;
      }
    }
    if (4 * i + 4 <= nbytes && ((uintptr_t)(packed + 4 * i) & 3) == 0) {
      *(uint32_t*)(packed + 4 * i) = word;
    } else {
      for (int j = 0; 4 * i + j < nbytes; ++j) packed[4 * i + j] = (uint8_t)(word >> (8 * j));
    }
  }
}

// ---------------------------------------------------------------------------
// Walsh-Hadamard within a wave: lane l holds elements l + 64*k, k < E.
// Stage h pairs element e with e^h: lower index gets a+b, upper a-b
// (cache.py:14-18), stages in increasing h, then one IEEE division.
// ---------------------------------------------------------------------------
template <int E>
__global__ void k_fwht_rows(const float* __restrict__ x, float* __restrict__ y, int64_t rows) {
  const int d = 64 * E;
  const int l = (int)lane_id();
  int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t r = wave; r < rows; r += nwaves) {
    float v[E];
#pragma unroll
    for (int k = 0; k < E; ++k) v[k] = x[r * d + l + 64 * k];
    wave_fwht<E>(v, d);
#pragma unroll
    for (int k = 0; k < E; ++k) y[r * d + l + 64 * k] = v[k];
  }
}

// Small d (< 64): one thread per row, same butterflies.
__global__ void k_fwht_small(const float* __restrict__ x, float* __restrict__ y, int64_t rows,
                             int d) {
  int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float v[32];
  for (int i = 0; i < d; ++i) v[i] = x[r * d + i];
  for (int h = 1; h < d; h <<= 1)
    for (int i = 0; i < d; ++i)
      if ((i & h) == 0) {
        float a = v[i], b = v[i + h];
        v[i] = add_rn(a, b);
        v[i + h] = sub_rn(a, b);
      }
  const float s = (float)sqrt((double)d);
  for (int i = 0; i < d; ++i) y[r * d + i] = div_rn(v[i], s);
}

// ---------------------------------------------------------------------------
// VQ front half: hadamard(fp32(v)) -> channel abs max -> normalized subvectors
// ---------------------------------------------------------------------------
// Workgroup (x, b) rotates rows [x R, (x + 1) R) of head b (R = ceil(seq /
// gridDim.x), at most kVqSlots workgroups per head).  Two passes over V:
//   NORM = false: FWHT only, writing the workgroup's channel maxima of |x|
//                 as one partial (a fold kernel takes the max over partials);
//   NORM = true:  FWHT again (the same values) divided by the folded channel
//                 scale, stored as x.
// Recomputing the FWHT moves less data than storing x and normalizing it in
// place (2 B read per element instead of 4 B written + 4 B read + 4 B written).
constexpr int kVqSlots = 64;

template <int E, bool NORM>
__global__ __launch_bounds__(256) void k_vq_rot(const uint16_t* __restrict__ v, int64_t bh,
                                                int64_t seq, int64_t bh_stride,
                                                float* __restrict__ part,
                                                const float* __restrict__ ch,
                                                float* __restrict__ xo) {
  constexpr int d = 64 * E;
  constexpr int RS = 4;  // rows per step: all their loads are issued before any FWHT
  __shared__ float red[4][d];
  const int l = (int)lane_id();
  const int w = (int)(threadIdx.x >> 6);
  const int64_t R = (seq + gridDim.x - 1) / gridDim.x;
  const int64_t per_wave = (R + 3) / 4;
  for (int64_t b = blockIdx.y; b < bh; b += gridDim.y) {
    const int64_t t_blk = (int64_t)blockIdx.x * R;
    const int64_t t_blk_end = t_blk + R < seq ? t_blk + R : seq;
    const int64_t t0 = t_blk + w * per_wave;
    const int64_t t1 = t0 + per_wave < t_blk_end ? t0 + per_wave : t_blk_end;
    const uint16_t* src = v + b * bh_stride;
    float* dst = xo + b * seq * d;
    // lane l holds channels E l .. E l + E - 1 (contiguous-layout FWHT)
    // pass 2 divides by sqrt(d), then by the channel scale, each division
    // through its divisor's correctly rounded reciprocal (div_by_rcp: the
    // quotients of finite fp16 rows are normal, |FWHT| being >= 2^-24 or 0
    // and the scales in [1e-8, 1e6]).  A head with an infinite value (so an
    // infinite channel scale) divides with div_rn throughout.
    float m[E], cs[E], rcs[E];
    const float sd = (float)sqrt((double)d), rsd = div_rn(1.f, sd);
    bool finite = true;
#pragma unroll
    for (int k = 0; k < E; ++k) {
      m[k] = 0.f;
      if constexpr (NORM) {
        cs[k] = ch[b * d + E * l + k];
        rcs[k] = div_rn(1.f, cs[k]);
        finite = finite && fabsf(cs[k]) <= 0x1.fffffep127f;
      }
    }
    const bool by_rcp = __ballot(!finite) == 0;  // wave-uniform
    // raw rows (E halves per lane) of a step; the next step's loads are issued
    // before this step's transforms
    auto load_rows = [&](int64_t tt, uint32_t (&u)[RS][(E + 1) / 2]) {
#pragma unroll
      for (int q = 0; q < RS; ++q) {
        const uint16_t* p = src + (tt + q) * d + E * l;
        if constexpr (E == 1) {
          u[q][0] = tt + q < t1 ? p[0] : 0u;
        } else if constexpr (E == 2) {
          u[q][0] = tt + q < t1 ? *(const uint32_t*)p : 0u;
        } else {
          const uint2 v2 = tt + q < t1 ? *(const uint2*)p : make_uint2(0u, 0u);
          u[q][0] = v2.x;
          u[q][1] = v2.y;
        }
      }
    };
    uint32_t un[RS][(E + 1) / 2];
    if (t0 < t1) load_rows(t0, un);
    for (int64_t t = t0; t < t1; t += RS) {
      float x[RS][E];
#pragma unroll
      for (int q = 0; q < RS; ++q)
#pragma unroll
        for (int k = 0; k < E; ++k) x[q][k] = h2f((uint16_t)(un[q][k >> 1] >> (16 * (k & 1))));
      if (t + RS < t1) load_rows(t + RS, un);
#pragma unroll
      for (int q = 0; q < RS; ++q) {
        if (t + q >= t1) break;  // wave-uniform
        // the statistics pass keeps max |y| of the unscaled transform: dividing
        // by sqrt(d) rounds monotonically, so max |RN(y / s)| = RN(max |y| / s)
        wave_fwht_contig<E, false>(x[q], d);
        if constexpr (NORM) {
          float y[E];
          if (by_rcp) {
#pragma unroll
            for (int k = 0; k < E; ++k)
              y[k] = div_by_rcp(div_by_rcp(x[q][k], sd, rsd), cs[k], rcs[k]);
          } else {
#pragma unroll
            for (int k = 0; k < E; ++k) y[k] = div_rn(div_rn(x[q][k], sd), cs[k]);
          }
          float* o = dst + (t + q) * d + E * l;
          if constexpr (E == 1) {
            o[0] = y[0];
          } else if constexpr (E == 2) {
            *(float2*)o = make_float2(y[0], y[1]);
          } else {
            *(float4*)o = make_float4(y[0], y[1], y[2], y[3]);
          }
        } else {
#pragma unroll
          for (int k = 0; k < E; ++k) m[k] = fmaxf(m[k], fabsf(x[q][k]));
        }
      }
    }
    if constexpr (!NORM) {
      __syncthreads();  // red is reused across heads
#pragma unroll
      for (int k = 0; k < E; ++k) red[w][E * l + k] = m[k];
      __syncthreads();
      const float sd = (float)sqrt((double)d);
      for (int c = threadIdx.x; c < d; c += 256)
        part[(b * kVqSlots + blockIdx.x) * d + c] =
            div_rn(fmaxf(fmaxf(red[0][c], red[1][c]), fmaxf(red[2][c], red[3][c])), sd);
    }
  }
}

// Channel scales of head blockIdx.x: max over the head's partials (thread
// (c, j) takes slots j, j + 256 / d, ... of channel c), clamped to 1e-8; also
// the fp32 / fp16 copies the caller asked for.
__global__ __launch_bounds__(256) void k_vq_fold(const float* __restrict__ part, int64_t bh, int d,
                                                 int nslots, float* __restrict__ ch, float* ch_f32,
                                                 uint16_t* ch_f16, float* ch_rcp = nullptr) {
  __shared__ float red[256];
  const int tid = threadIdx.x, c = tid & (d - 1), j0 = tid / d, nj = 256 / d;
  for (int64_t b = blockIdx.x; b < bh; b += gridDim.x) {
    float m = 0.f;
#pragma unroll 8
    for (int x = j0; x < nslots; x += nj) m = fmaxf(m, part[(b * kVqSlots + x) * d + c]);
    __syncthreads();
    red[tid] = m;
    __syncthreads();
    if (tid < d) {
      for (int j = 1; j < nj; ++j) m = fmaxf(m, red[j * d + tid]);
      const float v = fmaxf(m, 1e-8f);
      ch[b * d + tid] = v;
      if (ch_f32) ch_f32[b * d + tid] = v;
      if (ch_f16) ch_f16[b * d + tid] = f2h(v);
      if (ch_rcp) ch_rcp[b * d + tid] = div_rn(1.f, v);
    }
  }
}

// ---------------------------------------------------------------------------
// Nearest centroid (triton_kernels.py:689-746 formula; first index on ties)
// ---------------------------------------------------------------------------
template <int D>
__global__ void k_vq_assign(const float* __restrict__ x, int64_t n,
                            const float* __restrict__ c, int k, int32_t* __restrict__ idx) {
  extern __shared__ float cs[];
  for (int i = threadIdx.x; i < k * D; i += blockDim.x) cs[i] = c[i];
  __syncthreads();
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < n; r += stride) {
    float xv[D];
#pragma unroll
    for (int j = 0; j < D; ++j) xv[j] = x[r * D + j];
    float best = INFINITY;
    int arg = 0;
    for (int q = 0; q < k; ++q) {
      float dist = 0.f;
#pragma unroll
      for (int j = 0; j < D; ++j) {
        float df = sub_rn(xv[j], cs[q * D + j]);
        dist = add_rn(dist, mul_rn(df, df));
      }
      if (dist < best) {
        best = dist;
        arg = q;
      }
    }
    idx[r] = arg;
  }
}

// ---------------------------------------------------------------------------
// Nearest centroid of 4-dim rows among k = 32 NB centroids (NB <= 8): the
// same result as k_vq_assign, found in two stages.
//  1. Screen on MFMA.  key(c) = bias + |c|^2 - 2 x.c (= |x - c|^2 - |x|^2 +
//     bias) for 32 rows x 32 centroids per pair of v_mfma_f32_32x32x16_bf16
//     (32 k slots): x and t = -2c are split into three bf16 parts each and
//     x.t ~ xh.th + xm.th + xh.tm + xl.th + xm.tm + xh.tl; |c|^2 takes three
//     slots and the row's bias bf16(1.03125 S) one.  S = max|c|^2 + 2 sum_j
//     |x_j| max|c_j| bounds ||c|^2 - 2 x.c|, so every key is a positive float
//     and orders like its bits as an unsigned integer.  The low 4 mantissa
//     bits of every key are replaced by the centroid's register index within
//     its 32-centroid block, and each lane keeps the two smallest keys of
//     every block (v_min_u32, v_med3_u32: 3 VALU ops per row and centroid).
//  2. Certify.  Every key is within 1.13e-5 S of the exact bias + |c|^2 -
//     2 x.c: dropped split products 4.01 2^-24 |x_j t_j| (2.4e-7 S), |c|^2 in
//     fp32 and its parts (4.5e-7 S), fp32 accumulation of the 28 terms
//     (< 27 2^-23 of their absolute sum <= 2.1 S: 6.8e-6 S, a worst case) and
//     the code (15 ulp of a key < 2.1 S: 3.8e-6 S).  The reference's direct
//     fp32 distance is within 6.01 2^-24 (relative) of |x - c|^2 (six
//     roundings of non-negative terms), so a centroid whose key exceeds
//     thr = min key + 2^-15 (S + |x|^2) (more than the 2 E + 12.1 2^-24
//     (|x|^2 + S) needed) can neither be the reference's argmin nor tie with
//     it.  If the second smallest key exceeds thr the smallest key's centroid
//     is the answer.  Otherwise the lane evaluates the reference's direct
//     distance for the tracked keys under thr (rescanning a block whose
//     second key is under thr, as it may hold a third), and for rows or
//     centroids that are non-finite or outside [2^-60, 2^64] in scale (where
//     the relative bounds could fail) for every centroid, keeping the
//     smallest distance and, among equal ones, the smallest index, as the
//     sequential strict-< scan does (an index-0 answer when no distance is
//     finite).
// ---------------------------------------------------------------------------

// the direct distance of the reference kernel's statement, uncontracted (this
// library's rule: no FMA): fp32 sum of squared differences in dim order
__device__ __forceinline__ float vq_dist4(const float (&xv)[4], const float4 cv) {
  const float cc[4] = {cv.x, cv.y, cv.z, cv.w};
  float dist = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float df = sub_rn(xv[j], cc[j]);
    dist = add_rn(dist, mul_rn(df, df));
  }
  return dist;
}

__device__ __forceinline__ uint32_t umin(uint32_t a, uint32_t b) { return a < b ? a : b; }
__device__ __forceinline__ uint32_t umax(uint32_t a, uint32_t b) { return a < b ? b : a; }
// median of three unsigned values in one VALU op (no builtin exists for the
// integer form, and the compiler rewrites the min/max expression of it)
__device__ __forceinline__ uint32_t umed3(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ uint32_t umin3(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_min3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// x = h + m + l in bf16 parts, |x - h - m - l| <= 2^-24 |x| (both
// differences are exact in fp32)
__device__ __forceinline__ void split3(float v, __bf16& h, __bf16& m, __bf16& l) {
  h = (__bf16)v;
  const float r = v - (float)h;
  m = (__bf16)r;
  l = (__bf16)(r - (float)m);
}

// (256, 2): at most 256 registers per lane, so the MFMA results land in VGPRs
template <int NB>
__global__ __launch_bounds__(256, 2)
void k_vq_assign_mfma(const float* __restrict__ x, int64_t n, const float* __restrict__ c,
                      int32_t* __restrict__ idx) {
  constexpr int K = 32 * NB;
  __shared__ float4 cs[K];
  __shared__ bf16x8 atab[NB][2][64];  // the A operands again, for the rare rescans
  const int tid = threadIdx.x, lane = tid & 63, col = lane & 31, hh = lane >> 5;
  for (int i = tid; i < K; i += 256) cs[i] = ((const float4*)c)[i];
  __syncthreads();

  // A operands of block b: lane (centroid 32 b + col, half hh) holds k slots
  // 8 hh .. 8 hh + 7 of each MFMA: first [th, tm] (hh 0) | [th, tl] (hh 1),
  // second [th, tm] (hh 0) | [|c|^2 in three parts, 1, 0, 0, 0, 0] (hh 1)
  bf16x8 a1[NB], a2[NB];
  float cnmax = 0.f, cm[4] = {0.f, 0.f, 0.f, 0.f};
  bool bad = false;
  const __bf16 one = (__bf16)1.f, nil = (__bf16)0.f;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const float4 cv = cs[32 * b + col];
    const float cc[4] = {cv.x, cv.y, cv.z, cv.w};
    __bf16 th[4], tm[4], tl[4];
    float cn = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      split3(-2.f * cc[j], th[j], tm[j], tl[j]);
      cn = cn + cc[j] * cc[j];
      cm[j] = fmaxf(cm[j], fabsf(cc[j]));
      bad |= !(fabsf(cc[j]) <= 0x1p60f);
    }
    __bf16 n0, n1, n2;
    split3(cn, n0, n1, n2);
    cnmax = fmaxf(cnmax, cn);
    const bf16x8 htm = {th[0], th[1], th[2], th[3], tm[0], tm[1], tm[2], tm[3]};
    a1[b] = hh == 0 ? htm : bf16x8{th[0], th[1], th[2], th[3], tl[0], tl[1], tl[2], tl[3]};
    a2[b] = hh == 0 ? htm : bf16x8{n0, n1, n2, one, nil, nil, nil, nil};
    if (tid < 64) {  // every wave builds the same operands; wave 0 stores them
      atab[b][0][lane] = a1[b];
      atab[b][1][lane] = a2[b];
    }
  }
  __syncthreads();
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) {
    cnmax = fmaxf(cnmax, __shfl_xor(cnmax, o));
#pragma unroll
    for (int j = 0; j < 4; ++j) cm[j] = fmaxf(cm[j], __shfl_xor(cm[j], o));
  }
  bad = __ballot(bad) != 0;  // wave-uniform

  const int64_t ngroups = (n + 31) / 32;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const float16v zero = {};
  for (int64_t g = ((int64_t)blockIdx.x * blockDim.x + tid) >> 6; g < ngroups; g += nwaves) {
    const int64_t row = g * 32 + col;
    const bool valid = row < n;
    const float4 x4 = ((const float4*)x)[valid ? row : 0];
    const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
    // B operands: lane (row col, half hh): first [xh, xh] (hh 0) | [xm, xh]
    // (hh 1), second [xl, xm] (hh 0) | [1, 1, 1, bias, 0, 0, 0, 0] (hh 1)
    __bf16 xh[4], xm[4], xl[4];
    float S = 0.f, xx = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      split3(xv[j], xh[j], xm[j], xl[j]);
      S = S + fabsf(xv[j]) * cm[j];
      xx = xx + xv[j] * xv[j];
    }
    S = cnmax + 2.f * S;
    const bool in_range = !bad && S >= 0x1p-60f && S <= 0x1p64f && xx <= 0x1p64f;
    const bf16x8 b1 = hh == 0 ? bf16x8{xh[0], xh[1], xh[2], xh[3], xh[0], xh[1], xh[2], xh[3]}
                              : bf16x8{xm[0], xm[1], xm[2], xm[3], xh[0], xh[1], xh[2], xh[3]};
    const bf16x8 b2 = hh == 0 ? bf16x8{xl[0], xl[1], xl[2], xl[3], xm[0], xm[1], xm[2], xm[3]}
                              : bf16x8{one, one, one, (__bf16)(1.03125f * S), nil, nil, nil, nil};
    auto keys = [&](int b) {
      return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          a2[b], b2, __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1[b], b1, zero, 0, 0, 0), 0, 0, 0);
    };
    // 1. the two smallest coded keys of each block; C reg i of block b is
    //    centroid 32 b + 8 (i / 4) + 4 hh + i % 4, code i.  Keys enter in
    //    pairs (a, b): the new second smallest of {m1 <= m2, a, b} is
    //    min(m2, med3(m1, a, b)) and the new smallest min3(m1, a, b), three
    //    compare ops per two keys.  The next block's MFMAs are issued before
    //    this block's keys are consumed.
    uint32_t m1[NB], m2[NB];
    float16v acc = keys(0);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      float16v nxt;
      if (b + 1 < NB) nxt = keys(b + 1);
      uint32_t e[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) e[i] = (__float_as_uint(acc[i]) & ~15u) | (uint32_t)i;
      m1[b] = umin(e[0], e[1]);
      m2[b] = umax(e[0], e[1]);
#pragma unroll
      for (int i = 2; i < 16; i += 2) {
        m2[b] = umin(m2[b], umed3(m1[b], e[i], e[i + 1]));
        m1[b] = umin3(m1[b], e[i], e[i + 1]);
      }
      if (b + 1 < NB) acc = nxt;
    }
    // smallest key of the lane, its block, and the lane's second smallest key
    // (the second smallest block minimum or a second key of any block)
    uint32_t T1 = m1[0], S1 = 0xFFFFFFFFu, T2 = m2[0];
    int blk = 0;
#pragma unroll
    for (int b = 1; b < NB; ++b) {
      S1 = umed3(T1, S1, m1[b]);
      blk = m1[b] < T1 ? b : blk;
      T1 = umin(T1, m1[b]);
      T2 = umin(T2, m2[b]);
    }
    T2 = umin(T2, S1);
    // the other half of the lane pair holds the row's other 16 centroids of each block
    const uint32_t oT1 = __shfl_xor(T1, 32), oT2 = __shfl_xor(T2, 32);
    const int oblk = __shfl_xor(blk, 32);
    const bool other = oT1 < T1;
    const uint32_t R2 = umin(umax(T1, oT1), umin(T2, oT2));
    const uint32_t R1 = umin(T1, oT1);
    const int ci = (int)(R1 & 15u);
    int best = 32 * (other ? oblk : blk) + 8 * (ci >> 2) + 4 * (other ? hh ^ 1 : hh) + (ci & 3);
    // 2. certify, or decide by the reference's distances
    const float thr = __uint_as_float(R1) + 0x1p-15f * (S + xx);
    const bool amb = valid && !(in_range && __uint_as_float(R2) > thr);
    if (__ballot(amb) != 0) {
      const bool all = amb && !in_range;
      const uint32_t lim = amb && in_range ? __float_as_uint(thr) : 0u;  // keys are > 0
      float bd = INFINITY;
      int bi = 0;
      auto consider = [&](int j) {
        const float d = vq_dist4(xv, cs[j]);
        if (d < bd || (d == bd && j < bi && d < INFINITY)) {
          bd = d;
          bi = j;
        }
      };
      auto centroid = [&](int b, int i) { return 32 * b + 8 * (i >> 2) + 4 * hh + (i & 3); };
      if (__ballot(all) != 0) {
#pragma unroll 1
        for (int j = 0; j < 16 * NB; ++j)
          if (all) consider(centroid(j >> 4, j & 15));
      }
      uint32_t more = 0;  // blocks whose second key is under thr may hold a third
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (m1[b] <= lim) consider(centroid(b, (int)(m1[b] & 15u)));
        if (m2[b] <= lim) {
          consider(centroid(b, (int)(m2[b] & 15u)));
          more |= 1u << b;
        }
      }
#pragma unroll 1
      for (int b = 0; b < NB; ++b) {
        const bool mb = (more >> b) & 1u;
        if (__ballot(mb) != 0) {
          const float16v acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              atab[b][1][lane], b2,
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(atab[b][0][lane], b1, zero, 0, 0, 0), 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 16; ++i)
            if (mb && __float_as_uint(acc[i]) <= lim) consider(centroid(b, i));
        }
      }
      const float od = __shfl_xor(bd, 32);
      const int oi = __shfl_xor(bi, 32);
      if (od < bd || (od == bd && oi < bi && od < INFINITY)) bi = oi;
      if (amb) best = bi;
    }
    if (hh == 0 && valid) idx[row] = best;
  }
}

// ---------------------------------------------------------------------------
// Nearest centroid of 4-dim rows through a candidate table (k = 32 NB <= 256):
// the same result as k_vq_assign, with most rows decided by the reference's
// direct distance to a few centroids.
//
// The box [lo, hi]^4 is cut into nbins^4 cells.  For each cell the table
// lists, in increasing index order, every centroid that can be the answer for
// (or tie with the answer for) some row of the cell.
//
// Why a centroid c may be left out of cell Q = prod_j [l_j, h_j]: the exact
// D(x, c) - D(x, c') (squared distances) is a sum over dims of terms linear in
// x_j, so its minimum over Q is
//   L = sum_j min((l_j - c_j)^2 - (l_j - c'_j)^2, (h_j - c_j)^2 - (h_j - c'_j)^2)
// and D(x, c) <= Dmax(c) = sum_j max((l_j - c_j)^2, (h_j - c_j)^2) on Q.  The
// reference's fp32 distance is within 6.01 2^-24 D of D (six roundings of
// non-negative terms) and L evaluated in fp32 is within 8 2^-24 (Dmax(c) +
// Dmax(c')) of its exact value, so
//   L > 2^-17 (Dmax(c) + Dmax(c')) + 2^-100
// (nine times the 14.01 2^-24 needed, plus an absolute term for underflow)
// means that at every row of Q the reference's distance to c exceeds its
// distance to c': c is neither the strict-< argmin nor tied with it.  Every
// left-out centroid is beaten at every row by some other centroid, so the
// first-index argmin is always listed, and the sequential strict-< scan of
// the ascending list returns it.  The build keeps c when no other centroid of
// a first survivor set (those the centroid nearest the cell centre does not
// beat) beats it.
//
// Cells: l_j = lo + i_j w - w/1024 and h_j = lo + (i_j + 1) w + w/1024 with
// w = (hi - lo)/nbins.  A row whose cell coordinate t_j = (x_j - lo) nbins /
// (hi - lo) (fp32) lies in [-2^-12, nbins + 2^-12] goes to cell
// clamp(trunc(t_j)): its fp32 error is below 1e-5 cells (96 2^-24 nbins) and
// the box corners are within 130 2^-24 (hi - lo) of their exact values when
// max(|lo|, |hi|) <= 64 (hi - lo), which the build requires, so the row lies
// in that cell's widened box.  Rows outside the box, non-finite rows and rows
// of cells with more than kVqTabCap candidates are appended to a list that
// k_vq_list_direct finishes with the direct distance to every centroid (fine
// for the few rows normalized data leaves there; rows not normalized to the
// box belong with shard_vq_assign).  A centroid set holding a non-finite
// value or one above 2^32 in magnitude lists every cell out.
//
// Table: a 64-byte header (nbins, k, lo, hi, a tag), one count byte per cell
// (kVqTabFull: listed out), then kVqTabCap candidate bytes per cell padded
// with the last candidate (a repeated candidate changes nothing under <).
// ---------------------------------------------------------------------------
constexpr int kVqTabCap = 32;
constexpr int kVqTabFull = 255;
constexpr int kVqTabHeader = 64;
constexpr int kVqTabMaxBins = 32;
constexpr int kVqTabSurv = 128;  // first-test survivors a build thread can hold
constexpr uint32_t kVqTabTag = 0x54715653u;

struct VqTabHeader {
  int32_t nbins, k;
  float lo, hi;
  uint32_t tag;
  int32_t pad[11];
};

__host__ __device__ inline int64_t vq_tab_cells(int nbins) {
  return (int64_t)nbins * nbins * nbins * nbins;
}
__host__ __device__ inline int64_t vq_tab_counts_bytes(int nbins) {
  return (vq_tab_cells(nbins) + 15) & ~(int64_t)15;
}

// the cell's box, widened by w/1024 on every side
__device__ __forceinline__ void vq_cell_box(int64_t cell, int nbins, float lo, float hi,
                                            float (&l)[4], float (&h)[4]) {
  const float w = (hi - lo) / (float)nbins, pad = w * 0x1p-10f;
  int64_t r = cell;
#pragma unroll
  for (int j = 3; j >= 0; --j) {
    const int i = (int)(r % nbins);
    r /= nbins;
    l[j] = lo + (float)i * w - pad;
    h[j] = lo + (float)(i + 1) * w + pad;
  }
}

// Four lanes per cell, 64 cells per 256-thread workgroup.  Lane q of a cell
// scans centroids q, q + 4, ...: the centroid nearest the cell centre (a quad
// reduction), then the first test against it, whose survivors set bits of
// the cell's LDS bitmap; the quad's first lane lists them in index order; each
// lane then tests every fourth survivor against all the others and marks the
// ones no survivor beats in a second bitmap, which the first lane writes out.
constexpr int kVqTabCells = 64;  // cells per build workgroup

__global__ __launch_bounds__(256) void k_vq_table_build(const float* __restrict__ c, int k,
                                                        float lo, float hi, int nbins,
                                                        uint8_t* __restrict__ table) {
  __shared__ float4 cs[256];
  __shared__ uint32_t first[kVqTabCells][8], keep[kVqTabCells][8];
  __shared__ __align__(4) uint8_t surv[kVqTabCells][kVqTabSurv];
  __shared__ int nsurv[kVqTabCells];
  const int tid = threadIdx.x, slot = tid >> 2, q = tid & 3;
  int bad = 0;
  for (int i = tid; i < k; i += 256) {
    const float4 v = ((const float4*)c)[i];
    cs[i] = v;
    bad |= !(fabsf(v.x) <= 0x1p32f && fabsf(v.y) <= 0x1p32f && fabsf(v.z) <= 0x1p32f &&
             fabsf(v.w) <= 0x1p32f);
  }
  for (int i = tid; i < kVqTabCells * 8; i += 256) {
    (&first[0][0])[i] = 0u;
    (&keep[0][0])[i] = 0u;
  }
  bad = __syncthreads_or(bad);
  if (blockIdx.x == 0 && tid == 0) {
    VqTabHeader hd = {};
    hd.nbins = nbins;
    hd.k = k;
    hd.lo = lo;
    hd.hi = hi;
    hd.tag = kVqTabTag;
    *(VqTabHeader*)table = hd;
  }
  const int64_t cell = (int64_t)blockIdx.x * kVqTabCells + slot;
  const bool live = cell < vq_tab_cells(nbins) && !bad;
  uint8_t* counts = table + kVqTabHeader;
  uint4* lists = (uint4*)(counts + vq_tab_counts_bytes(nbins));
  float l[4], h[4];
  vq_cell_box(live ? cell : 0, nbins, lo, hi, l, h);
  // corner terms of a centroid: (l_j - c_j)^2, (h_j - c_j)^2 and Dmax
  auto corners = [&](const float4 v, float (&a)[4], float (&b)[4]) {
    const float cc[4] = {v.x, v.y, v.z, v.w};
    float dm = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float p = l[j] - cc[j], r = h[j] - cc[j];
      a[j] = p * p;
      b[j] = r * r;
      dm += fmaxf(a[j], b[j]);
    }
    return dm;
  };
  // does the centroid with corner terms (a2, b2, d2) beat the one with (a, b, d) on the cell?
  auto beaten = [](const float (&a)[4], const float (&b)[4], float d, const float (&a2)[4],
                   const float (&b2)[4], float d2) {
    float L = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) L += fminf(a[j] - a2[j], b[j] - b2[j]);
    return L > 0x1p-17f * (d + d2) + 0x1p-100f;
  };
  if (live) {
    // the centroid nearest the centre (any one: it only orders the work)
    float best = INFINITY;
    int c0 = q;
#pragma unroll 4
    for (int i = q; i < k; i += 4) {
      const float4 v = cs[i];
      const float cc[4] = {v.x, v.y, v.z, v.w};
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float e = 0.5f * (l[j] + h[j]) - cc[j];
        d += e * e;
      }
      if (d < best) {
        best = d;
        c0 = i;
      }
    }
#pragma unroll
    for (int o = 1; o < 4; o <<= 1) {
      const float ob = __shfl_xor(best, o);
      const int oc = __shfl_xor(c0, o);
      if (ob < best || (ob == best && oc < c0)) {
        best = ob;
        c0 = oc;
      }
    }
    float a0[4], b0[4];
    const float d0 = corners(cs[c0], a0, b0);
#pragma unroll 4
    for (int i = q; i < k; i += 4) {
      float a[4], b[4];
      const float d = corners(cs[i], a, b);
      if (!beaten(a, b, d, a0, b0, d0)) atomicOr(&first[slot][i >> 5], 1u << (i & 31));
    }
  }
  __syncthreads();
  if (live && q == 0) {  // the survivors in index order
    int n = 0;
    for (int w = 0; w < 8; ++w) {
      uint32_t bits = first[slot][w];
      while (bits) {
        const int i = 32 * w + __builtin_ctz(bits);
        bits &= bits - 1;
        if (n < kVqTabSurv) surv[slot][n] = (uint8_t)i;
        ++n;
      }
    }
    nsurv[slot] = n;
  }
  __syncthreads();
  const int n = live ? nsurv[slot] : 0;
  if (live && n <= kVqTabSurv) {
    // survivors q, q + 4, ... against all the others, four comparators per
    // step (their indices in one LDS word; bytes past n are never used)
    for (int s = q; s < n; s += 4) {
      float a[4], b[4];
      const int ci = surv[slot][s];
      const float d = corners(cs[ci], a, b);
      bool out = false;
      for (int t0 = 0; t0 < n && !out; t0 += 4) {
        const uint32_t w = *(const uint32_t*)&surv[slot][t0];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float a2[4], b2[4];
          const float d2 = corners(cs[(w >> (8 * r)) & 255u], a2, b2);
          const int t = t0 + r;
          out = out || (t < n && t != s && beaten(a, b, d, a2, b2, d2));
        }
      }
      if (!out) atomicOr(&keep[slot][ci >> 5], 1u << (ci & 31));
    }
  }
  __syncthreads();
  if (!(cell < vq_tab_cells(nbins)) || q != 0) return;
  int m = 0;
  if (live && n <= kVqTabSurv) {
    int last = 0;
    for (int w = 0; w < 8; ++w) {
      uint32_t bits = keep[slot][w];
      while (bits) {
        const int i = 32 * w + __builtin_ctz(bits);
        bits &= bits - 1;
        if (m < kVqTabCap) surv[slot][m] = (uint8_t)i;  // the survivor list is done with
        last = i;
        ++m;
      }
    }
    // (m >= 1 always: a beating chain cannot close)
    if (m >= 1 && m <= kVqTabCap)
      for (int s = m; s < kVqTabCap; ++s) surv[slot][s] = (uint8_t)last;
  }
  if (m < 1 || m > kVqTabCap) {  // listed out: its rows take the other path
    counts[cell] = (uint8_t)kVqTabFull;
    return;
  }
  counts[cell] = (uint8_t)m;
  const uint32_t* sw = (const uint32_t*)&surv[slot][0];
  lists[2 * cell] = make_uint4(sw[0], sw[1], sw[2], sw[3]);
  lists[2 * cell + 1] = make_uint4(sw[4], sw[5], sw[6], sw[7]);
}

// Undecided rows: wave w of a table assignment appends its rows (and, when
// it formed them itself, their values) to region w of the workspace
// (vq_list_per rows, the most it can meet) and stores their count in
// counts[w], with no atomic; k_vq_list_direct reads every region.
struct VqList {
  int32_t* counts;  // one per wave of the launch
  int32_t* rows;    // nwaves * per
  float4* xs;       // nwaves * per values, or null
  int64_t per;      // rows per region
};
inline void vq_list_geometry(int64_t n, int* grid, int64_t* per) {
  const int64_t groups = (n + 63) / 64;  // 64 rows per wave
  *grid = grid_cap((groups + 3) / 4, 4096);
  const int64_t nwaves = (int64_t)*grid * 4;
  *per = (groups + nwaves - 1) / nwaves * 64;
}

// The rows a table left undecided: the reference's direct distance to every
// centroid in index order, strict < (k_vq_assign's rule).  A small kernel on
// purpose: it follows every table assignment, usually to find every region
// empty (then each workgroup returns after reading its share of the counts),
// and must start at once beside other streams' kernels.
template <bool WITH_X>
__global__ __launch_bounds__(256) void k_vq_list_direct(const float* __restrict__ x,
                                                        const float* __restrict__ c, int k,
                                                        int32_t* __restrict__ idx,
                                                        const VqList lst, int nregions) {
  // thread t owns regions t, t + T, t + 2 T, ... (T threads in all)
  const int t0 = blockIdx.x * 256 + threadIdx.x, nt = gridDim.x * 256;
  int any = 0;
  for (int r = t0; r < nregions; r += nt) any |= lst.counts[r] != 0;
  if (!__syncthreads_or(any)) return;
  __shared__ float4 cs[256];
  for (int i = threadIdx.x; i < k; i += 256) cs[i] = ((const float4*)c)[i];
  __syncthreads();
  for (int r = t0; r < nregions; r += nt) {
    const int cnt = lst.counts[r];
    for (int i = 0; i < cnt; ++i) {
      const int64_t slot = (int64_t)r * lst.per + i;
      const int row = lst.rows[slot];
      const float4 x4 = WITH_X ? lst.xs[slot] : ((const float4*)x)[row];
      const float xv[4] = {x4.x, x4.y, x4.z, x4.w};
      float bd = INFINITY;
      int bi = 0;
      for (int q = 0; q < k; ++q) {
        const float d = vq_dist4(xv, cs[q]);
        if (d < bd) {
          bd = d;
          bi = q;
        }
      }
      idx[row] = bi;
    }
  }
}

// Rows for k_vq_assign_table<true>: computed from V (head_dim 128) as
// shard_vq_prepare's pass 2 computes them, instead of read from x.
struct VqFromV {
  const uint16_t* v;
  int64_t seq, bh_stride;
  const float* ch;   // (bh, 128) channel scales
  const float* rch;  // their correctly rounded reciprocals
};

// wave = 64 rows, one per lane; the candidates of the lane's cell are scanned
// in order up to the wave's largest count (a scalar loop bound).  FROM_V: the
// wave's rows are two tokens' 32 subvectors, lane l holding subvector l % 32
// of token 2 g + l / 32: the lane loads its 4 values of V, the FWHT runs
// within each half-wave (strides 1, 2 in the lane, then lanes 1..16 apart:
// the reference's stage order), and the row is divided by sqrt(128) and its
// channel scales; undecided rows go to the list with their values.
template <bool FROM_V>
__global__ __launch_bounds__(256) void k_vq_assign_table(
    const float* __restrict__ x, int64_t n, const float* __restrict__ c, int k,
    const uint8_t* __restrict__ table, int nbins, float lo, float hi, int32_t* __restrict__ idx,
    const VqList lst, const VqFromV fv) {
  __shared__ float4 cs[256];
  for (int i = threadIdx.x; i < k; i += 256) cs[i] = ((const float4*)c)[i];
  __syncthreads();
  const VqTabHeader* hd = (const VqTabHeader*)table;
  const bool ok = hd->tag == kVqTabTag && hd->nbins == nbins && hd->k == k &&
                  __float_as_uint(hd->lo) == __float_as_uint(lo) &&
                  __float_as_uint(hd->hi) == __float_as_uint(hi);
  const uint8_t* counts = table + kVqTabHeader;
  const uint4* lists = (const uint4*)(counts + vq_tab_counts_bytes(nbins));
  const float inv_w = (float)nbins / (hi - lo), tmax = (float)nbins + 0x1p-12f;
  const int lane = threadIdx.x & 63;
  const int64_t ngroups = (n + 63) / 64;
  const int64_t nwaves = ((int64_t)gridDim.x * blockDim.x) >> 6;
  const float sd = (float)sqrt(128.0), rsd = div_rn(1.f, sd);
  // a row's inputs (x, or its V values and channel scales) are loaded one
  // group ahead
  struct In {
    uint4 a;       // x, or (V's 4 halves, -, -)
    float4 c, r;   // FROM_V: the channel scales and their reciprocals
  };
  const int64_t g0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  auto load_in = [&](int64_t g) {
    const int64_t row = g * 64 + lane;
    const bool live = row < n;
    In in_;
    if constexpr (FROM_V) {
      const int64_t tok = live ? row >> 5 : 0;
      const int64_t b = tok / fv.seq, t = tok - b * fv.seq;
      const int j = lane & 31;
      const uint2 raw = *(const uint2*)(fv.v + b * fv.bh_stride + t * 128 + 4 * j);
      in_.a = make_uint4(raw.x, raw.y, 0u, 0u);
      in_.c = *(const float4*)(fv.ch + b * 128 + 4 * j);
      in_.r = *(const float4*)(fv.rch + b * 128 + 4 * j);
    } else {
      in_.a = __builtin_bit_cast(uint4, ((const float4*)x)[live ? row : 0]);
    }
    return in_;
  };
  In nxt = {};
  if (g0 < ngroups) nxt = load_in(g0);
  const int64_t region = g0 * lst.per;  // this wave's undecided rows
  int filled = 0;
  for (int64_t g = g0; g < ngroups; g += nwaves) {
    const int64_t row = g * 64 + lane;
    const bool live = row < n;
    const In in_ = nxt;
    if (g + nwaves < ngroups) nxt = load_in(g + nwaves);
    float xv[4];
    if constexpr (FROM_V) {
      const uint2 raw = make_uint2(in_.a.x, in_.a.y);
      float u[4] = {h2f((uint16_t)raw.x), h2f((uint16_t)(raw.x >> 16)), h2f((uint16_t)raw.y),
                    h2f((uint16_t)(raw.y >> 16))};
      // strides 1 and 2 inside the lane, then 4 .. 64 across lanes 1 .. 16 apart
#pragma unroll
      for (int h = 1; h < 4; h <<= 1)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((e & h) == 0) {
            const float a0 = u[e], a1 = u[e | h];
            u[e] = add_rn(a0, a1);
            u[e | h] = sub_rn(a0, a1);
          }
      fwht_lane_stage<1>(u, lane);
      fwht_lane_stage<2>(u, lane);
      fwht_lane_stage<4>(u, lane);
      fwht_lane_stage<8>(u, lane);
      fwht_lane_stage<16>(u, lane);
      const float cc[4] = {in_.c.x, in_.c.y, in_.c.z, in_.c.w};
      const float rr[4] = {in_.r.x, in_.r.y, in_.r.z, in_.r.w};
      bool finite = true;
#pragma unroll
      for (int e = 0; e < 4; ++e) finite = finite && fabsf(cc[e]) <= 0x1.fffffep127f;
      if (__ballot(!finite) == 0) {  // as shard_vq_prepare: reciprocals unless a scale is infinite
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = div_by_rcp(div_by_rcp(u[e], sd, rsd), cc[e], rr[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = div_rn(div_rn(u[e], sd), cc[e]);
      }
    } else {
      const float4 x4 = __builtin_bit_cast(float4, in_.a);
      xv[0] = x4.x;
      xv[1] = x4.y;
      xv[2] = x4.z;
      xv[3] = x4.w;
    }
    bool in = ok && live;
    int cell = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float t = (xv[j] - lo) * inv_w;
      in = in && t >= -0x1p-12f && t <= tmax;
      const int i = (int)(in ? fmaxf(t, 0.f) : 0.f);
      cell = cell * nbins + (i < nbins ? i : nbins - 1);
    }
    // the count and the list together (a listed-out cell's list bytes are
    // never written; its rows use no candidate, and any byte indexes cs)
    int cnt = kVqTabFull;
    uint4 c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
    if (in) {
      cnt = counts[cell];
      c0 = lists[2 * cell];
      c1 = lists[2 * cell + 1];
    }
    const bool fast = cnt != kVqTabFull;
    // the wave's largest count, bit by bit from ballots (counts <= 32)
    const int cv = fast ? cnt : 0;
    int top = 0;
#pragma unroll
    for (int b = 5; b >= 0; --b)
      if (__ballot(cv >= (top | (1 << b)))) top |= 1 << b;
    const uint32_t wl[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    float bd = INFINITY;
    int bi = 0;
    // four candidates per list word; the bytes past a lane's count repeat its
    // last candidate
#pragma unroll
    for (int w = 0; w < kVqTabCap / 4; ++w) {
      if (4 * w < top) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int ci = (int)((wl[w] >> (8 * q)) & 255u);
          const float d = vq_dist4(xv, cs[ci]);
          if (d < bd) {
            bd = d;
            bi = ci;
          }
        }
      }
    }
    if (fast && live) idx[row] = bi;
    const bool rest = live && !fast;
    const uint64_t mask = __ballot(rest);
    if (mask) {
      const int64_t slot = region + filled + (int)__popcll(mask & ((1ull << lane) - 1));
      if (rest) {
        lst.rows[slot] = (int32_t)row;
        if constexpr (FROM_V) lst.xs[slot] = make_float4(xv[0], xv[1], xv[2], xv[3]);
      }
      filled += (int)__popcll(mask);
    }
  }
  if (lane == 0) lst.counts[g0] = filled;  // every wave, 0 included
}

// ---------------------------------------------------------------------------
// Deterministic k-means update: stable counting sort of the rows by centroid
// into a sorted copy, then each (centroid, dim) sums its rows in increasing
// row order (torch CPU index_add_ order), divides by the count, and keeps
// empty centroids.
//   blk[q * nblk + b]: rows of block b (KM_R rows) with centroid q; after the
//   scan, the first slot of those rows within centroid q's run.
// ---------------------------------------------------------------------------
constexpr int KM_R = 4096;   // rows per block of the counting sort
constexpr int KM_DMAX = 8;   // widest rows the sorted copy holds

__global__ __launch_bounds__(256) void k_km_hist(const int32_t* __restrict__ idx, int64_t n, int k,
                                                 int64_t nblk, int32_t* __restrict__ blk) {
  __shared__ int32_t h[1024];
  for (int i = threadIdx.x; i < k; i += blockDim.x) h[i] = 0;
  __syncthreads();
  const int64_t r0 = (int64_t)blockIdx.x * KM_R;
  for (int i = threadIdx.x; i < KM_R; i += blockDim.x)
    if (r0 + i < n) atomicAdd(&h[idx[r0 + i]], 1);
  __syncthreads();
  for (int q = threadIdx.x; q < k; q += blockDim.x) blk[(int64_t)q * nblk + blockIdx.x] = h[q];
}

// For each centroid (one workgroup): exclusive scan of its per-block counts
// (contiguous, 256 at a time: wave scans, then the four wave totals) in place,
// and its total count.
__global__ __launch_bounds__(256) void k_km_scan_blocks(int32_t* __restrict__ blk, int64_t nblk,
                                                        int32_t* __restrict__ count) {
  __shared__ int32_t wsum[4];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  int32_t* row = blk + (int64_t)blockIdx.x * nblk;
  int32_t carry = 0;
  for (int64_t base = 0; base < nblk; base += 256) {
    const int64_t i = base + t;
    const int32_t v = i < nblk ? row[i] : 0;
    int32_t sc = v;  // inclusive scan over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int32_t u = __shfl_up(sc, o, 64);
      if (lane >= o) sc += u;
    }
    if (lane == 63) wsum[w] = sc;
    __syncthreads();
    int32_t pre = carry;
    for (int u = 0; u < w; ++u) pre += wsum[u];
    if (i < nblk) row[i] = pre + sc - v;
    carry += wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();  // wsum is rewritten by the next round
  }
  if (t == 0) count[blockIdx.x] = carry;
}

__global__ void k_km_offsets(const int32_t* __restrict__ count, int k, int32_t* __restrict__ off) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    int32_t run = 0;
    for (int q = 0; q < k; ++q) {
      off[q] = run;
      run += count[q];
    }
  }
}

// One wave per block of KM_R rows, 64 rows per round in increasing order.  A
// row's slot is its centroid's running count in the block (LDS) plus the
// number of lower lanes of the round with the same centroid (lanes that agree
// on every bit of the centroid index, from one ballot per bit); the last lane
// of each centroid's group then advances the count.  The row's D values go to
// the sorted copy at that slot.
template <int D>
__global__ __launch_bounds__(64) void k_km_scatter(const float* __restrict__ x,
                                                   const int32_t* __restrict__ idx, int64_t n,
                                                   int k, int64_t nblk,
                                                   const int32_t* __restrict__ blk,
                                                   const int32_t* __restrict__ off,
                                                   float* __restrict__ xs) {
  __shared__ int32_t run[1024];
  const int lane = threadIdx.x;
  const int64_t b = blockIdx.x;
  for (int q = lane; q < k; q += 64) run[q] = off[q] + blk[(int64_t)q * nblk + b];
  __syncthreads();
  const int nbits = k > 1 ? 32 - __builtin_clz((unsigned)(k - 1)) : 0;
  const uint64_t below = (1ull << lane) - 1ull;
  const int64_t r0 = b * KM_R;
  constexpr int RU = 4;  // rounds whose loads go out together
  for (int rr = 0; rr < KM_R && r0 + rr < n; rr += 64 * RU) {
    int key[RU];
    float xv[RU][D];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int64_t r = r0 + rr + 64 * u + lane;
      const bool valid = rr + 64 * u < KM_R && r < n;
      key[u] = valid ? idx[r] : -1;
#pragma unroll
      for (int j = 0; j < D; ++j) xv[u][j] = valid ? x[r * D + j] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const bool valid = key[u] >= 0;
      const int kk = valid ? key[u] : 0;
      uint64_t m = __ballot(valid);
      for (int bit = 0; bit < nbits; ++bit) {
        const bool on = (kk >> bit) & 1;
        const uint64_t bb = __ballot(on);
        m &= on ? bb : ~bb;
      }
      const int rank = __popcll(m & below);
      const int grp = __popcll(m);
      const int slot = valid ? run[kk] + rank : 0;
      // every lane has read its centroid's count (LDS is in order within the
      // wave) before the group's last lane advances it
      if (valid && rank == grp - 1) run[kk] += grp;
      if (valid) {
#pragma unroll
        for (int j = 0; j < D; ++j) xs[(int64_t)slot * D + j] = xv[u][j];
      }
    }
  }
}

// One workgroup per centroid over its run of the sorted copy (increasing row
// order).  Chunks of 256 P rows are loaded (coalesced) one chunk ahead and
// staged in LDS dim-major (columns padded so the D lanes read distinct
// banks), double-buffered; lanes 0..D-1 of wave 0 add them in order, one
// running sum per dim, with the LDS reads of the next 32 values in flight
// while the current 32 are added.
template <int D>
__global__ __launch_bounds__(256) void k_km_sum(const float* __restrict__ xs,
                                                const int32_t* __restrict__ count,
                                                const int32_t* __restrict__ off,
                                                const float* __restrict__ c, int k,
                                                float* __restrict__ newc, uint32_t* __restrict__ maxd) {
  constexpr int P = D <= 4 ? 4 : 2;  // rows per thread per chunk
  constexpr int CH = 256 * P;        // rows per chunk
  constexpr int CS = CH + 4;         // column stride
  __shared__ __align__(16) float buf[2][D][CS];
  const int q = blockIdx.x;
  const int t = threadIdx.x;
  const int32_t cnt = count[q];
  const float* src = xs + (int64_t)off[q] * D;
  float xv[P][D];
  auto load = [&](int32_t base) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int32_t row = base + 256 * p + t;
      if (row < cnt) {
#pragma unroll
        for (int j = 0; j < D; ++j) xv[p][j] = src[(int64_t)row * D + j];
      }
    }
  };
  load(0);
  float acc = 0.f;
  int cur = 0;
  for (int32_t base = 0; base < cnt; base += CH) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (base + 256 * p + t < cnt) {
#pragma unroll
        for (int j = 0; j < D; ++j) buf[cur][j][256 * p + t] = xv[p][j];
      }
    }
    __syncthreads();
    load(base + CH);
    if (t < D) {
      const int n_here = cnt - base < CH ? cnt - base : CH;
      const float* col = buf[cur][t];
      const float4* c4 = (const float4*)col;
      const int nb = n_here >> 5;  // blocks of 32 values
      float4 va[8], vb[8];
      auto rd = [&](float4 (&r)[8], int blk) {  // a block past the end reads the last one (unused)
        const int bb = blk < nb ? blk : nb - 1;
#pragma unroll
        for (int u = 0; u < 8; ++u) r[u] = c4[8 * bb + u];
      };
      auto sum32 = [&](const float4 (&r)[8]) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          acc = add_rn(acc, r[u].x);
          acc = add_rn(acc, r[u].y);
          acc = add_rn(acc, r[u].z);
          acc = add_rn(acc, r[u].w);
        }
      };
      if (nb > 0) rd(va, 0);
      int blk = 0;
      for (; blk + 2 <= nb; blk += 2) {  // va holds block blk
        rd(vb, blk + 1);
        sum32(va);
        rd(va, blk + 2);
        sum32(vb);
      }
      if (blk < nb) sum32(va);
      for (int i = nb * 32; i < n_here; ++i) acc = add_rn(acc, col[i]);
    }
    cur ^= 1;
  }
  if (t < D) {
    const int idx = q * D + t;
    const float old = c[idx];
    const float nv = cnt > 0 ? div_rn(acc, (float)cnt) : old;
    newc[idx] = nv;
    atomicMax(maxd, __float_as_uint(fabsf(sub_rn(nv, old))));
  }
}

__global__ void k_km_zero(uint32_t* p) { *p = 0u; }

// ---------------------------------------------------------------------------
// Per-token 8-bit Lloyd-Max stream quantizer (cache.py:207-215, streaming.py:59-72)
// one wave per row, E = hd/64 elements per lane.
// ---------------------------------------------------------------------------
// Input and outputs of one tensor; blockIdx.y picks one of two (a token's K
// and V quantized by one launch).
struct StreamIO {
  const uint16_t* x[2];
  uint8_t* idx[2];
  uint16_t* norm[2];
  uint8_t* qsign[2];
  uint16_t* qscale[2];
  uint16_t* deq[2];
};

// Quantize row r held by one wave (t = its fp16 values as fp32, lane l holds
// elements l + 64 k) with the codebook cb (LDS); outputs at row r.
template <int E>
__device__ __forceinline__ void stream_quant_row(float (&t)[E], int64_t r,
                                                 const float* __restrict__ signs,
                                                 const float* cb, int n_codes,
                                                 uint8_t* __restrict__ idx,
                                                 uint16_t* __restrict__ norm,
                                                 uint8_t* __restrict__ qsign,
                                                 uint16_t* __restrict__ qscale,
                                                 uint16_t* __restrict__ deq) {
  constexpr int D = 64 * E;
  const int l = (int)lane_id();
  float sq[E], res[E];
#pragma unroll
  for (int k = 0; k < E; ++k) sq[k] = mul_rn(t[k], t[k]);  // exact: fp16-derived values square exactly in fp32
  // torch CPU fp32 norm: accumulator j (< 8) sums elements j, j+8, j+16, ... in
  // increasing order; the 8 accumulators are then added left to right.
  float acc = 0.f;
#pragma unroll
  for (int m = 0; m < D / 8; ++m) {
    float v = __shfl(sq[(8 * m) >> 6], (l + 8 * m) & 63, 64);
    acc = add_rn(acc, v);  // meaningful in lanes 0..7 (lane j holds accumulator j)
  }
  float tot = __shfl(acc, 0, 64);
#pragma unroll
  for (int j = 1; j < 8; ++j) tot = add_rn(tot, __shfl(acc, j, 64));
  float n = fmaxf(sqrtf(tot), 1e-8f);
#pragma unroll
  for (int k = 0; k < E; ++k) t[k] = mul_sign(div_rn(t[k], n), signs[l + 64 * k]);
  wave_fwht<E>(t, D);
#pragma unroll
  for (int k = 0; k < E; ++k) {
    float v = t[k];
    int lo = 0, hi = n_codes;  // first i with v <= cb[i] (torch.bucketize, right=False)
    while (lo < hi) {
      int mid = (lo + hi) >> 1;
      if (cb[mid] < v) lo = mid + 1; else hi = mid;
    }
    int i = lo < n_codes - 1 ? lo : n_codes - 1;
    int left = i > 0 ? i - 1 : 0;
    float dl = fabsf(sub_rn(cb[left], v));
    float di = fabsf(sub_rn(cb[i], v));
    const int code = dl < di ? left : i;
    idx[r * D + l + 64 * k] = (uint8_t)code;
    res[k] = sub_rn(v, cb[code]);  // QJL residual (streaming.py:69)
    t[k] = cb[code];
  }
  const uint16_t nh = f2h(n);
  if (l == 0) norm[r] = nh;
  if (qsign) {
    // QJL: sign bit of the residual per element, fp16 mean |residual| per row
    // (streaming.py:68-70), the mean in torch CPU's order for a contiguous
    // fp32 row: element i goes to accumulator (i / 8) % 4, lane i % 8, in
    // increasing i; the 4 accumulators are added in order per lane, then the
    // 8 lanes in order; then one division by the row length.
    float ares[E];
#pragma unroll
    for (int k = 0; k < E; ++k) {
      qsign[r * D + l + 64 * k] = res[k] >= 0.f ? 1 : 0;
      ares[k] = fabsf(res[k]);
    }
    float acc = 0.f;  // lane L < 32 holds accumulator (L / 8, L % 8): elements L + 32 m
#pragma unroll
    for (int m = 0; m < D / 32; ++m) {
      const float v = __shfl(ares[(32 * m) >> 6], (l + 32 * m) & 63, 64);
      acc = add_rn(acc, v);
    }
    float tot = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float vj = __shfl(acc, j, 64);
#pragma unroll
      for (int a = 1; a < 4; ++a) vj = add_rn(vj, __shfl(acc, j + 8 * a, 64));
      tot = j == 0 ? vj : add_rn(tot, vj);
    }
    const uint16_t sh = f2h(div_rn(tot, (float)D));
    if (l == 0) qscale[r] = sh;
    const float sf = h2f(sh);
#pragma unroll
    for (int k = 0; k < E; ++k) t[k] = add_rn(t[k], res[k] >= 0.f ? sf : -sf);
  }
  if (deq) {
    // reference dequant: fp16(fp16(hadamard(cb[idx] (+ qjl)) * signs) * fp16 norm)
    wave_fwht<E>(t, D);
    const float nf = h2f(nh);
#pragma unroll
    for (int k = 0; k < E; ++k)
      deq[r * D + l + 64 * k] = f2h_opaque(h2f(f2h(mul_sign(t[k], signs[l + 64 * k]))) * nf);
  }
}

template <int E>
__global__ void k_stream_quant(const StreamIO io, int64_t rows,
                               const float* __restrict__ signs, const float* __restrict__ cb_g,
                               int n_codes) {
  constexpr int D = 64 * E;
  const int job = blockIdx.y;
  __shared__ float cb[256];
  for (int i = threadIdx.x; i < n_codes; i += blockDim.x) cb[i] = cb_g[i];
  __syncthreads();
  const int l = (int)lane_id();
  const int w = threadIdx.x >> 6;
  int64_t r = (int64_t)blockIdx.x * (blockDim.x >> 6) + w;
  if (r >= rows) return;  // no block-level barrier below this point
  const uint16_t* __restrict__ x = io.x[job];
  float t[E];
#pragma unroll
  for (int k = 0; k < E; ++k) t[k] = h2f(x[r * D + l + 64 * k]);
  stream_quant_row<E>(t, r, signs, cb, n_codes, io.idx[job], io.norm[job], io.qsign[job],
                      io.qscale[job], io.deq[job]);
}

// ---------------------------------------------------------------------------
// Decode-step front end: RoPE of q and k with transformers' fp16 arithmetic
// (apply_rotary_pos_emb: q * cos + rotate_half(q) * sin, each product and the
// sum rounded to fp16 as torch's half ops do), then the new token's k and v
// quantized into the stream (as k_stream_quant).  One wave per row: rows
// [0, B H) are q rows (-> q_out), the next B G rows k, the last B G rows v.
// E >= 2 and even: the RoPE pair (d, d + D / 2) of element l + 64 k is element
// l + 64 (k + E / 2) of the same lane.
// ---------------------------------------------------------------------------
template <int E>
__device__ __forceinline__ void rope_row(float (&t)[E], const uint16_t* __restrict__ c,
                                         const uint16_t* __restrict__ sn) {
  const int l = (int)lane_id();
  float o[E];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    const int d = l + 64 * k;
    float rot;  // rotate_half
    if constexpr (E == 1) {  // head_dim 64: the partner dim is 32 lanes away
      const float pt = __shfl_xor(t[0], 32);
      rot = l < 32 ? -pt : pt;
    } else {
      rot = k < E / 2 ? -t[k + E / 2] : t[k - E / 2];
    }
    const float a = h2f(f2h(mul_rn(t[k], h2f(c[d]))));
    const float b = h2f(f2h(mul_rn(rot, h2f(sn[d]))));
    o[k] = h2f(f2h(add_rn(a, b)));
  }
#pragma unroll
  for (int k = 0; k < E; ++k) t[k] = o[k];
}

template <int E>
__global__ void k_rope_stream(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kx,
                              const uint16_t* __restrict__ vx, const uint16_t* __restrict__ cosv,
                              const uint16_t* __restrict__ sinv, int64_t cs_stride, int B,
                              int H, int G, uint16_t* __restrict__ q_out, const StreamIO io,
                              const float* __restrict__ signs, const float* __restrict__ cb_g,
                              int n_codes, const int32_t* __restrict__ row_dev, int row_cap) {
  constexpr int D = 64 * E;
  __shared__ float cb[256];
  for (int i = threadIdx.x; i < n_codes; i += blockDim.x) cb[i] = cb_g[i];
  __syncthreads();
  const int l = (int)lane_id();
  const int64_t r = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t nq = (int64_t)B * H, nk = (int64_t)B * G;
  if (r >= nq + 2 * nk) return;  // no block-level barrier below this point
  float t[E];
  if (r < nq) {
    const int64_t b = r / H;
#pragma unroll
    for (int k = 0; k < E; ++k) t[k] = h2f(q[r * D + l + 64 * k]);
    rope_row<E>(t, cosv + b * cs_stride, sinv + b * cs_stride);
#pragma unroll
    for (int k = 0; k < E; ++k) q_out[r * D + l + 64 * k] = f2h(t[k]);
    return;
  }
  const int job = r < nq + nk ? 0 : 1;  // 0: k, 1: v
  const int64_t rr = r - nq - job * nk;
  const uint16_t* __restrict__ x = job == 0 ? kx : vx;
#pragma unroll
  for (int k = 0; k < E; ++k) t[k] = h2f(x[rr * D + l + 64 * k]);
  if (job == 0) rope_row<E>(t, cosv + (rr / G) * cs_stride, sinv + (rr / G) * cs_stride);
  uint8_t* idx = io.idx[job];
  uint16_t* norm = io.norm[job];
  uint8_t* qsign = io.qsign[job];
  uint16_t* qscale = io.qscale[job];
  uint16_t* deq = io.deq[job];
  if (row_dev) {
    // the outputs are the buffers' bases and the token's row comes from device
    // memory (a captured graph replays one launch for every decode step); a
    // row outside [0, row_cap) writes nothing
    const int64_t row = *row_dev;
    if (row < 0 || row >= row_cap) return;
    idx += row * nk * D;
    norm += row * nk;
    if (qsign) {
      qsign += row * nk * D;
      qscale += row * nk;
    }
    if (deq) deq += row * nk * D;
  }
  stream_quant_row<E>(t, rr, signs, cb, n_codes, idx, norm, qsign, qscale, deq);
}

// ---------------------------------------------------------------------------
// Prefill K preparation: undo RoPE (fp32), subtract mean, fp16 GEMM operand.
// ---------------------------------------------------------------------------
// One workgroup per token t of the window: the token's hd/2 RoPE phases are
// computed once (shared by every batch row and kv head), then thread (i4, y)
// undoes pairs 4 i4 .. 4 i4 + 3 of the (b, g) rows y, y + blockDim.y, ...
// (8-byte loads; hd a multiple of 8).  OutT = uint16_t writes the centred rows
// rounded once to fp16 (the fp16 GEMM operand); OutT = float writes them as
// computed, the fp32 rows the reference projects (cache.py:370-392).
template <typename OutT>
__global__ __launch_bounds__(256) void k_k_prepare(const uint16_t* __restrict__ k, int batch,
                                                   int n_kv, int seq, int hd, int start, int n_comp,
                                                   const float* __restrict__ inv_freq,
                                                   const float* __restrict__ mean,
                                                   OutT* __restrict__ out) {
  __shared__ float2 ph[256];  // (cos, sin) of the token's phases, hd / 2 <= 256
  const int hd2 = hd >> 1, D = n_kv * hd;
  const int t = blockIdx.x, pos = start + t;
  const int flat = threadIdx.y * blockDim.x + threadIdx.x;
  const int i0 = 4 * threadIdx.x;  // blockDim.x == hd / 8
  // the first rows' loads go out before the phases are computed
  const int nbg = batch * n_kv;
  auto row_src = [&](int bg) {
    const int b = bg / n_kv, g = bg - b * n_kv;
    return k + (((int64_t)b * n_kv + g) * seq + pos) * hd;
  };
  uint2 lo_n = make_uint2(0u, 0u), hi_n = make_uint2(0u, 0u);
  if (threadIdx.y < nbg) {
    const uint16_t* src = row_src(threadIdx.y);
    lo_n = *(const uint2*)(src + i0);
    hi_n = *(const uint2*)(src + hd2 + i0);
  }
  for (int i = flat; i < hd2; i += blockDim.x * blockDim.y) {
    float sn, cs;
    sincosf(mul_rn((float)pos, inv_freq[i]), &sn, &cs);
    ph[i] = make_float2(cs, sn);
  }
  __syncthreads();
  float2 p[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) p[j] = ph[i0 + j];
  for (int bg = threadIdx.y; bg < nbg; bg += blockDim.y) {
    const int b = bg / n_kv, g = bg - b * n_kv;
    const uint2 lo4 = lo_n, hi4 = hi_n;
    if (bg + blockDim.y < nbg) {  // next row's loads before this row's math
      const uint16_t* src = row_src(bg + blockDim.y);
      lo_n = *(const uint2*)(src + i0);
      hi_n = *(const uint2*)(src + hd2 + i0);
    }
    const uint16_t lo[4] = {(uint16_t)lo4.x, (uint16_t)(lo4.x >> 16), (uint16_t)lo4.y,
                            (uint16_t)(lo4.y >> 16)};
    const uint16_t hi[4] = {(uint16_t)hi4.x, (uint16_t)(hi4.x >> 16), (uint16_t)hi4.y,
                            (uint16_t)(hi4.y >> 16)};
    const float* mn = mean + g * hd;
    float clo[4], chi[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float l = h2f(lo[j]), h = h2f(hi[j]);
      // undo_rope: k*cos - rotate_half(k)*sin, rotate_half = [-hi, lo]
      const float ulo = add_rn(mul_rn(l, p[j].x), mul_rn(h, p[j].y));
      const float uhi = sub_rn(mul_rn(h, p[j].x), mul_rn(l, p[j].y));
      clo[j] = sub_rn(ulo, mn[i0 + j]);
      chi[j] = sub_rn(uhi, mn[hd2 + i0 + j]);
    }
    OutT* o = out + ((int64_t)b * n_comp + t) * D + g * hd;
    if constexpr (sizeof(OutT) == 4) {
      *(float4*)(o + i0) = make_float4(clo[0], clo[1], clo[2], clo[3]);
      *(float4*)(o + hd2 + i0) = make_float4(chi[0], chi[1], chi[2], chi[3]);
    } else {
      uint16_t olo[4], ohi[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        olo[j] = f2h(clo[j]);
        ohi[j] = f2h(chi[j]);
      }
      *(uint2*)(o + i0) = make_uint2(olo[0] | ((uint32_t)olo[1] << 16), olo[2] | ((uint32_t)olo[3] << 16));
      *(uint2*)(o + hd2 + i0) =
          make_uint2(ohi[0] | ((uint32_t)ohi[1] << 16), ohi[2] | ((uint32_t)ohi[3] << 16));
    }
  }
}

template <typename OutT>
inline int k_prepare_launch(const uint16_t* k, int32_t batch, int32_t n_kv, int32_t seq, int32_t hd,
                            int32_t start, int32_t n_comp, const float* inv_freq, const float* mean,
                            OutT* out, void* stream, const char* name) {
  if (!k || !inv_freq || !mean || !out || batch <= 0 || n_kv <= 0 || n_comp <= 0) return SHARD_ERR_ARG;
  if ((hd & 7) || hd > 512 || start < 0 || start + n_comp > seq) return SHARD_ERR_SHAPE;
  // 8-byte input vectors, 4-element output vectors
  if (((uintptr_t)k & 7) || ((uintptr_t)out & (4 * sizeof(OutT) - 1))) return SHARD_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const int hd8 = hd / 8;
  const dim3 block(hd8, 256 / hd8 < 1 ? 1 : 256 / hd8);
  hipLaunchKernelGGL(k_k_prepare<OutT>, dim3((unsigned)n_comp), block, 0, s, k, batch, n_kv, seq, hd,
                     start, n_comp, inv_freq, mean, out);
  SHARD_LAUNCH_CHECK(name);
  return SHARD_OK;
}

}  // namespace shard

using namespace shard;

extern "C" {

size_t shard_int4_quant_pack_workspace(int64_t n_rows, int32_t keep) {
  if (n_rows <= 0 || keep <= 0) return 0;
  // pmin, pmax, pamax partials (kI4Blocks x keep), lo, rng (keep), the int4
  // table (keep x 256 bytes) and, for an odd keep (whose nibble pairs cross
  // rows: a separate packing pass), the group codes (n_rows x keep bytes)
  return (size_t)(3 * kI4Blocks + 2) * keep * sizeof(uint32_t) + (size_t)keep * 256 +
         ((keep & 1) ? (size_t)n_rows * keep : 0);
}

int shard_int4_quant_pack(const float* proj, int64_t n_rows, int32_t keep, const int32_t* bits,
                          uint8_t* packed, float* coeff_scale, float* lo, float* rng,
                          uint8_t* codes, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (!proj || !bits || !packed || !coeff_scale || n_rows <= 0 || keep <= 0) return SHARD_ERR_ARG;
  if (keep > 1024) return SHARD_ERR_SHAPE;
  if (!workspace || workspace_bytes < shard_int4_quant_pack_workspace(n_rows, keep))
    return SHARD_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  uint32_t* pmin = (uint32_t*)workspace;
  uint32_t* pmax = pmin + (size_t)kI4Blocks * keep;
  uint32_t* pamax = pmax + (size_t)kI4Blocks * keep;
  float* clo = (float*)(pamax + (size_t)kI4Blocks * keep);
  float* crng = clo + keep;
  int8_t* qtab = (int8_t*)(crng + keep);
  uint8_t* ccodes = codes ? codes : (uint8_t*)(qtab + (size_t)keep * 256);
  const int tpb = ((keep + 63) / 64) * 64;
  const int rg = 1024 / tpb < 4 ? 1024 / tpb : 4;
  const int64_t nblk = n_rows / rg < kI4Blocks ? (n_rows + rg - 1) / rg : kI4Blocks;
  const int64_t rpb = (n_rows + nblk - 1) / nblk;
  const dim3 cgrid((unsigned)nblk), cblock(tpb, rg);
  const dim3 fgrid((unsigned)((keep + 3) / 4)), fblock(256);  // a wave per column
  hipLaunchKernelGGL(k_int4_minmax, cgrid, cblock, 0, s, proj, n_rows, keep, rpb, pmin, pmax);
  if ((keep & 1) == 0) {
    // two passes over the projection: column min/max, then codes + packing
    hipLaunchKernelGGL(k_int4_fold, fgrid, fblock, 0, s, pmin, pmax, (int)nblk, keep, bits, clo,
                       crng, qtab, coeff_scale, lo, rng);
    // the element pass has no partials to bound its grid: slabs of 16 rows
    // per thread (two rounds of eight loads in flight), about one round of
    // workgroups at config 4's 32K rows
    const int words = (keep & 7) == 0 && ((uintptr_t)packed & 3) == 0;
    const int64_t pblk = grid_cap((n_rows + 16 * rg - 1) / (16 * rg), 1 << 20);
    const int64_t prpb = (n_rows + pblk - 1) / pblk;  // rows per block
#define SHARD_PACK(W, C)                                                                     \
  hipLaunchKernelGGL((k_int4_pack_rows<W, C>), dim3((unsigned)pblk), cblock, 0, s, proj, n_rows, \
                     keep, prpb, bits, clo, crng, qtab, codes, packed)
    if (words) {
      if (codes) SHARD_PACK(true, true); else SHARD_PACK(true, false);
    } else {
      if (codes) SHARD_PACK(false, true); else SHARD_PACK(false, false);
    }
#undef SHARD_PACK
    SHARD_LAUNCH_CHECK("shard_int4_quant_pack");
    return SHARD_OK;
  }
  hipLaunchKernelGGL(k_int4_fold_minmax, fgrid, fblock, 0, s, pmin, pmax, (int)nblk, keep, clo, crng);
  hipLaunchKernelGGL(k_int4_absmax, cgrid, cblock, 0, s, proj, n_rows, keep, rpb, bits, clo, crng,
                     pamax, ccodes);
  hipLaunchKernelGGL(k_int4_fold_absmax, fgrid, fblock, 0, s, pamax, (int)nblk, keep, bits, clo,
                     crng, qtab, coeff_scale, lo, rng);
  const int64_t total = n_rows * keep;
  const int64_t nquads = ((total + 1) / 2 + 3) / 4;
  const dim3 pgrid(grid_cap((nquads + 255) / 256, 8192));
  if (total < (1ll << 31))
    hipLaunchKernelGGL(k_int4_pack<uint32_t>, pgrid, dim3(256), 0, s, ccodes, (uint32_t)total, keep,
                       qtab, packed);
  else
    hipLaunchKernelGGL(k_int4_pack<uint64_t>, pgrid, dim3(256), 0, s, ccodes, (uint64_t)total, keep,
                       qtab, packed);
  SHARD_LAUNCH_CHECK("shard_int4_quant_pack");
  return SHARD_OK;
}

int shard_fwht(const float* x, float* y, int64_t rows, int32_t d, void* stream) {
  if (!x || !y || rows <= 0 || d < 2) return SHARD_ERR_ARG;
  if (d & (d - 1)) return SHARD_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  if (d < 64) {
    if (d > 32) return SHARD_ERR_SHAPE;
    hipLaunchKernelGGL(k_fwht_small, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, x, y,
                       rows, d);
  } else {
    int64_t waves = rows;
    int blocks = grid_cap((waves + 3) / 4, 4096);
    switch (d) {
      case 64: hipLaunchKernelGGL(k_fwht_rows<1>, dim3(blocks), dim3(256), 0, s, x, y, rows); break;
      case 128: hipLaunchKernelGGL(k_fwht_rows<2>, dim3(blocks), dim3(256), 0, s, x, y, rows); break;
      case 256: hipLaunchKernelGGL(k_fwht_rows<4>, dim3(blocks), dim3(256), 0, s, x, y, rows); break;
      case 512: hipLaunchKernelGGL(k_fwht_rows<8>, dim3(blocks), dim3(256), 0, s, x, y, rows); break;
      case 1024: hipLaunchKernelGGL(k_fwht_rows<16>, dim3(blocks), dim3(256), 0, s, x, y, rows); break;
      default: return SHARD_ERR_SHAPE;
    }
  }
  SHARD_LAUNCH_CHECK("shard_fwht");
  return SHARD_OK;
}

size_t shard_vq_prepare_workspace(int64_t bh, int32_t hd) {
  // kVqSlots channel-max partials per head, then the folded channel scales
  return (size_t)(kVqSlots + 1) * (bh > 0 ? bh : 0) * (hd > 0 ? hd : 0) * sizeof(float);
}

int shard_vq_prepare(const uint16_t* v, int64_t bh, int64_t seq, int32_t hd, int64_t v_bh_stride,
                     float* x_out, float* ch_f32, uint16_t* ch_f16, void* workspace,
                     size_t workspace_bytes, void* stream) {
  if (!v || !x_out || bh <= 0 || seq <= 0) return SHARD_ERR_ARG;
  if (hd != 64 && hd != 128 && hd != 256) return SHARD_ERR_SHAPE;
  // rows load as hd/64-half vectors and store as hd/64-float vectors
  const int E = hd / 64;
  if (((uintptr_t)v & (2 * E - 1)) || (v_bh_stride % E) || ((uintptr_t)x_out & (4 * E - 1)))
    return SHARD_ERR_SHAPE;
  if (!workspace || workspace_bytes < shard_vq_prepare_workspace(bh, hd)) return SHARD_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  float* ch = part + (size_t)kVqSlots * bh * hd;
  // workgroups per head: up to kVqSlots, at least 16 rows per wave
  const int64_t nx = (seq + 63) / 64 < kVqSlots ? (seq + 63) / 64 : kVqSlots;
  const dim3 rgrid((unsigned)nx, (unsigned)(bh < 65535 ? bh : 65535)), rblock(256);
  const dim3 fgrid((unsigned)(bh < 65535 ? bh : 65535)), fblock(256);
#define SHARD_VQ_PASSES(E)                                                                      \
  hipLaunchKernelGGL((k_vq_rot<E, false>), rgrid, rblock, 0, s, v, bh, seq, v_bh_stride, part,  \
                     (const float*)nullptr, (float*)nullptr);                                  \
  hipLaunchKernelGGL(k_vq_fold, fgrid, fblock, 0, s, part, bh, hd, (int)nx, ch, ch_f32, ch_f16); \
  hipLaunchKernelGGL((k_vq_rot<E, true>), rgrid, rblock, 0, s, v, bh, seq, v_bh_stride,         \
                     (float*)nullptr, (const float*)ch, x_out)
  switch (hd) {
    case 64: SHARD_VQ_PASSES(1); break;
    case 128: SHARD_VQ_PASSES(2); break;
    default: SHARD_VQ_PASSES(4); break;
  }
#undef SHARD_VQ_PASSES
  SHARD_LAUNCH_CHECK("shard_vq_prepare");
  return SHARD_OK;
}

int shard_vq_scales(const uint16_t* v, int64_t bh, int64_t seq, int32_t hd, int64_t v_bh_stride,
                    float* ch_f32, uint16_t* ch_f16, float* ch_rcp, void* workspace,
                    size_t workspace_bytes, void* stream) {
  if (!v || !ch_f32 || bh <= 0 || seq <= 0) return SHARD_ERR_ARG;
  if (hd != 64 && hd != 128 && hd != 256) return SHARD_ERR_SHAPE;
  const int E = hd / 64;
  if (((uintptr_t)v & (2 * E - 1)) || (v_bh_stride % E)) return SHARD_ERR_SHAPE;
  if (!workspace || workspace_bytes < shard_vq_prepare_workspace(bh, hd)) return SHARD_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  float* part = (float*)workspace;
  float* ch = part + (size_t)kVqSlots * bh * hd;
  const int64_t nx = (seq + 63) / 64 < kVqSlots ? (seq + 63) / 64 : kVqSlots;
  const dim3 rgrid((unsigned)nx, (unsigned)(bh < 65535 ? bh : 65535)), rblock(256);
  const dim3 fgrid((unsigned)(bh < 65535 ? bh : 65535)), fblock(256);
#define SHARD_VQ_PASS1(E)                                                                       \
  hipLaunchKernelGGL((k_vq_rot<E, false>), rgrid, rblock, 0, s, v, bh, seq, v_bh_stride, part,  \
                     (const float*)nullptr, (float*)nullptr)
  switch (hd) {
    case 64: SHARD_VQ_PASS1(1); break;
    case 128: SHARD_VQ_PASS1(2); break;
    default: SHARD_VQ_PASS1(4); break;
  }
#undef SHARD_VQ_PASS1
  hipLaunchKernelGGL(k_vq_fold, fgrid, fblock, 0, s, part, bh, hd, (int)nx, ch, ch_f32, ch_f16,
                     ch_rcp);
  SHARD_LAUNCH_CHECK("shard_vq_scales");
  return SHARD_OK;
}

// workspace of a table assignment: per wave of its launch an undecided-row
// count, then the waves' row regions, then (with values) their values
static size_t vq_list_bytes(int64_t n, bool with_x, VqList* lst, void* base) {
  int grid;
  int64_t per;
  vq_list_geometry(n, &grid, &per);
  const int64_t nwaves = (int64_t)grid * 4;
  const size_t counts = (size_t)((4 * nwaves + 15) & ~(int64_t)15);
  const size_t rows = (size_t)((4 * nwaves * per + 15) & ~(int64_t)15);
  if (lst) {
    char* b = (char*)base;
    lst->counts = (int32_t*)b;
    lst->rows = (int32_t*)(b + counts);
    lst->xs = with_x ? (float4*)(b + counts + rows) : nullptr;
    lst->per = per;
  }
  return counts + rows + (with_x ? (size_t)nwaves * per * 16 : 0);
}

size_t shard_vq_encode_table_workspace(int64_t n_rows) {
  if (n_rows <= 0 || n_rows >= ((int64_t)1 << 31)) return 0;
  return vq_list_bytes(n_rows, true, nullptr, nullptr);
}

int shard_vq_encode_table(const uint16_t* v, int64_t bh, int64_t seq, int32_t hd,
                          int64_t v_bh_stride, const float* ch_f32, const float* ch_rcp,
                          const float* centroids, int32_t k, const void* table, size_t table_bytes,
                          int32_t nbins, float lo, float hi, int32_t* idx, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (!v || !ch_f32 || !ch_rcp || !centroids || !table || !idx || bh <= 0 || seq <= 0)
    return SHARD_ERR_ARG;
  if (hd != 128) return SHARD_ERR_SHAPE;
  const int64_t n = bh * seq * 32;  // 4-value subvectors
  if (n >= ((int64_t)1 << 31)) return SHARD_ERR_SHAPE;
  if (k <= 0 || k > 256 || k % 32 || nbins < 1 || nbins > kVqTabMaxBins) return SHARD_ERR_SHAPE;
  if (((uintptr_t)v & 7) || (v_bh_stride % 4) || ((uintptr_t)ch_f32 & 15) ||
      ((uintptr_t)ch_rcp & 15) || ((uintptr_t)centroids & 15) || ((uintptr_t)table & 15))
    return SHARD_ERR_SHAPE;
  if (table_bytes < shard_vq_table_bytes(k, nbins)) return SHARD_ERR_WORKSPACE;
  if (!workspace || ((uintptr_t)workspace & 15) ||
      workspace_bytes < shard_vq_encode_table_workspace(n))
    return SHARD_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  VqList lst;
  vq_list_bytes(n, true, &lst, workspace);
  int grid;
  int64_t per;
  vq_list_geometry(n, &grid, &per);
  hipLaunchKernelGGL(k_vq_assign_table<true>, dim3(grid), dim3(256), 0, s, (const float*)nullptr,
                     n, centroids, (int)k, (const uint8_t*)table, (int)nbins, lo, hi, idx, lst,
                     VqFromV{v, seq, v_bh_stride, ch_f32, ch_rcp});
  hipLaunchKernelGGL(k_vq_list_direct<true>, dim3(64), dim3(256), 0, s, (const float*)nullptr,
                     centroids, (int)k, idx, lst, 4 * grid);
  SHARD_LAUNCH_CHECK("shard_vq_encode_table");
  return SHARD_OK;
}

int shard_vq_assign(const float* x, int64_t n, int32_t d, const float* centroids, int32_t k,
                    int32_t* idx, void* stream) {
  if (!x || !centroids || !idx || n <= 0 || k <= 0 || d <= 0) return SHARD_ERR_ARG;
  if (k > 1024 || d > 8) return SHARD_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  if (d == 4 && k % 32 == 0 && k <= 256 && ((uintptr_t)x & 15) == 0 &&
      ((uintptr_t)centroids & 15) == 0) {
    const int64_t groups = (n + 31) / 32;  // 32 rows per wave
    const dim3 grid(grid_cap((groups + 3) / 4, 2048)), block(256);
    switch (k / 32) {
      case 1: hipLaunchKernelGGL(k_vq_assign_mfma<1>, grid, block, 0, s, x, n, centroids, idx); break;
      case 2: hipLaunchKernelGGL(k_vq_assign_mfma<2>, grid, block, 0, s, x, n, centroids, idx); break;
      case 3: hipLaunchKernelGGL(k_vq_assign_mfma<3>, grid, block, 0, s, x, n, centroids, idx); break;
      case 4: hipLaunchKernelGGL(k_vq_assign_mfma<4>, grid, block, 0, s, x, n, centroids, idx); break;
      case 5: hipLaunchKernelGGL(k_vq_assign_mfma<5>, grid, block, 0, s, x, n, centroids, idx); break;
      case 6: hipLaunchKernelGGL(k_vq_assign_mfma<6>, grid, block, 0, s, x, n, centroids, idx); break;
      case 7: hipLaunchKernelGGL(k_vq_assign_mfma<7>, grid, block, 0, s, x, n, centroids, idx); break;
      default: hipLaunchKernelGGL(k_vq_assign_mfma<8>, grid, block, 0, s, x, n, centroids, idx); break;
    }
    SHARD_LAUNCH_CHECK("shard_vq_assign");
    return SHARD_OK;
  }
  int blocks = grid_cap((n + 255) / 256, 8192);
  size_t lds = (size_t)k * d * sizeof(float);
  switch (d) {
    case 1: hipLaunchKernelGGL(k_vq_assign<1>, dim3(blocks), dim3(256), lds, s, x, n, centroids, k, idx); break;
    case 2: hipLaunchKernelGGL(k_vq_assign<2>, dim3(blocks), dim3(256), lds, s, x, n, centroids, k, idx); break;
    case 4: hipLaunchKernelGGL(k_vq_assign<4>, dim3(blocks), dim3(256), lds, s, x, n, centroids, k, idx); break;
    case 8: hipLaunchKernelGGL(k_vq_assign<8>, dim3(blocks), dim3(256), lds, s, x, n, centroids, k, idx); break;
    default: return SHARD_ERR_SHAPE;
  }
  SHARD_LAUNCH_CHECK("shard_vq_assign");
  return SHARD_OK;
}

size_t shard_vq_table_bytes(int32_t k, int32_t nbins) {
  if (k <= 0 || k > 256 || nbins < 1 || nbins > kVqTabMaxBins) return 0;
  return (size_t)(kVqTabHeader + vq_tab_counts_bytes(nbins) + vq_tab_cells(nbins) * kVqTabCap);
}

int shard_vq_table_build(const float* centroids, int32_t k, float lo, float hi, int32_t nbins,
                         void* table, size_t table_bytes, void* stream) {
  if (!centroids || !table) return SHARD_ERR_ARG;
  if (k <= 0 || k > 256 || k % 32 || nbins < 1 || nbins > kVqTabMaxBins) return SHARD_ERR_SHAPE;
  if (!(std::isfinite(lo) && std::isfinite(hi) && hi > lo)) return SHARD_ERR_ARG;
  if (std::max(std::fabs(lo), std::fabs(hi)) > 64.f * (hi - lo)) return SHARD_ERR_ARG;
  if (((uintptr_t)centroids & 15) || ((uintptr_t)table & 15)) return SHARD_ERR_SHAPE;
  if (table_bytes < shard_vq_table_bytes(k, nbins)) return SHARD_ERR_WORKSPACE;
  const int64_t cells = vq_tab_cells(nbins);
  hipLaunchKernelGGL(k_vq_table_build, dim3((unsigned)((cells + kVqTabCells - 1) / kVqTabCells)),
                     dim3(4 * kVqTabCells), 0,
                     (hipStream_t)stream, centroids, k, lo, hi, nbins, (uint8_t*)table);
  SHARD_LAUNCH_CHECK("shard_vq_table_build");
  return SHARD_OK;
}

size_t shard_vq_assign_table_workspace(int64_t n) {
  if (n <= 0 || n >= ((int64_t)1 << 31)) return 0;
  return vq_list_bytes(n, false, nullptr, nullptr);
}

int shard_vq_assign_table(const float* x, int64_t n, const float* centroids, int32_t k,
                          const void* table, size_t table_bytes, int32_t nbins, float lo,
                          float hi, int32_t* idx, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (!x || !centroids || !table || !idx || n <= 0) return SHARD_ERR_ARG;
  if (n >= ((int64_t)1 << 31)) return SHARD_ERR_SHAPE;
  if (k <= 0 || k > 256 || k % 32 || nbins < 1 || nbins > kVqTabMaxBins) return SHARD_ERR_SHAPE;
  if (((uintptr_t)x & 15) || ((uintptr_t)centroids & 15) || ((uintptr_t)table & 15))
    return SHARD_ERR_SHAPE;
  if (table_bytes < shard_vq_table_bytes(k, nbins)) return SHARD_ERR_WORKSPACE;
  if (!workspace || ((uintptr_t)workspace & 15) ||
      workspace_bytes < shard_vq_assign_table_workspace(n))
    return SHARD_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  VqList lst;
  vq_list_bytes(n, false, &lst, workspace);
  int grid;
  int64_t per;
  vq_list_geometry(n, &grid, &per);
  hipLaunchKernelGGL(k_vq_assign_table<false>, dim3(grid), dim3(256), 0, s, x, n, centroids,
                     (int)k, (const uint8_t*)table, (int)nbins, lo, hi, idx, lst, VqFromV{});
  // the rows the table left undecided (usually none)
  hipLaunchKernelGGL(k_vq_list_direct<false>, dim3(64), dim3(256), 0, s, x, centroids, (int)k,
                     idx, lst, 4 * grid);
  SHARD_LAUNCH_CHECK("shard_vq_assign_table");
  return SHARD_OK;
}

size_t shard_kmeans_update_workspace_d(int64_t n, int32_t k, int32_t d) {
  if (n <= 0 || k <= 0 || d <= 0 || d > KM_DMAX) return 0;
  const int64_t nblk = (n + KM_R - 1) / KM_R;
  // per-block counts, counts, offsets, then the sorted copy of the rows
  const int64_t ints = ((nblk * k + 2 * (int64_t)k) + 3) & ~(int64_t)3;
  return (size_t)ints * sizeof(int32_t) + (size_t)n * d * sizeof(float);
}

size_t shard_kmeans_update_workspace(int64_t n, int32_t k) {
  return shard_kmeans_update_workspace_d(n, k, KM_DMAX);
}

int shard_kmeans_update(const float* x, int64_t n, int32_t d, const int32_t* idx,
                        const float* centroids, int32_t k, float* new_centroids,
                        float* max_delta, void* workspace, size_t workspace_bytes,
                        void* stream) {
  if (!x || !idx || !centroids || !new_centroids || !max_delta || n <= 0 || k <= 0)
    return SHARD_ERR_ARG;
  if (k > 1024 || (d != 1 && d != 2 && d != 4 && d != 8)) return SHARD_ERR_SHAPE;
  if (n > INT32_MAX) return SHARD_ERR_SHAPE;  // slots are int32
  if (!workspace || workspace_bytes < shard_kmeans_update_workspace_d(n, k, d)) return SHARD_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  const int64_t nblk = (n + KM_R - 1) / KM_R;
  int32_t* blk = (int32_t*)workspace;
  int32_t* count = blk + nblk * k;
  int32_t* off = count + k;
  float* xs = (float*)(blk + (((nblk * k + 2 * (int64_t)k) + 3) & ~(int64_t)3));
  hipLaunchKernelGGL(k_km_hist, dim3((unsigned)nblk), dim3(256), 0, s, idx, n, k, nblk, blk);
  hipLaunchKernelGGL(k_km_scan_blocks, dim3((unsigned)k), dim3(256), 0, s, blk, nblk, count);
  hipLaunchKernelGGL(k_km_offsets, dim3(1), dim3(64), 0, s, count, k, off);
  hipLaunchKernelGGL(k_km_zero, dim3(1), dim3(1), 0, s, (uint32_t*)max_delta);
  const unsigned kb = (unsigned)k, nb = (unsigned)nblk;
  switch (d) {
    case 1:
      hipLaunchKernelGGL(k_km_scatter<1>, dim3(nb), dim3(64), 0, s, x, idx, n, k, nblk, blk, off, xs);
      hipLaunchKernelGGL(k_km_sum<1>, dim3(kb), dim3(256), 0, s, xs, count, off, centroids, k, new_centroids, (uint32_t*)max_delta);
      break;
    case 2:
      hipLaunchKernelGGL(k_km_scatter<2>, dim3(nb), dim3(64), 0, s, x, idx, n, k, nblk, blk, off, xs);
      hipLaunchKernelGGL(k_km_sum<2>, dim3(kb), dim3(256), 0, s, xs, count, off, centroids, k, new_centroids, (uint32_t*)max_delta);
      break;
    case 4:
      hipLaunchKernelGGL(k_km_scatter<4>, dim3(nb), dim3(64), 0, s, x, idx, n, k, nblk, blk, off, xs);
      hipLaunchKernelGGL(k_km_sum<4>, dim3(kb), dim3(256), 0, s, xs, count, off, centroids, k, new_centroids, (uint32_t*)max_delta);
      break;
    default:
      hipLaunchKernelGGL(k_km_scatter<8>, dim3(nb), dim3(64), 0, s, x, idx, n, k, nblk, blk, off, xs);
      hipLaunchKernelGGL(k_km_sum<8>, dim3(kb), dim3(256), 0, s, xs, count, off, centroids, k, new_centroids, (uint32_t*)max_delta);
      break;
  }
  SHARD_LAUNCH_CHECK("shard_kmeans_update");
  return SHARD_OK;
}

static int stream_quant_launch(const StreamIO& io, int jobs, int64_t rows, int32_t hd,
                               const float* signs, const float* codebook, int32_t n_codes,
                               void* stream) {
  if (!signs || !codebook || rows <= 0 || n_codes <= 0) return SHARD_ERR_ARG;
  for (int j = 0; j < jobs; ++j) {
    if (!io.x[j] || !io.idx[j] || !io.norm[j]) return SHARD_ERR_ARG;
    if ((io.qsign[j] == nullptr) != (io.qscale[j] == nullptr)) return SHARD_ERR_ARG;
  }
  if (n_codes > 256) return SHARD_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((rows + 3) / 4), (unsigned)jobs);
  switch (hd) {
    case 64: hipLaunchKernelGGL(k_stream_quant<1>, grid, dim3(256), 0, s, io, rows, signs, codebook, n_codes); break;
    case 128: hipLaunchKernelGGL(k_stream_quant<2>, grid, dim3(256), 0, s, io, rows, signs, codebook, n_codes); break;
    case 256: hipLaunchKernelGGL(k_stream_quant<4>, grid, dim3(256), 0, s, io, rows, signs, codebook, n_codes); break;
    default: return SHARD_ERR_SHAPE;
  }
  SHARD_LAUNCH_CHECK("shard_stream_quant");
  return SHARD_OK;
}

int shard_stream_quant_qjl(const uint16_t* x, int64_t rows, int32_t hd, const float* signs,
                           const float* codebook, int32_t n_codes, uint8_t* idx, uint16_t* norm,
                           uint8_t* qsign, uint16_t* qscale, uint16_t* deq, void* stream) {
  const StreamIO io = {{x, nullptr}, {idx, nullptr}, {norm, nullptr},
                       {qsign, nullptr}, {qscale, nullptr}, {deq, nullptr}};
  return stream_quant_launch(io, 1, rows, hd, signs, codebook, n_codes, stream);
}

static int rope_stream_launch(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint16_t* cos, const uint16_t* sin, int64_t cos_stride,
                              int32_t batch, int32_t n_q_heads, int32_t n_kv_heads, int32_t hd,
                              uint16_t* q_rope, const float* signs, const float* codebook,
                              int32_t n_codes, uint8_t* k_idx, uint16_t* k_norm, uint16_t* k_deq,
                              uint8_t* v_idx, uint16_t* v_norm, uint16_t* v_deq,
                              uint8_t* k_qsign, uint16_t* k_qscale, uint8_t* v_qsign,
                              uint16_t* v_qscale, const int32_t* row_dev, int32_t row_cap,
                              void* stream) {
  if (!q || !k || !v || !cos || !sin || !q_rope || !signs || !codebook || !k_idx || !k_norm ||
      !v_idx || !v_norm)
    return SHARD_ERR_ARG;
  if (batch <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || n_codes <= 0) return SHARD_ERR_ARG;
  if (cos_stride != 0 && cos_stride < hd) return SHARD_ERR_SHAPE;
  if ((k_qsign == nullptr) != (k_qscale == nullptr) || (v_qsign == nullptr) != (v_qscale == nullptr))
    return SHARD_ERR_ARG;
  if (n_codes > 256) return SHARD_ERR_SHAPE;
  const StreamIO io = {{k, v}, {k_idx, v_idx}, {k_norm, v_norm},
                       {k_qsign, v_qsign}, {k_qscale, v_qscale}, {k_deq, v_deq}};
  hipStream_t s = (hipStream_t)stream;
  const int64_t rows = (int64_t)batch * (n_q_heads + 2 * n_kv_heads);
  const dim3 grid((unsigned)((rows + 3) / 4));
  switch (hd) {
    case 64: hipLaunchKernelGGL(k_rope_stream<1>, grid, dim3(256), 0, s, q, k, v, cos, sin, cos_stride, batch, n_q_heads, n_kv_heads, q_rope, io, signs, codebook, n_codes, row_dev, row_cap); break;
    case 128: hipLaunchKernelGGL(k_rope_stream<2>, grid, dim3(256), 0, s, q, k, v, cos, sin, cos_stride, batch, n_q_heads, n_kv_heads, q_rope, io, signs, codebook, n_codes, row_dev, row_cap); break;
    case 256: hipLaunchKernelGGL(k_rope_stream<4>, grid, dim3(256), 0, s, q, k, v, cos, sin, cos_stride, batch, n_q_heads, n_kv_heads, q_rope, io, signs, codebook, n_codes, row_dev, row_cap); break;
    default: return SHARD_ERR_SHAPE;
  }
  SHARD_LAUNCH_CHECK("shard_rope_stream_append");
  return SHARD_OK;
}

int shard_rope_stream_append(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             const uint16_t* cos, const uint16_t* sin, int64_t cos_stride,
                             int32_t batch,
                             int32_t n_q_heads, int32_t n_kv_heads, int32_t hd,
                             uint16_t* q_rope, const float* signs, const float* codebook,
                             int32_t n_codes, uint8_t* k_idx, uint16_t* k_norm, uint16_t* k_deq,
                             uint8_t* v_idx, uint16_t* v_norm, uint16_t* v_deq,
                             uint8_t* k_qsign, uint16_t* k_qscale, uint8_t* v_qsign,
                             uint16_t* v_qscale, void* stream) {
  return rope_stream_launch(q, k, v, cos, sin, cos_stride, batch, n_q_heads, n_kv_heads, hd,
                            q_rope, signs, codebook, n_codes, k_idx, k_norm, k_deq, v_idx,
                            v_norm, v_deq, k_qsign, k_qscale, v_qsign, v_qscale, nullptr, 0,
                            stream);
}

int shard_rope_stream_append_dev(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* cos, const uint16_t* sin, int64_t cos_stride,
                                 int32_t batch, int32_t n_q_heads, int32_t n_kv_heads, int32_t hd,
                                 uint16_t* q_rope, const float* signs, const float* codebook,
                                 int32_t n_codes, uint8_t* k_idx, uint16_t* k_norm,
                                 uint16_t* k_deq, uint8_t* v_idx, uint16_t* v_norm,
                                 uint16_t* v_deq, uint8_t* k_qsign, uint16_t* k_qscale,
                                 uint8_t* v_qsign, uint16_t* v_qscale, const int32_t* row_dev,
                                 int32_t row_cap, void* stream) {
  if (!row_dev || row_cap <= 0) return SHARD_ERR_ARG;
  return rope_stream_launch(q, k, v, cos, sin, cos_stride, batch, n_q_heads, n_kv_heads, hd,
                            q_rope, signs, codebook, n_codes, k_idx, k_norm, k_deq, v_idx,
                            v_norm, v_deq, k_qsign, k_qscale, v_qsign, v_qscale, row_dev,
                            row_cap, stream);
}

int shard_stream_quant_kv(const uint16_t* k, const uint16_t* v, int64_t rows, int32_t hd,
                          const float* signs, const float* codebook, int32_t n_codes,
                          uint8_t* k_idx, uint16_t* k_norm, uint16_t* k_deq,
                          uint8_t* v_idx, uint16_t* v_norm, uint16_t* v_deq,
                          uint8_t* k_qsign, uint16_t* k_qscale, uint8_t* v_qsign,
                          uint16_t* v_qscale, void* stream) {
  const StreamIO io = {{k, v}, {k_idx, v_idx}, {k_norm, v_norm},
                       {k_qsign, v_qsign}, {k_qscale, v_qscale}, {k_deq, v_deq}};
  return stream_quant_launch(io, 2, rows, hd, signs, codebook, n_codes, stream);
}

int shard_stream_quant(const uint16_t* x, int64_t rows, int32_t hd, const float* signs,
                       const float* codebook, int32_t n_codes, uint8_t* idx, uint16_t* norm,
                       uint16_t* deq, void* stream) {
  return shard_stream_quant_qjl(x, rows, hd, signs, codebook, n_codes, idx, norm, nullptr, nullptr,
                                deq, stream);
}

int shard_k_prepare(const uint16_t* k, int32_t batch, int32_t n_kv, int32_t seq, int32_t hd,
                    int32_t start, int32_t n_comp, const float* inv_freq, const float* mean,
                    uint16_t* out, void* stream) {
  return k_prepare_launch(k, batch, n_kv, seq, hd, start, n_comp, inv_freq, mean, out, stream,
                          "shard_k_prepare");
}

int shard_k_prepare_f32(const uint16_t* k, int32_t batch, int32_t n_kv, int32_t seq, int32_t hd,
                        int32_t start, int32_t n_comp, const float* inv_freq, const float* mean,
                        float* out, void* stream) {
  return k_prepare_launch(k, batch, n_kv, seq, hd, start, n_comp, inv_freq, mean, out, stream,
                          "shard_k_prepare_f32");
}

}  // extern "C"
