// PCA projection GEMM of prefill compression on gfx950 MFMA:
//   C[m, n] (fp32) = A[m, k] (fp16, row-major) . Bt[n, k]^T (fp16, row-major)
// Workgroup = 8 waves, one 128-row tile of A and all n <= 256 columns: wave w
// owns rows 32 (w % 4) .. + 32 and column half w / 4 (n/32 accumulator blocks
// of v_mfma_f32_32x32x16_f16 split over the two halves), so every SIMD runs
// two waves.  The basis side Bt is small and read by every workgroup: it is
// staged in LDS 64 k at a time, double-buffered; both its pieces and the A
// fragments are loaded into registers three chunks ahead (a 4-slot ring), so
// L2 and HBM latency hide behind the MFMAs of the chunks in between; one
// barrier per chunk.  All global loads are raw buffer loads whose bounds
// (rows past m, k past the row end) are handled by an out-of-range offset that
// the hardware answers with zeros: no load sits under a branch, so the
// compiler's wait counters stay exact and a chunk waits only for its own data.
#include <algorithm>

#include "common.h"

namespace shard {

constexpr int kPcaThreads = 512;
constexpr int kPcaRows = 128;
#ifndef SHARD_PCA_KC
#define SHARD_PCA_KC 64
#endif
constexpr int kKc = SHARD_PCA_KC;  // k chunk staged in LDS
// buffer resource word 3 for raw (untyped, unswizzled) dword access on gfx9
constexpr int kBufWord3 = 0x00020000;
constexpr int kOutOfRange = 0x7fffff00;  // a byte offset past every buffer here

template <int NB32>
__global__ __launch_bounds__(kPcaThreads, 1)
void k_pca_project(const uint16_t* __restrict__ A, int64_t m, int k, int64_t lda,
                   const uint16_t* __restrict__ Bt, float* __restrict__ C, int64_t ldc) {
  constexpr int kRowStride = kKc + 8;            // halves per staged row (bank spread)
  constexpr int NH = (NB32 + 1) / 2;             // column blocks per wave half
  constexpr int kPieces = NB32 * 32 * (kKc / 8);  // 16-byte pieces of one Bt chunk
  constexpr int kPer = (kPieces + kPcaThreads - 1) / kPcaThreads;
  __shared__ __align__(16) uint16_t bs[2][NB32 * 32 * kRowStride];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rw = w & 3, half = w >> 2;
  const int col = lane & 31, hh = lane >> 5;
  const int j0 = half * NH;
  const int nj = NB32 - j0 < NH ? NB32 - j0 : NH;  // this wave's column blocks
  const int64_t blk0 = (int64_t)blockIdx.x * kPcaRows;
  const int64_t row0 = blk0 + 32 * rw;
  // buffer resources: this workgroup's rows of A, and all of Bt (byte sizes
  // < 2^31, checked by the host); offsets at or past the size read as zero
  const int64_t nrows = m - blk0 < kPcaRows ? m - blk0 : kPcaRows;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A + blk0 * lda), (short)0, (int)(nrows * lda * 2), kBufWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)Bt, (short)0, NB32 * 32 * k * 2, kBufWord3);
  const int a_off = (32 * rw + col) * (int)lda * 2;  // byte offset of this lane's A row
  const int nc = (k + kKc - 1) / kKc;

  auto load_b = [&](int c, uint4 (&pb)[kPer]) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int pc = tid + kPcaThreads * u;
      const int r = pc / (kKc / 8), kk = kKc * c + 8 * (pc % (kKc / 8));
      const int off = (pc < kPieces && kk < k) ? (r * k + kk) * 2 : kOutOfRange;
      pb[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
    }
  };
  auto store_b = [&](int buf, const uint4 (&pb)[kPer]) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int pc = tid + kPcaThreads * u;
      if (pc < kPieces) *(uint4*)(&bs[buf][(pc / (kKc / 8)) * kRowStride + 8 * (pc % (kKc / 8))]) = pb[u];
    }
  };
  auto load_a = [&](int c, half8 (&af)[kKc / 16]) {
#pragma unroll
    for (int s = 0; s < kKc / 16; ++s) {
      const int kk = kKc * c + 16 * s + 8 * hh;
      const int off = kk < k ? a_off + kk * 2 : kOutOfRange;
      af[s] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
    }
  };

  float16v acc[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j) acc[j] = {};

  // ring: chunk c's basis pieces and A fragments live in slot c % 4
  uint4 pb[4][kPer];
  half8 af[4][kKc / 16];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    load_b(d, pb[d]);
    load_a(d, af[d]);
  }
  store_b(0, pb[0]);
  __syncthreads();

  // chunk c: MFMAs from LDS buffer c & 1; then chunk c + 1's pieces into the
  // other buffer (last read in iteration c - 1) and chunk c + 3's loads into
  // the slot chunk c - 1 used.  The chunk count is rounded up to a multiple of
  // the ring length: chunks past k read zeros (out-of-range offsets) and add
  // exact zeros, so the loop body is one straight-line block and the
  // compiler's wait counts name exactly the chunk being consumed.
  auto step = [&](const int c, const half8 (&a)[kKc / 16], half8 (&a3)[kKc / 16],
                  const uint4 (&b1)[kPer], uint4 (&b3)[kPer]) {
    const uint16_t* b = bs[c & 1];
#pragma unroll
    for (int s = 0; s < kKc / 16; ++s) {
#pragma unroll
      for (int jj = 0; jj < NH; ++jj) {
        if (NB32 % 2 == 0 || jj < nj) {
          const uint4 bv = *(const uint4*)(b + (32 * (j0 + jj) + col) * kRowStride + 16 * s + 8 * hh);
          acc[jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[s], __builtin_bit_cast(half8, bv), acc[jj], 0, 0, 0);
        }
      }
    }
    store_b((c + 1) & 1, b1);
    load_b(c + 3, b3);
    load_a(c + 3, a3);
    __syncthreads();
  };
  const int nc4 = (nc + 3) & ~3;
  for (int c0 = 0; c0 < nc4; c0 += 4) {
    step(c0, af[0], af[3], pb[1], pb[3]);
    step(c0 + 1, af[1], af[0], pb[2], pb[0]);
    step(c0 + 2, af[2], af[1], pb[3], pb[1]);
    step(c0 + 3, af[3], af[2], pb[0], pb[2]);
  }
  // C layout of the 32x32 block: lane (col, hh), reg i -> row 8*(i/4) + 4*hh + i%4
#pragma unroll
  for (int jj = 0; jj < NH; ++jj) {
    if (jj < nj) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t r = row0 + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (r < m) C[r * ldc + 32 * (j0 + jj) + col] = acc[jj][i];
      }
    }
  }
}

// The same GEMM in fp32 (C = A . Bt^T with fp32 A and Bt): the projection of
// _compress_k in the reference's own arithmetic (cache.py:389-392 projects
// (flat - mean) @ (basis_q * scale) with fp32 operands).  v_mfma_f32_32x32x2_f32
// multiplies fp32 operands with an fp32 sum, so the projection differs from a
// sequential fp32 dot product only by the order of its roundings.
// Same workgroup shape as k_pca_project (8 waves, 128 rows, two column
// halves).  A k step of the MFMA takes k pairs {k0 + j, k0 + 4 + j} from the
// two lane halves: lane (row, hh) loads A[row][k0 + 4 hh .. + 3] as one 16-byte
// vector and feeds element j to step j, and the B side (from LDS) follows the
// same order, so four MFMAs consume 8 consecutive k.  Bt is staged in LDS 32 k
// at a time, double-buffered, with A and the Bt pieces loaded three chunks
// ahead into a 4-slot register ring (raw buffer loads, out-of-range offsets
// read zeros, as in k_pca_project).
template <int NB32>
__global__ __launch_bounds__(kPcaThreads, 1)
void k_pca_project_f32(const float* __restrict__ A, int64_t m, int k, int64_t lda,
                       const float* __restrict__ Bt, float* __restrict__ C, int64_t ldc) {
  constexpr int KC = 32;                          // k chunk staged in LDS
  constexpr int kRowStride = KC + 4;              // floats per staged row (bank spread)
  constexpr int NH = (NB32 + 1) / 2;              // column blocks per wave half
  constexpr int kPieces = NB32 * 32 * (KC / 4);   // 16-byte pieces of one Bt chunk
  constexpr int kPer = (kPieces + kPcaThreads - 1) / kPcaThreads;
  __shared__ __align__(16) float bs[2][NB32 * 32 * kRowStride];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rw = w & 3, half = w >> 2;
  const int col = lane & 31, hh = lane >> 5;
  const int j0 = half * NH;
  const int nj = NB32 - j0 < NH ? NB32 - j0 : NH;
  const int64_t blk0 = (int64_t)blockIdx.x * kPcaRows;
  const int64_t row0 = blk0 + 32 * rw;
  const int64_t nrows = m - blk0 < kPcaRows ? m - blk0 : kPcaRows;
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(A + blk0 * lda), (short)0, (int)(nrows * lda * 4), kBufWord3);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)Bt, (short)0, NB32 * 32 * k * 4, kBufWord3);
  const int a_off = (32 * rw + col) * (int)lda * 4;
  const int nc = (k + KC - 1) / KC;

  auto load_b = [&](int c, float4v (&pb)[kPer]) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int pc = tid + kPcaThreads * u;
      const int r = pc / (KC / 4), kk = KC * c + 4 * (pc % (KC / 4));
      const int off = (pc < kPieces && kk < k) ? (r * k + kk) * 4 : kOutOfRange;
      pb[u] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
    }
  };
  auto store_b = [&](int buf, const float4v (&pb)[kPer]) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int pc = tid + kPcaThreads * u;
      if (pc < kPieces) *(float4v*)(&bs[buf][(pc / (KC / 4)) * kRowStride + 4 * (pc % (KC / 4))]) = pb[u];
    }
  };
  auto load_a = [&](int c, float4v (&af)[KC / 8]) {
#pragma unroll
    for (int s = 0; s < KC / 8; ++s) {
      const int kk = KC * c + 8 * s + 4 * hh;
      const int off = kk < k ? a_off + kk * 4 : kOutOfRange;
      af[s] = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
    }
  };

  float16v acc[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j) acc[j] = {};

  float4v pb[4][kPer];
  float4v af[4][KC / 8];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    load_b(d, pb[d]);
    load_a(d, af[d]);
  }
  store_b(0, pb[0]);
  __syncthreads();

  auto step = [&](const int c, const float4v (&a)[KC / 8], float4v (&a3)[KC / 8],
                  const float4v (&b1)[kPer], float4v (&b3)[kPer]) {
    const float* b = bs[c & 1];
#pragma unroll
    for (int s = 0; s < KC / 8; ++s) {
#pragma unroll
      for (int jj = 0; jj < NH; ++jj) {
        if (NB32 % 2 == 0 || jj < nj) {
          const float4v bv = *(const float4v*)(b + (32 * (j0 + jj) + col) * kRowStride + 8 * s + 4 * hh);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s][j], bv[j], acc[jj], 0, 0, 0);
        }
      }
    }
    store_b((c + 1) & 1, b1);
    load_b(c + 3, b3);
    load_a(c + 3, a3);
    __syncthreads();
  };
  const int nc4 = (nc + 3) & ~3;
  for (int c0 = 0; c0 < nc4; c0 += 4) {
    step(c0, af[0], af[3], pb[1], pb[3]);
    step(c0 + 1, af[1], af[0], pb[2], pb[0]);
    step(c0 + 2, af[2], af[1], pb[3], pb[1]);
    step(c0 + 3, af[3], af[2], pb[0], pb[2]);
  }
#pragma unroll
  for (int jj = 0; jj < NH; ++jj) {
    if (jj < nj) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t r = row0 + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (r < m) C[r * ldc + 32 * (j0 + jj) + col] = acc[jj][i];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The fp16 projection with its front end fused: A is undo-RoPE of post-RoPE
// keys read straight from the K cache layout (B, G, T, 128) fp16, so the fp16
// operand of k_k_prepare is never written.  Row r = b * n_comp + t takes the
// token at position start + t; its undo rotation uses the phase table
// (cos, sin)(fl(pos * inv_freq[i])) of k_rope_phases (the phases k_k_prepare
// computes) and k_k_prepare's arithmetic (this file is built without fp
// contraction, so the fp16 operand is bit-identical to k_k_prepare's).
// Workgroup shape as k_pca_project (8 waves, 128 rows, two column halves).
// The k order is permuted so that one lane's 8-element MFMA fragment holds 4
// dims of the low half of a head and their 4 RoPE partners of the high half:
// chunk c (64 k) = head c / 2, pairs 32 (c % 2) .. + 31 (a head's first pair
// half, then its second: the two chunks of a head read the two halves of the
// same 128-byte lines of each key row, so every line is fetched from HBM
// once), k step s = 2 j + o and lane half hh: element e is dim d0 + 4 o + e
// (e < 4) or 64 + d0 + 4 o + e - 4 (e >= 4), d0 = 32 (c % 2) + 16 j + 8 hh.
// Btp holds the basis columns in that order (the host permutes them once).
// The phases of the workgroup's 128 rows sit in LDS (the same in every head);
// a lane reads the 16 of its chunk's pair half before the chunk's undo.
// C = fp16(undo(k)) . Btp^T - bias (bias: mean . basis, nullable).  Btp is
// staged in LDS 64 k at a time, double-buffered; the keys and the Btp pieces
// are loaded R - 1 chunks ahead into an R-slot register ring.
constexpr int kRopePairs = 64;  // head_dim 128
constexpr int kPhStride = kRopePairs + 2;  // float2 per staged row: rows 4 banks apart
#ifndef SHARD_ROPE_RING
#define SHARD_ROPE_RING 4
#endif

template <int NB32>
__global__ __launch_bounds__(kPcaThreads, 1)
void k_pca_project_rope(const uint16_t* __restrict__ K, int n_kv, int seq, int start, int n_comp,
                        int64_t m, const float2* __restrict__ phases,
                        const uint16_t* __restrict__ Btp, const float* __restrict__ bias,
                        float* __restrict__ C, int64_t ldc) {
  constexpr int kRowStride = kKc + 8;
  constexpr int NH = (NB32 + 1) / 2;
  constexpr int kPieces = NB32 * 32 * (kKc / 8);
  constexpr int kPer = (kPieces + kPcaThreads - 1) / kPcaThreads;
  constexpr int R = SHARD_ROPE_RING;
  static_assert(kKc == 64, "a chunk is half a head: 32 RoPE pairs");
  static_assert(R == 4, "a ring of 4 slots: each step's pair half (c % 2) is static");
  __shared__ __align__(16) uint16_t bs[2][NB32 * 32 * kRowStride];
  __shared__ __align__(16) float2 phs[kPcaRows * kPhStride];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rw = w & 3, half = w >> 2;
  const int col = lane & 31, hh = lane >> 5;
  const int j0 = half * NH;
  const int nj = NB32 - j0 < NH ? NB32 - j0 : NH;
  const int k = n_kv * 128;
  const int64_t blk0 = (int64_t)blockIdx.x * kPcaRows;
  const int64_t row0 = blk0 + 32 * rw;
  // this lane's A row (clamped past m: its loads stay in bounds, never stored)
  const int64_t r = row0 + col < m ? row0 + col : m - 1;
  const int64_t bb = r / n_comp, t = r - bb * n_comp;
  const uint16_t* krow = K + ((bb * n_kv) * (int64_t)seq + start + t) * 128 + 8 * hh;  // head 0
  const int64_t head_stride = (int64_t)seq * 128;
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)Btp, (short)0, NB32 * 32 * k * 2, kBufWord3);
  const int nc = k / kKc;

  // the phases of the workgroup's rows (rows past m take row m - 1's) into
  // LDS: 128 rows x 64 pairs, 8 float4 per thread
#pragma unroll
  for (int u = 0; u < kPcaRows * kRopePairs / 2 / kPcaThreads; ++u) {
    const int pc = tid + kPcaThreads * u;
    const int lr = pc / (kRopePairs / 2), pq = pc % (kRopePairs / 2);
    const int64_t gr = blk0 + lr < m ? blk0 + lr : m - 1;
    const int64_t tt = gr - gr / n_comp * n_comp;
    *(float4*)&phs[lr * kPhStride + 2 * pq] = *(const float4*)(phases + tt * kRopePairs + 2 * pq);
  }
  const float2* myph = phs + (32 * rw + col) * kPhStride + 8 * hh;

  auto load_b = [&](int c, uint4 (&pb)[kPer]) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int pc = tid + kPcaThreads * u;
      const int rr = pc / (kKc / 8), kk = kKc * c + 8 * (pc % (kKc / 8));
      const int off = (pc < kPieces && kk < k) ? (rr * k + kk) * 2 : kOutOfRange;
      pb[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 0));
    }
  };
  auto store_b = [&](int buf, const uint4 (&pb)[kPer]) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int pc = tid + kPcaThreads * u;
      if (pc < kPieces) *(uint4*)(&bs[buf][(pc / (kKc / 8)) * kRowStride + 8 * (pc % (kKc / 8))]) = pb[u];
    }
  };
  // raw keys of chunk c (chunks past the end read chunk 0: loaded, multiplied
  // by zero pieces): [2 j] = dims d0 .. d0 + 7, [2 j + 1] = dims 64 + d0 .. + 7
  auto load_a = [&](int c, uint4 (&ka)[4]) {
    const int cc = c < nc ? c : 0;
    const int ph = cc & 1;
    const uint16_t* kh = krow + (cc >> 1) * head_stride + 32 * ph;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      ka[2 * j] = *(const uint4*)(kh + 16 * j);
      ka[2 * j + 1] = *(const uint4*)(kh + 64 + 16 * j);
    }
  };

  float16v acc[NH];
#pragma unroll
  for (int j = 0; j < NH; ++j) acc[j] = {};

  uint4 pb[R][kPer];
  uint4 ka[R][4];
#pragma unroll
  for (int d = 0; d < R - 1; ++d) {
    load_b(d, pb[d]);
    load_a(d, ka[d]);
  }
  store_b(0, pb[0]);
  __syncthreads();

  auto step = [&](const int c, const uint4 (&a)[4], uint4 (&an)[4],
                  const uint4 (&b1)[kPer], uint4 (&bn)[kPer]) {
    // the lane's 16 phases of this chunk's pair half: pairs 32 (c % 2) + 16 j + 8 hh + e
    float2 phc[2][8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float4 v = *(const float4*)(myph + 32 * (c & 1) + 16 * j + e);
        phc[j][e] = make_float2(v.x, v.y);
        phc[j][e + 1] = make_float2(v.z, v.w);
      }
    const uint16_t* b = bs[c & 1];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint16_t* lo = (const uint16_t*)&a[2 * j];
      const uint16_t* hi = (const uint16_t*)&a[2 * j + 1];
      half8 f[2];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float2 cs = phc[j][e];
        const float l = h2f(lo[e]), h = h2f(hi[e]);
        // undo_rope: k cos - rotate_half(k) sin, rotate_half = [-hi, lo] (k_k_prepare's arithmetic)
        f[e >> 2][e & 3] = (half_t)__fadd_rn(__fmul_rn(l, cs.x), __fmul_rn(h, cs.y));
        f[e >> 2][4 + (e & 3)] = (half_t)__fsub_rn(__fmul_rn(h, cs.x), __fmul_rn(l, cs.y));
      }
#pragma unroll
      for (int o = 0; o < 2; ++o) {
        const int s = 2 * j + o;
#pragma unroll
        for (int jj = 0; jj < NH; ++jj) {
          if (NB32 % 2 == 0 || jj < nj) {
            const uint4 bv = *(const uint4*)(b + (32 * (j0 + jj) + col) * kRowStride + 16 * s + 8 * hh);
            acc[jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[o], __builtin_bit_cast(half8, bv), acc[jj], 0, 0, 0);
          }
        }
      }
    }
    store_b((c + 1) & 1, b1);
    load_b(c + R - 1, bn);
    load_a(c + R - 1, an);
    __syncthreads();
  };
  // the chunk count rounded up to the ring: chunks past nc multiply by zero
  // Btp pieces (out-of-range reads) and add exact zeros
  const int ncr = (nc + R - 1) / R * R;
  for (int c0 = 0; c0 < ncr; c0 += R) {
    step(c0, ka[0], ka[3], pb[1], pb[3]);
    step(c0 + 1, ka[1], ka[0], pb[2], pb[0]);
    step(c0 + 2, ka[2], ka[1], pb[3], pb[1]);
    step(c0 + 3, ka[3], ka[2], pb[0], pb[2]);
  }
  // C layout of the 32x32 block: lane (col, hh), reg i -> row 8 (i / 4) + 4 hh + i % 4
#pragma unroll
  for (int jj = 0; jj < NH; ++jj) {
    if (jj < nj) {
      const float bz = bias ? bias[32 * (j0 + jj) + col] : 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t rr = row0 + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (rr < m) C[rr * ldc + 32 * (j0 + jj) + col] = acc[jj][i] - bz;
      }
    }
  }
}

// (cos, sin)(fl(pos * inv_freq[i])) for pos = start + t, t < n, i < hd2: the
// phases of k_k_prepare, one table per token range (shared by every batch
// row, head and layer that undoes RoPE at those positions).
__global__ void k_rope_phases(int start, int n, int hd2, const float* __restrict__ inv_freq,
                              float2* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)n * hd2) return;
  const int t = (int)(i / hd2), p = (int)(i - (int64_t)t * hd2);
  float sn, cs;
  sincosf(__fmul_rn((float)(start + t), inv_freq[p]), &sn, &cs);
  out[i] = make_float2(cs, sn);
}

}  // namespace shard

using namespace shard;

static constexpr int32_t kPcaMaxCols = 256;  // output columns of one projection launch

extern "C" int shard_pca_project(const uint16_t* a, int64_t m, int32_t k, int64_t lda,
                                 const uint16_t* bt, int32_t n, float* c, int64_t ldc,
                                 void* stream) {
  if (!a || !bt || !c || m <= 0 || k <= 0 || n <= 0) return SHARD_ERR_ARG;
  if (k % 16 != 0 || n % 32 != 0 || lda < k || ldc < n || (lda % 8) != 0)
    return SHARD_ERR_SHAPE;
  // byte ranges of the buffer resources (one workgroup's A rows, one launch's Bt)
  if ((int64_t)kPcaRows * lda * 2 >= (1ll << 31) - 256 ||
      (int64_t)std::min(n, kPcaMaxCols) * k * 2 >= (1ll << 31) - 256)
    return SHARD_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)((m + kPcaRows - 1) / kPcaRows));
  // up to 256 columns per launch (the accumulators of a wave); wider
  // projections (ranks above 256) take one launch per 256 columns
  for (int32_t c0 = 0; c0 < n; c0 += kPcaMaxCols) {
    const int32_t nc = std::min(n - c0, kPcaMaxCols);
    const uint16_t* btc = bt + (int64_t)c0 * k;
    float* cc = c + c0;
    switch (nc / 32) {
      case 1: hipLaunchKernelGGL(k_pca_project<1>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 2: hipLaunchKernelGGL(k_pca_project<2>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 3: hipLaunchKernelGGL(k_pca_project<3>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 4: hipLaunchKernelGGL(k_pca_project<4>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 5: hipLaunchKernelGGL(k_pca_project<5>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 6: hipLaunchKernelGGL(k_pca_project<6>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 7: hipLaunchKernelGGL(k_pca_project<7>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      default: hipLaunchKernelGGL(k_pca_project<8>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
    }
    SHARD_LAUNCH_CHECK("shard_pca_project");
  }
  return SHARD_OK;
}

extern "C" int shard_pca_project_f32(const float* a, int64_t m, int32_t k, int64_t lda,
                                     const float* bt, int32_t n, float* c, int64_t ldc,
                                     void* stream) {
  if (!a || !bt || !c || m <= 0 || k <= 0 || n <= 0) return SHARD_ERR_ARG;
  if (k % 8 != 0 || n % 32 != 0 || lda < k || ldc < n || (lda % 4) != 0)
    return SHARD_ERR_SHAPE;
  if (((uintptr_t)a & 15) || ((uintptr_t)bt & 15)) return SHARD_ERR_SHAPE;  // 16-byte vectors
  if ((int64_t)kPcaRows * lda * 4 >= (1ll << 31) - 256 ||
      (int64_t)std::min(n, kPcaMaxCols) * k * 4 >= (1ll << 31) - 256)
    return SHARD_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)((m + kPcaRows - 1) / kPcaRows));
  for (int32_t c0 = 0; c0 < n; c0 += kPcaMaxCols) {  // as shard_pca_project: 256 columns per launch
    const int32_t nc = std::min(n - c0, kPcaMaxCols);
    const float* btc = bt + (int64_t)c0 * k;
    float* cc = c + c0;
    switch (nc / 32) {
      case 1: hipLaunchKernelGGL(k_pca_project_f32<1>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 2: hipLaunchKernelGGL(k_pca_project_f32<2>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 3: hipLaunchKernelGGL(k_pca_project_f32<3>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 4: hipLaunchKernelGGL(k_pca_project_f32<4>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 5: hipLaunchKernelGGL(k_pca_project_f32<5>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 6: hipLaunchKernelGGL(k_pca_project_f32<6>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      case 7: hipLaunchKernelGGL(k_pca_project_f32<7>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
      default: hipLaunchKernelGGL(k_pca_project_f32<8>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, btc, cc, ldc); break;
    }
    SHARD_LAUNCH_CHECK("shard_pca_project_f32");
  }
  return SHARD_OK;
}

extern "C" int shard_rope_phases(int32_t start, int32_t n, int32_t hd2, const float* inv_freq,
                                 float* out, void* stream) {
  if (!inv_freq || !out || n <= 0 || hd2 <= 0 || start < 0) return SHARD_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const int64_t total = (int64_t)n * hd2;
  hipLaunchKernelGGL(k_rope_phases, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, start, n,
                     hd2, inv_freq, (float2*)out);
  SHARD_LAUNCH_CHECK("shard_rope_phases");
  return SHARD_OK;
}

extern "C" int shard_pca_project_rope(const uint16_t* k, int32_t batch, int32_t n_kv, int32_t seq,
                                      int32_t hd, int32_t start, int32_t n_comp,
                                      const float* phases, const uint16_t* btp, int32_t n,
                                      const float* bias, float* c, int64_t ldc, void* stream) {
  if (!k || !phases || !btp || !c || batch <= 0 || n_kv <= 0 || n_comp <= 0 || n <= 0)
    return SHARD_ERR_ARG;
  if (hd != 128 || n % 32 != 0 || n > 256 || ldc < n || start < 0 ||
      start + n_comp > seq)
    return SHARD_ERR_SHAPE;
  if (((uintptr_t)k & 15) || ((uintptr_t)phases & 15) || ((uintptr_t)btp & 15)) return SHARD_ERR_SHAPE;
  if ((int64_t)n * n_kv * 128 * 2 >= (1ll << 31) - 256) return SHARD_ERR_SHAPE;
  const int64_t m = (int64_t)batch * n_comp;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)((m + kPcaRows - 1) / kPcaRows));
#define SHARD_PR(NB) hipLaunchKernelGGL(k_pca_project_rope<NB>, grid, dim3(kPcaThreads), 0, s, k, n_kv, \
                                        seq, start, n_comp, m, (const float2*)phases, btp, bias, c, ldc)
  switch (n / 32) {
    case 1: SHARD_PR(1); break;
    case 2: SHARD_PR(2); break;
    case 3: SHARD_PR(3); break;
    case 4: SHARD_PR(4); break;
    case 5: SHARD_PR(5); break;
    case 6: SHARD_PR(6); break;
    case 7: SHARD_PR(7); break;
    case 8: SHARD_PR(8); break;
    default: return SHARD_ERR_SHAPE;
  }
#undef SHARD_PR
  SHARD_LAUNCH_CHECK("shard_pca_project_rope");
  return SHARD_OK;
}
