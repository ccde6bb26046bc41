// PCA projection GEMM of prefill compression on gfx950 MFMA:
//   C[m, n] (fp32) = A[m, k] (fp16, row-major) . Bt[n, k]^T (fp16, row-major)
// The basis side Bt (n <= 256 components) is tiny and shared by every
// workgroup, so it is staged in LDS per 64-wide k chunk; A streams from HBM.
// Workgroup = 4 waves x 32 rows = 128 rows; each wave owns all n columns
// (n/32 accumulator blocks of v_mfma_f32_32x32x16_f16).
#include "common.h"

namespace shard {

constexpr int kPcaThreads = 256;
constexpr int kPcaRows = 128;
constexpr int kKc = 64;  // k chunk staged in LDS

template <int NB32>
__global__ __launch_bounds__(kPcaThreads, 2)
void k_pca_project(const uint16_t* __restrict__ A, int64_t m, int k, int64_t lda,
                   const uint16_t* __restrict__ Bt, float* __restrict__ C, int64_t ldc) {
  // Bt chunk: NB32*32 rows x 64 halves, padded row stride to spread LDS banks
  constexpr int kRowStride = kKc + 8;
  __shared__ __align__(16) uint16_t bs[NB32 * 32 * kRowStride];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int col = lane & 31, hh = lane >> 5;
  const int64_t row0 = (int64_t)blockIdx.x * kPcaRows + 32 * w;
  const int64_t arow = row0 + col;
  const bool arow_ok = arow < m;
  const uint16_t* ap = A + (arow_ok ? arow : 0) * lda;

  float16v acc[NB32];
#pragma unroll
  for (int j = 0; j < NB32; ++j) acc[j] = {};

  for (int k0 = 0; k0 < k; k0 += kKc) {
    // stage Bt[:, k0:k0+64] (16-byte pieces)
    const int pieces = NB32 * 32 * (kKc / 8);
    for (int pc = tid; pc < pieces; pc += kPcaThreads) {
      const int r = pc / (kKc / 8), c8 = pc % (kKc / 8);
      const int kk = k0 + 8 * c8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (kk < k) v = *(const uint4*)(Bt + (int64_t)r * k + kk);
      *(uint4*)(bs + r * kRowStride + 8 * c8) = v;
    }
    // A fragments for the 4 k-steps of this chunk (16 B per lane per step)
    half8 af[kKc / 16];
#pragma unroll
    for (int s = 0; s < kKc / 16; ++s) {
      const int kk = k0 + 16 * s + 8 * hh;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (arow_ok && kk < k) v = *(const uint4*)(ap + kk);
      af[s] = __builtin_bit_cast(half8, v);
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < kKc / 16; ++s) {
#pragma unroll
      for (int j = 0; j < NB32; ++j) {
        const uint4 bv = *(const uint4*)(bs + (32 * j + col) * kRowStride + 16 * s + 8 * hh);
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s], __builtin_bit_cast(half8, bv),
                                                        acc[j], 0, 0, 0);
      }
    }
    __syncthreads();
  }
  // C layout of the 32x32 block: lane (col, hh), reg i -> row 8*(i/4) + 4*hh + i%4
#pragma unroll
  for (int j = 0; j < NB32; ++j)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t r = row0 + 8 * (i >> 2) + 4 * hh + (i & 3);
      if (r < m) C[r * ldc + 32 * j + col] = acc[j][i];
    }
}

}  // namespace shard

using namespace shard;

extern "C" int shard_pca_project(const uint16_t* a, int64_t m, int32_t k, int64_t lda,
                                 const uint16_t* bt, int32_t n, float* c, int64_t ldc,
                                 void* stream) {
  if (!a || !bt || !c || m <= 0 || k <= 0 || n <= 0) return SHARD_ERR_ARG;
  if (k % 16 != 0 || n % 32 != 0 || n > 256 || lda < k || ldc < n || (lda % 8) != 0)
    return SHARD_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)((m + kPcaRows - 1) / kPcaRows));
  switch (n / 32) {
    case 1: hipLaunchKernelGGL(k_pca_project<1>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, bt, c, ldc); break;
    case 2: hipLaunchKernelGGL(k_pca_project<2>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, bt, c, ldc); break;
    case 3: hipLaunchKernelGGL(k_pca_project<3>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, bt, c, ldc); break;
    case 4: hipLaunchKernelGGL(k_pca_project<4>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, bt, c, ldc); break;
    case 5: hipLaunchKernelGGL(k_pca_project<5>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, bt, c, ldc); break;
    case 6: hipLaunchKernelGGL(k_pca_project<6>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, bt, c, ldc); break;
    case 7: hipLaunchKernelGGL(k_pca_project<7>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, bt, c, ldc); break;
    case 8: hipLaunchKernelGGL(k_pca_project<8>, grid, dim3(kPcaThreads), 0, s, a, m, k, lda, bt, c, ldc); break;
    default: return SHARD_ERR_SHAPE;
  }
  SHARD_LAUNCH_CHECK("shard_pca_project");
  return SHARD_OK;
}
