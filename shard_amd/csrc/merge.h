// Merge of split partial rows into the attention output, shared by the
// compressed decode call and the fp16 split-K baseline.  Layout of the
// partial rows (one per (batch row, query head, split), row-major in that
// order): m (base-2 running max), l (sum of 2^(s - m)), acc (128 fp32 sums,
// of which the first `hd` are the output's: hd 64 for head_dim-64 layers).
#pragma once

#include "common.h"

namespace shard {
namespace {   // internal linkage: each code object gets its own kernels

constexpr int kMergeHD = 128;

// --------------------------------------------------------------------------
// Merge of the split partial rows (all in the plain basis):
//   out = sum_s w_s acc_s / sum_s w_s l_s,  w_s = 2^(m_s - M).
// MS workgroups of 256 threads per (query head, batch row), each owning 128/MS
// dims; thread = (row group g, dim pair dp), rows g, g + RG, g + 2 RG, ...
// Every row load of a thread is issued before the first use; a wave
// reduction and one barrier give M, shuffles and a second barrier sum over
// the row groups.  The slice count spreads the reads over more CUs: the
// partial rows were just written back by the split kernel, so the merge is
// bound by how many loads are in flight, not by bytes (at 8K, batch 1, one
// workgroup per head: 17.5 us per call, 8 slices: 14.9 us).
// --------------------------------------------------------------------------
struct MergeParams {
  int32_t H, nsp;   // query heads per batch row, partial rows per query head
  int32_t hd;       // output dims per query head: 128, or 64 (the first 64 of each row)
  // kv_nq > 0: the partial rows of (batch row, kv head) group i were written
  // on XCD i mod 8 (kv_nq query heads per kv head); the group's slices run there
  int32_t kv_nq;
  const float* ws_m;
  const float* ws_l;
  const float* ws_acc;
  uint16_t* out;
};

template <int MS>
__global__ __launch_bounds__(256)
void k_decode_merge(const MergeParams p) {
  constexpr int DP = kMergeHD / 2 / MS;   // dim pairs per slice
  constexpr int RG = 256 / DP;       // row groups
  constexpr int RU = 128 / RG;       // rows per thread loaded up front (128 rows in all)
  __shared__ float wmax[4];
  __shared__ __align__(16) float2 wacc[4][DP];
  __shared__ float wl[4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int dp = tid % DP, g = tid / DP;
  // the MS slices of a head share one XCD (workgroups go to XCD id mod 8), so
  // one L2 fetches each 128-byte line of the partial rows once
  const int bx = blockIdx.x;
  int slice, head, brow;
  if (p.kv_nq) {
    const int L = blockIdx.y * gridDim.x + bx, r = L >> 3;
    slice = r % MS;
    const int grp_i = (L & 7) + 8 * (r / (MS * p.kv_nq));
    const int G = p.H / p.kv_nq;
    brow = grp_i / G;
    head = (grp_i % G) * p.kv_nq + (r / MS) % p.kv_nq;
  } else {
    slice = (bx >> 3) % MS;
    head = (bx & 7) + 8 * (bx / (8 * MS));
    brow = blockIdx.y;
  }
  if (slice * 2 * DP >= p.hd) return;  // a slice past the output's dims (whole workgroup)
  const int64_t hrow = (int64_t)brow * p.H + head;
  const int nsp = p.nsp;
  const float* mrow = p.ws_m + hrow * nsp;
  const float* lrow = p.ws_l + hrow * nsp;
  const float* arow = p.ws_acc + hrow * nsp * kMergeHD + slice * (2 * DP) + 2 * dp;
  float2 av[RU];
  float mv[RU], lv[RU];
#pragma unroll
  for (int u = 0; u < RU; ++u) {
    const int s = g + RG * u;
    av[u] = make_float2(0.f, 0.f);
    mv[u] = -INFINITY;
    lv[u] = 0.f;
    if (s < nsp) {
      av[u] = *(const float2*)(arow + (int64_t)s * kMergeHD);
      mv[u] = mrow[s];
      lv[u] = lrow[s];
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < RU; ++u) mx = fmaxf(mx, mv[u]);
  for (int s = g + RG * RU; s < nsp; s += RG) mx = fmaxf(mx, mrow[s]);
  mx = wave64_reduce(mx, OpMax());
  if (lane == 0) wmax[w] = mx;
  __syncthreads();
  float M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  if (M == -INFINITY) M = 0.f;  // everything masked: all weights are zero
  float a0 = 0.f, a1 = 0.f, l = 0.f;
#pragma unroll
  for (int u = 0; u < RU; ++u) {
    const float wt = mv[u] != -INFINITY ? exp2f(mv[u] - M) : 0.f;
    a0 += wt * av[u].x;
    a1 += wt * av[u].y;
    l += wt * lv[u];
  }
  for (int s = g + RG * RU; s < nsp; s += RG) {
    const float m = mrow[s];
    const float wt = m != -INFINITY ? exp2f(m - M) : 0.f;
    const float2 v = *(const float2*)(arow + (int64_t)s * kMergeHD);
    a0 += wt * v.x;
    a1 += wt * v.y;
    l += wt * lrow[s];
  }
  // sum over the wave's row groups (lanes with the same dim pair)
#pragma unroll
  for (int off = DP; off < 64; off <<= 1) {
    a0 += __shfl_xor(a0, off);
    a1 += __shfl_xor(a1, off);
    l += __shfl_xor(l, off);
  }
  if (lane < DP) wacc[w][lane] = make_float2(a0, a1);
  if (lane == 0) wl[w] = l;
  __syncthreads();
  if (tid < DP && slice * (2 * DP) + 2 * tid < p.hd) {
    float2 t = wacc[0][tid];
    float lt = wl[0];
#pragma unroll
    for (int u = 1; u < 4; ++u) {
      t.x += wacc[u][tid].x;
      t.y += wacc[u][tid].y;
      lt += wl[u];
    }
    const float inv_l = 1.0f / lt;
    half2v o;
    o[0] = (half_t)(t.x * inv_l);
    o[1] = (half_t)(t.y * inv_l);
    *(half2v*)(p.out + hrow * p.hd + slice * (2 * DP) + 2 * tid) = o;
  }
}

// The slice count is the most of 8, 4, 2, 1 that keeps the grid at or below
// 512 workgroups (measured best at batch 1, 4 and 16 of 32 heads).
// The XCD-aware slice order needs H % 8 == 0; other head counts take one slice.
inline void launch_partial_merge(const MergeParams& mp, int batch, hipStream_t s) {
  const int64_t pairs = (int64_t)batch * mp.H;
  const int ms = mp.H % 8 ? 1 : pairs * 8 <= 512 ? 8 : pairs * 4 <= 512 ? 4 : pairs * 2 <= 512 ? 2 : 1;
  const dim3 grid((unsigned)(mp.H * ms), (unsigned)batch);
  switch (ms) {
    case 8: hipLaunchKernelGGL(k_decode_merge<8>, grid, dim3(256), 0, s, mp); break;
    case 4: hipLaunchKernelGGL(k_decode_merge<4>, grid, dim3(256), 0, s, mp); break;
    case 2: hipLaunchKernelGGL(k_decode_merge<2>, grid, dim3(256), 0, s, mp); break;
    default: hipLaunchKernelGGL(k_decode_merge<1>, grid, dim3(256), 0, s, mp); break;
  }
}

}  // namespace
}  // namespace shard
