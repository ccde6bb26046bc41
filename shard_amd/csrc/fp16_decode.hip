// fp16 split-K GQA decode attention over uncompressed K/V, written for gfx950:
// the same-GPU FlashDecoding-style baseline the benchmark times next to the
// compressed path.  It is not part of the compressed-KV path and no product
// code calls it.
//
//   k_fp16_split  grid = (n_splits * G, B), 256 threads (4 waves).  One kv
//     head x a range of tokens; wave w takes the 32-token tiles w, w + 4, ...
//     Scores of the head's 4 query heads on MFMA 32x32x16 f16 (A = q, rows =
//     query heads; B = K^T, each lane one token's 8 dims: one 16-byte load),
//     online softmax (fp32, base 2) per wave, values on the VALU (lane = 8
//     dims of one token in 4, 16-byte loads), the next tile's K and V loads in
//     flight during the current one.  The waves merge in LDS and write one
//     partial row (m, l, 128 sums) per query head and split.
//   k_decode_merge (merge.h): the log-sum-exp weighted sum of the splits.
#include <math.h>

#include "common.h"
#include "merge.h"

namespace shard {

namespace {

constexpr int kFdHD = 128;
constexpr int kFdGQA = 4;
constexpr int kFdWaves = 4;
constexpr float kFdLog2e = 1.4426950408889634f;

struct Fp16Params {
  int32_t B, G, T, n_splits, chunk;
  int64_t ld;  // rows between consecutive (batch row, kv head) heads in k / v (>= T)
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  float* ws_m;
  float* ws_l;
  float* ws_acc;
};

__global__ __launch_bounds__(64 * kFdWaves, 2)
void k_fp16_split(const Fp16Params p) {
  __shared__ __align__(16) float pw[kFdWaves][32][kFdGQA];        // softmax numerators
  __shared__ __align__(16) float racc[kFdWaves][kFdGQA][kFdHD];  // per-wave value sums
  __shared__ float rml[kFdWaves][2][kFdGQA];                      // per-wave m, l

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = blockIdx.x % p.G, split = blockIdx.x / p.G, b = blockIdx.y;
  const int H = p.G * kFdGQA;
  const int t_begin = split * p.chunk;
  const int t_end = min(t_begin + p.chunk, p.T);
  const int n_tiles = t_end > t_begin ? (t_end - t_begin + 31) / 32 : 0;

  const uint16_t* kh = p.k + ((int64_t)b * p.G + g) * p.ld * kFdHD;
  const uint16_t* vh = p.v + ((int64_t)b * p.G + g) * p.ld * kFdHD;

  // A operand: q rows 0-3 (query heads), k-step s covers dims 16 s .. 16 s + 15
  const int col = lane & 31, hh = lane >> 5;
  half8 Aq[8];
  {
    const uint16_t* qv = p.q + ((int64_t)b * H + g * kFdGQA + min(col, kFdGQA - 1)) * kFdHD + 8 * hh;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint4 v4 = *(const uint4*)(qv + 16 * s);
      Aq[s] = __builtin_bit_cast(half8, col < kFdGQA ? v4 : make_uint4(0u, 0u, 0u, 0u));
    }
  }
  const float sc = kFdLog2e * 0.08838834764831845f;  // log2(e) / sqrt(128)

  // V stage: lane = (token group tg, dims 8 dq .. 8 dq + 7)
  const int tg = lane >> 4, dq = lane & 15;
  float m_run[kFdGQA], l_run[kFdGQA], acc[kFdGQA][8];
#pragma unroll
  for (int h = 0; h < kFdGQA; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }

  uint4 kb[2][8], vb[2][8];
  auto load = [&](int tile, uint4 (&k_)[8], uint4 (&v_)[8]) {
    const int t0 = t_begin + 32 * tile;
    const int tk = min(t0 + col, t_end - 1);  // clamped rows are masked below
#pragma unroll
    for (int s = 0; s < 8; ++s) k_[s] = *(const uint4*)(kh + (int64_t)tk * kFdHD + 16 * s + 8 * hh);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int tv = min(t0 + 4 * j + tg, t_end - 1);
      v_[j] = *(const uint4*)(vh + (int64_t)tv * kFdHD + 8 * dq);
    }
  };
  auto run = [&](int tile, const uint4 (&k_)[8], const uint4 (&v_)[8]) {
    const int t0 = t_begin + 32 * tile;
    float16v sacc = {};
#pragma unroll
    for (int s = 0; s < 8; ++s)
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aq[s], __builtin_bit_cast(half8, k_[s]), sacc, 0, 0, 0);
    // rows 0-3 (query heads) sit in elements 0-3 of lanes 0-31, column = token
    const bool valid = hh == 0 && t0 + col < t_end;
    float al[kFdGQA];
#pragma unroll
    for (int h = 0; h < kFdGQA; ++h) {
      const float s = valid ? sacc[h] * sc : -INFINITY;
      const float m_new = fmaxf(m_run[h], wave64_reduce(s, OpMax()));
      al[h] = m_new == -INFINITY ? 1.f : exp2f(m_run[h] - m_new);
      const float pv = s == -INFINITY ? 0.f : exp2f(s - m_new);
      l_run[h] = l_run[h] * al[h] + wave64_reduce(pv, OpAdd());
      m_run[h] = m_new;
      if (hh == 0) pw[w][col][h] = pv;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int h = 0; h < kFdGQA; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= al[h];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float4 pt = *(const float4*)&pw[w][4 * j + tg][0];
      const half8 vv = __builtin_bit_cast(half8, v_[j]);
      const float ph[4] = {pt.x, pt.y, pt.z, pt.w};
#pragma unroll
      for (int h = 0; h < kFdGQA; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] += ph[h] * (float)vv[e];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // pw is rewritten by the next tile
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  int tile = w;
  if (tile < n_tiles) load(tile, kb[0], vb[0]);
  while (tile < n_tiles) {
    const int nx = tile + kFdWaves;
    if (nx < n_tiles) load(nx, kb[1], vb[1]);
    run(tile, kb[0], vb[0]);
    if (nx >= n_tiles) break;
    const int nx2 = nx + kFdWaves;
    if (nx2 < n_tiles) load(nx2, kb[0], vb[0]);
    run(nx, kb[1], vb[1]);
    tile = nx2;
  }

  // ---- the 4 token groups of the wave, then the waves: racc / rml in LDS
#pragma unroll
  for (int h = 0; h < kFdGQA; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = acc[h][e];
      x += __shfl_xor(x, 16);
      x += __shfl_xor(x, 32);
      acc[h][e] = x;
    }
  if (tg == 0) {
#pragma unroll
    for (int h = 0; h < kFdGQA; ++h) {
      *(float4*)&racc[w][h][8 * dq] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      *(float4*)&racc[w][h][8 * dq + 4] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < kFdGQA; ++h) {
      rml[w][0][h] = m_run[h];
      rml[w][1][h] = l_run[h];
    }
  }
  __syncthreads();
  // wave h: query head h; lane = dims 2 lane, 2 lane + 1
  {
    const int h = w;
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < kFdWaves; ++u) M = fmaxf(M, rml[u][0][h]);
    float a0 = 0.f, a1 = 0.f, l = 0.f;
#pragma unroll
    for (int u = 0; u < kFdWaves; ++u) {
      const float mu = rml[u][0][h];
      const float wt = mu == -INFINITY ? 0.f : exp2f(mu - M);
      const float2 r = *(const float2*)&racc[u][h][2 * lane];
      a0 += wt * r.x;
      a1 += wt * r.y;
      l += wt * rml[u][1][h];
    }
    const int64_t widx = ((int64_t)b * H + g * kFdGQA + h) * p.n_splits + split;
    *(float2*)(p.ws_acc + widx * kFdHD + 2 * lane) = make_float2(a0, a1);
    if (lane == 0) {
      p.ws_m[widx] = M;
      p.ws_l[widx] = l;
    }
  }
}

}  // namespace

}  // namespace shard

using namespace shard;

extern "C" {

size_t shard_bench_fp16_decode_workspace(int32_t batch, int32_t n_kv_heads, int32_t n_splits) {
  if (batch <= 0 || n_kv_heads <= 0 || n_splits <= 0) return 0;
  return (size_t)batch * n_kv_heads * kFdGQA * n_splits * (kFdHD + 2) * sizeof(float);
}

int shard_bench_fp16_decode_ld(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               int32_t batch, int32_t n_kv_heads, int32_t seq, int64_t head_rows,
                               int32_t n_splits, uint16_t* out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !out || !workspace || batch <= 0 || n_kv_heads <= 0 || seq <= 0 ||
      n_splits <= 0 || head_rows < seq)
    return SHARD_ERR_ARG;
  if (((uintptr_t)q & 15) || ((uintptr_t)k & 15) || ((uintptr_t)v & 15) || ((uintptr_t)out & 3))
    return SHARD_ERR_ARG;
  if (workspace_bytes < shard_bench_fp16_decode_workspace(batch, n_kv_heads, n_splits))
    return SHARD_ERR_WORKSPACE;
  Fp16Params p;
  p.B = batch; p.G = n_kv_heads; p.T = seq; p.n_splits = n_splits; p.ld = head_rows;
  p.chunk = ((seq + n_splits - 1) / n_splits + 31) / 32 * 32;
  const int64_t nm = (int64_t)batch * n_kv_heads * kFdGQA * n_splits;
  float* ws = (float*)workspace;
  p.q = q; p.k = k; p.v = v;
  p.ws_m = ws; p.ws_l = ws + nm; p.ws_acc = ws + 2 * nm;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_fp16_split, dim3((unsigned)(n_splits * n_kv_heads), (unsigned)batch),
                     dim3(64 * kFdWaves), 0, s, p);
  SHARD_LAUNCH_CHECK("shard_bench_fp16_decode split");
  MergeParams mp;
  mp.H = n_kv_heads * kFdGQA; mp.nsp = n_splits; mp.hd = kMergeHD; mp.kv_nq = 0;
  mp.ws_m = p.ws_m; mp.ws_l = p.ws_l; mp.ws_acc = p.ws_acc; mp.out = out;
  launch_partial_merge(mp, batch, s);
  SHARD_LAUNCH_CHECK("shard_bench_fp16_decode merge");
  return SHARD_OK;
}

int shard_bench_fp16_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v, int32_t batch,
                            int32_t n_kv_heads, int32_t seq, int32_t n_splits, uint16_t* out,
                            void* workspace, size_t workspace_bytes, void* stream) {
  return shard_bench_fp16_decode_ld(q, k, v, batch, n_kv_heads, seq, seq, n_splits, out, workspace,
                                    workspace_bytes, stream);
}

}  // extern "C"
