// Fused decode attention over Shard's compressed KV cache, written for gfx950.
//
// Work split (one launch + one combine launch per layer-step):
//   split kernel   grid = (n_splits * n_kv/NB, B); a 256-thread workgroup owns
//                  NB kv heads x a chunk of compressed tokens.  Wave w owns the
//                  16 RoPE pairs [16w, 16w+16) of each of its NB heads, so the
//                  sin/cos of a (token, pair) is computed once per wave and the
//                  int4 coefficient tile is unpacked once for NB heads.
//     1. no-RoPE keys are rebuilt on chip with MFMA 32x32x16 f16:
//          K_n[rows, tok] = Basis'[rows, r] . coef[r, tok] + mean
//        Basis' = fp16(basis_f16 * coeff_scale) lives in VGPRs for the whole
//        kernel; coef are the packed nibbles (128-bit loads) turned into exact
//        fp16 integers n-8 with a magic-number trick.  Keys never reach HBM.
//     2. each (c, d) pair is rotated by phi = fl32(fl32(pos_t - pos_q) * theta_i)
//        (the relative-delta RoPE identity, attention.py:3-6) and dotted with
//        q_n = undo-RoPE(q, pos_q) by a second MFMA (rows = query heads).
//     3. the 4 waves' partial scores are summed in LDS, online softmax (fp32,
//        base-2), and the VQ values sum_t p_t * cb[idx_t] (rotated space) are
//        accumulated with the fp32 codebook in LDS.
//     4. per (query head, split): running max m, sum l and the 128-dim
//        accumulator go to the workspace.
//   combine kernel grid = (n_kv, B): merges the splits, applies ch and ONE
//                  inverse Hadamard to the VQ accumulator, adds the fp16 sink /
//                  window / decode segments and the 8-bit stream (dequantized
//                  bit-exactly like cache.py:243-279), normalizes, writes fp16.
#include "common.h"

namespace shard {

constexpr int kThreads = 256;
constexpr int kTile = 32;      // tokens per MFMA tile
constexpr int kHD = 128;       // head_dim
constexpr int kGQA = 4;        // query heads per kv head
constexpr int kMaxExtra = 2048;   // sink + window + decode + stream tokens per call
constexpr float kLog2e = 1.4426950408889634f;

struct SplitParams {
  int32_t B, H, G, rank, n_comp, cstart, pos_q, n_splits, chunk;
  const uint16_t* q;
  const float* inv_freq;
  const uint8_t* coef;
  const uint16_t* cs;
  const uint16_t* basis;
  const uint16_t* mean;
  const uint8_t* vidx;
  const uint16_t* vcb;
  const float* mask;
  int64_t mask_stride;
  int32_t n_sink;
  float* ws_m;
  float* ws_l;
  float* ws_acc;
};

// 8 packed nibbles (n0 in bits 0-3 ... n7 in bits 28-31) -> 8 exact fp16 values
// n-8 in element order (n0, n4, n1, n5, n2, n6, n3, n7).
__device__ __forceinline__ half8 nib8_to_half8(uint32_t x) {
  const uint32_t x8 = x >> 8;
  const uint32_t v0 = (x & 0x000F000Fu) | 0x64006400u;   // 1024 + n0 | 1024 + n4
  const uint32_t v1 = (x & 0x00F000F0u) | 0x64006400u;   // 1024 + 16 n1 | 1024 + 16 n5
  const uint32_t v2 = (x8 & 0x000F000Fu) | 0x64006400u;  // 1024 + n2 | 1024 + n6
  const uint32_t v3 = (x8 & 0x00F000F0u) | 0x64006400u;  // 1024 + 16 n3 | 1024 + 16 n7
  const half2v k1032 = {(half_t)1032.f, (half_t)1032.f};
  const half2v k16 = {(half_t)0.0625f, (half_t)0.0625f};
  const half2v k72 = {(half_t)72.f, (half_t)72.f};
  half2v h0 = __builtin_bit_cast(half2v, v0) - k1032;
  half2v h1 = __builtin_bit_cast(half2v, v1) * k16 - k72;
  half2v h2 = __builtin_bit_cast(half2v, v2) - k1032;
  half2v h3 = __builtin_bit_cast(half2v, v3) * k16 - k72;
  half8 r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

__device__ __forceinline__ int nib_perm(int e) { return ((e & 1) << 2) | (e >> 1); }

// Wave-local row rho (0..31) of the MFMA tile -> head dim: rows 0..15 are the
// first components c of pairs 16P+rho, rows 16..31 the second components d.
__device__ __forceinline__ int row_dim(int P, int rho) {
  return rho < 16 ? 16 * P + rho : 64 + 16 * P + (rho - 16);
}

template <int KS, int NB>
__global__ __launch_bounds__(kThreads, 1)
void k_decode_split(const SplitParams p) {
  constexpr int NQ = kGQA * NB;          // query heads of this workgroup
  constexpr int TS = 8 / NB;             // token subsets of the V stage
  constexpr int SPT = (NQ * kTile + kThreads - 1) / kThreads;

  __shared__ __align__(16) float sp[4][NQ][kTile];   // per-wave partial scores
  __shared__ __align__(16) float pp[kTile][NQ];      // softmax numerators of the tile
  __shared__ __align__(16) float alpha_s[NQ];        // rescale factors of the tile
  __shared__ __align__(16) float4 cbl[256];          // VQ codebook in fp32
  __shared__ __align__(16) float red[kThreads][16];  // end-of-chunk reduction

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int P = tid >> 6;                // wave = pair slice
  const int col = lane & 31;
  const int hh = lane >> 5;

  // ---- XCD-aware block -> (head group, split): all head groups of one split
  // land on the same XCD (block ids congruent mod 8) so the coefficient rows
  // of that split are fetched once into that XCD's L2.
  const int HG = p.G / NB;
  const int bid = blockIdx.x;
  const int slot = bid >> 3;
  const int hg = slot % HG;
  const int split = (slot / HG) * 8 + (bid & 7);
  const int b = blockIdx.y;
  const int t_begin = split * p.chunk;
  int t_end = t_begin + p.chunk;
  if (t_end > p.n_comp) t_end = p.n_comp;

  for (int i = tid; i < 256; i += kThreads) {
    const uint16_t* c4 = p.vcb + 4 * i;
    cbl[i] = make_float4(h2f(c4[0]), h2f(c4[1]), h2f(c4[2]), h2f(c4[3]));
  }

  // ---- lane constants: pairs, theta, basis A-operand, mean C-init, q_n A-operand
  int pr[8];
  float th[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    pr[i] = 16 * P + 8 * (i >> 2) + 4 * hh + (i & 3);
    th[i] = p.inv_freq[pr[i]];
  }

  half8 Ab[NB][KS];
  float16v meanC[NB];
  {
    const int rho = col;
    const int dim = row_dim(P, rho);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int g = hg * NB + j;
      const uint16_t* brow = p.basis + (int64_t)(g * kHD + dim) * p.rank;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int r0 = 8 * (KS * hh + s);
        half8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = r0 + nib_perm(e);
          v[e] = (half_t)(h2f(brow[r]) * h2f(p.cs[r]));
        }
        Ab[j][s] = v;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rho_i = 8 * (i >> 2) + 4 * hh + (i & 3);
        meanC[j][i] = h2f(p.mean[g * kHD + row_dim(P, rho_i)]);
      }
    }
  }

  // q_n = undo-RoPE(q_rope, pos_q): a = q_lo cos + q_hi sin, b = q_hi cos - q_lo sin
  half8 Aq[NB][2];
  {
    const int qr = col;  // MFMA row = query head within the workgroup
    float a_[8], b_[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { a_[i] = 0.f; b_[i] = 0.f; }
    if (qr < NQ) {
      const int qh = hg * NQ + qr;
      const uint16_t* qv = p.q + ((int64_t)b * p.H + qh) * kHD;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float sn, cs;
        sincosf((float)p.pos_q * th[i], &sn, &cs);
        const float lo = h2f(qv[pr[i]]), hi = h2f(qv[pr[i] + 64]);
        a_[i] = lo * cs + hi * sn;
        b_[i] = hi * cs - lo * sn;
      }
    }
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const bool mine = (qr >> 2) == j && qr < NQ;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Aq[j][0][e] = (half_t)(mine ? a_[e] : 0.f);
        Aq[j][1][e] = (half_t)(mine ? b_[e] : 0.f);
      }
    }
  }

  // ---- softmax-stage state (thread owns entries e = tid + 256*k)
  float m_run[SPT], l_part[SPT];
#pragma unroll
  for (int k = 0; k < SPT; ++k) { m_run[k] = -INFINITY; l_part[k] = 0.f; }
  const float sc = kLog2e * rsqrtf((float)kHD);

  // ---- V-stage mapping: tid = (j*TS + ts)*32 + G
  const int vG = tid & 31;
  const int vts = (tid >> 5) % TS;
  const int vj = (tid >> 5) / TS;
  const int vg = hg * NB + vj;
  float vacc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int e = 0; e < 4; ++e) vacc[a][e] = 0.f;

  const int rowb = KS * 4;  // bytes per lane-half of a coefficient row
  const int64_t coef_row_bytes = p.rank / 2;
  __syncthreads();

  for (int t0 = t_begin; t0 < t_end; t0 += kTile) {
    const int t = t0 + col;
    const bool tv = t < t_end;

    // V-stage index prefetch (latency hidden by the key MFMAs)
    uint8_t vcode[kTile / TS];
#pragma unroll
    for (int m = 0; m < kTile / TS; ++m) {
      const int tt = t0 + vts + TS * m;
      vcode[m] = tt < t_end ? p.vidx[(((int64_t)b * p.G + vg) * p.n_comp + tt) * 32 + vG] : 0;
    }

    // coefficient dwords of this lane: row (b, t), dwords [KS*hh, KS*hh+KS)
    uint32_t cw[KS];
    if (tv) {
      const uint8_t* rowp = p.coef + ((int64_t)b * p.n_comp + t) * coef_row_bytes + rowb * hh;
      if constexpr (KS % 4 == 0) {
#pragma unroll
        for (int s = 0; s < KS; s += 4) {
          uint4 v = *(const uint4*)(rowp + 4 * s);
          cw[s] = v.x; cw[s + 1] = v.y; cw[s + 2] = v.z; cw[s + 3] = v.w;
        }
      } else {
#pragma unroll
        for (int s = 0; s < KS; s += 2) {
          uint2 v = *(const uint2*)(rowp + 4 * s);
          cw[s] = v.x; cw[s + 1] = v.y;
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s) cw[s] = 0x88888888u;  // nibble 8 -> 0
    }

    // 1. no-RoPE keys of NB heads for 32 tokens (rows x tokens, fp32)
    float16v acc[NB];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const half8 bo = nib8_to_half8(cw[s]);
#pragma unroll
      for (int j = 0; j < NB; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ab[j][s], bo, s == 0 ? meanC[j] : acc[j], 0, 0, 0);
    }

    // 2. rotate pairs by phi(t, i), then dot with q_n on MFMA
    float sn[8], cs[8];
    const float delta = (float)(p.cstart + t - p.pos_q);
#pragma unroll
    for (int i = 0; i < 8; ++i) sincosf(delta * th[i], &sn[i], &cs[i]);
    float16v sacc = {};
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      half8 b0, b1;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float c = acc[j][i], d = acc[j][i + 8];
        b0[i] = (half_t)(c * cs[i] - d * sn[i]);
        b1[i] = (half_t)(d * cs[i] + c * sn[i]);
      }
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aq[j][0], b0, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aq[j][1], b1, sacc, 0, 0, 0);
    }
    // rows of sacc: 8*(i/4) + 4*hh + (i%4) = query head; column = token col
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 8 * (i >> 2) + 4 * hh + (i & 3);
      if (row < NQ) sp[P][row][col] = sacc[i];
    }
    __syncthreads();

    // 3a. online softmax over the tile (base 2, scores scaled by log2e/sqrt(D))
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int e = tid + kThreads * k;
      if (e < NQ * kTile) {
        const int qr = e >> 5, tt = e & 31;
        const int tok = t0 + tt;
        float s = -INFINITY;
        if (tok < t_end) {
          s = sp[0][qr][tt] + sp[1][qr][tt] + sp[2][qr][tt] + sp[3][qr][tt];
          s *= sc;
          if (p.mask) s += p.mask[(int64_t)b * p.mask_stride + p.n_sink + tok] * kLog2e;
        }
        float tmax = s;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o, 64));
        const float m_new = fmaxf(m_run[k], tmax);
        const float al = (m_new == -INFINITY) ? 1.f : exp2f(m_run[k] - m_new);
        const float pv = (s == -INFINITY) ? 0.f : exp2f(s - m_new);
        l_part[k] = l_part[k] * al + pv;
        m_run[k] = m_new;
        pp[tt][qr] = pv;
        if (tt == 0) alpha_s[qr] = al;
      }
    }
    __syncthreads();

    // 3b. VQ values: vacc[q][e] = alpha*vacc + sum_t p[q,t] * cb[idx[t,G]][e]
    {
      const float4 al4 = *(const float4*)&alpha_s[4 * vj];
      const float alv[4] = {al4.x, al4.y, al4.z, al4.w};
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int e = 0; e < 4; ++e) vacc[a][e] *= alv[a];
#pragma unroll
      for (int m = 0; m < kTile / TS; ++m) {
        const int tt = vts + TS * m;
        const float4 c4 = cbl[vcode[m]];
        const float4 p4 = *(const float4*)&pp[tt][4 * vj];
        const float pv[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          vacc[a][0] += pv[a] * c4.x;
          vacc[a][1] += pv[a] * c4.y;
          vacc[a][2] += pv[a] * c4.z;
          vacc[a][3] += pv[a] * c4.w;
        }
      }
    }
  }

  // ---- chunk epilogue: (m, l) per query head and the reduced accumulators
#pragma unroll
  for (int k = 0; k < SPT; ++k) {
    const int e = tid + kThreads * k;
    float l = l_part[k];
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
    if (e < NQ * kTile && (e & 31) == 0) {
      const int qr = e >> 5;
      const int qh = hg * NQ + qr;
      const int64_t widx = ((int64_t)b * p.H + qh) * p.n_splits + split;
      p.ws_m[widx] = m_run[k];
      p.ws_l[widx] = l;
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[tid][4 * a + e] = vacc[a][e];
  __syncthreads();
  if (vts == 0) {
    float sum[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) sum[i] = red[tid][i];
    for (int u = 1; u < TS; ++u)
#pragma unroll
      for (int i = 0; i < 16; ++i) sum[i] += red[tid + 32 * u][i];
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int qh = hg * NQ + 4 * vj + a;
      float* dst = p.ws_acc + (((int64_t)b * p.H + qh) * p.n_splits + split) * kHD + 4 * vG;
      *(float4*)dst = make_float4(sum[4 * a], sum[4 * a + 1], sum[4 * a + 2], sum[4 * a + 3]);
    }
  }
}

// --------------------------------------------------------------------------
// Combine: merge splits, fp16 segments and the 8-bit stream; one inverse FWHT.
// --------------------------------------------------------------------------
struct CombineParams {
  int32_t B, H, G, n_comp, n_splits;
  const uint16_t* q;
  const uint16_t* vch;
  const uint16_t *sink_k, *sink_v;
  int32_t n_sink;
  const uint16_t *win_k, *win_v;
  int32_t n_win;
  const uint16_t *dec_k, *dec_v;
  int32_t n_dec, dec_stride;
  const uint8_t *s_kidx, *s_vidx;
  const uint16_t *s_knorm, *s_vnorm;
  const float* s_signs;
  const float* s_cb;
  int32_t n_stream;
  const float* mask;
  int64_t mask_stride;
  const float* ws_m;
  const float* ws_l;
  const float* ws_acc;
  uint16_t* out;
};

// Butterflies over 128 values held as (lane, lane + 64); same pairing and
// per-op rounding as hadamard() (cache.py:10-19).
__device__ __forceinline__ void fwht128(float& x0, float& x1) {
  const int l = (int)lane_id();
#pragma unroll
  for (int h = 1; h < 64; h <<= 1) {
    const float p0 = __shfl_xor(x0, h, 64), p1 = __shfl_xor(x1, h, 64);
    x0 = (l & h) ? __fsub_rn(p0, x0) : __fadd_rn(x0, p0);
    x1 = (l & h) ? __fsub_rn(p1, x1) : __fadd_rn(x1, p1);
  }
  const float a = x0, c = x1;
  x0 = __fadd_rn(a, c);
  x1 = __fsub_rn(a, c);
  const float s = (float)sqrt(128.0);
  x0 = __fdiv_rn(x0, s);
  x1 = __fdiv_rn(x1, s);
}

// Stream token (K or V) as the reference dequantizes it (qjl off):
// fp16(fp16(hadamard(cb[idx]) * signs) * norm), returned in fp32.
__device__ __forceinline__ void stream_token(const uint8_t* idx, uint16_t norm_bits,
                                             const float* cb, const float* signs, float& y0,
                                             float& y1) {
  const int l = (int)lane_id();
  float x0 = cb[idx[l]], x1 = cb[idx[l + 64]];
  fwht128(x0, x1);
  const float n = h2f(norm_bits);
  y0 = h2f(f2h(h2f(f2h(__fmul_rn(x0, signs[l]))) * n));
  y1 = h2f(f2h(h2f(f2h(__fmul_rn(x1, signs[l + 64]))) * n));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Fetch extra token x (order: sink, window, decode, stream) of kv head g, row b.
__device__ __forceinline__ void extra_kv(const CombineParams& p, int b, int g, int x, bool want_v,
                                         const float* cb, const float* signs, float& y0,
                                         float& y1, int& mask_pos) {
  const int l = (int)lane_id();
  const uint16_t* src = nullptr;
  if (x < p.n_sink) {
    src = (want_v ? p.sink_v : p.sink_k) + (((int64_t)b * p.G + g) * p.n_sink + x) * kHD;
    mask_pos = x;
  } else if ((x -= p.n_sink) < p.n_win) {
    src = (want_v ? p.win_v : p.win_k) + (((int64_t)b * p.G + g) * p.n_win + x) * kHD;
    mask_pos = p.n_sink + p.n_comp + x;
  } else if ((x -= p.n_win) < p.n_dec) {
    src = (want_v ? p.dec_v : p.dec_k) + (((int64_t)b * p.G + g) * p.dec_stride + x) * kHD;
    mask_pos = p.n_sink + p.n_comp + p.n_win + x;
  } else {
    x -= p.n_dec;
    mask_pos = p.n_sink + p.n_comp + p.n_win + p.n_dec + x;
    const int64_t row = ((int64_t)x * p.B + b) * p.G + g;
    stream_token((want_v ? p.s_vidx : p.s_kidx) + row * kHD,
                 (want_v ? p.s_vnorm : p.s_knorm)[row], cb, signs, y0, y1);
    return;
  }
  y0 = h2f(src[l]);
  y1 = h2f(src[l + 64]);
}

__global__ __launch_bounds__(kThreads, 1)
void k_decode_combine(const CombineParams p) {
  __shared__ float sx[kGQA][kMaxExtra];
  __shared__ float wsp[kGQA][1024];
  __shared__ float cb[256];
  __shared__ float sg[kHD];
  __shared__ float Ms[kGQA], Ls[kGQA];
  __shared__ float red[4][kGQA][kHD];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = blockIdx.x, b = blockIdx.y;
  const int n_x = p.n_sink + p.n_win + p.n_dec + p.n_stream;
  if (p.n_stream > 0) {
    for (int i = tid; i < 256; i += kThreads) cb[i] = p.s_cb[i];
    for (int i = tid; i < kHD; i += kThreads) sg[i] = p.s_signs[i];
  }
  __syncthreads();

  const float inv_sqrt = 1.0f / sqrtf((float)kHD);
  float q0[kGQA], q1[kGQA];
#pragma unroll
  for (int a = 0; a < kGQA; ++a) {
    const uint16_t* qv = p.q + ((int64_t)b * p.H + g * kGQA + a) * kHD;
    q0[a] = h2f(qv[lane]);
    q1[a] = h2f(qv[lane + 64]);
  }

  // extra-token scores (natural log units, as the reference's fp32 scores)
  for (int x = w; x < n_x; x += 4) {
    float k0, k1;
    int mpos = 0;
    extra_kv(p, b, g, x, false, cb, sg, k0, k1, mpos);
    const float madd = p.mask ? p.mask[(int64_t)b * p.mask_stride + mpos] : 0.f;
#pragma unroll
    for (int a = 0; a < kGQA; ++a) {
      const float s = wave_sum(q0[a] * k0 + q1[a] * k1) * inv_sqrt + madd;
      if (lane == 0) sx[a][x] = s;
    }
  }
  __syncthreads();

  // per query head (wave w = head a): global max, weights, total sum
  {
    const int a = w;
    const int64_t base = ((int64_t)b * p.H + g * kGQA + a) * p.n_splits;
    float m = -INFINITY;
    for (int s = lane; s < p.n_splits; s += 64) m = fmaxf(m, p.ws_m[base + s] / kLog2e);
    for (int x = lane; x < n_x; x += 64) m = fmaxf(m, sx[a][x]);
    m = wave_max(m);
    float l = 0.f;
    for (int s = lane; s < p.n_splits; s += 64) {
      const float ms = p.ws_m[base + s];
      const float wv = (ms == -INFINITY) ? 0.f : exp2f(ms - m * kLog2e);
      wsp[a][s] = wv;
      l += wv * p.ws_l[base + s];
    }
    for (int x = lane; x < n_x; x += 64) {
      const float e = expf(sx[a][x] - m);
      sx[a][x] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) { Ms[a] = m; Ls[a] = l; }
  }
  __syncthreads();

  // compressed part: sum_s w_s acc_s, times ch, one inverse Hadamard
  float f0, f1;
  {
    const int a = w;
    const int64_t base = ((int64_t)b * p.H + g * kGQA + a) * p.n_splits;
    float s0 = 0.f, s1 = 0.f;
    for (int s = 0; s < p.n_splits; ++s) {
      const float wv = wsp[a][s];
      const float* ac = p.ws_acc + (base + s) * kHD;
      s0 += wv * ac[lane];
      s1 += wv * ac[lane + 64];
    }
    const uint16_t* ch = p.vch + ((int64_t)b * p.G + g) * kHD;
    f0 = s0 * h2f(ch[lane]);
    f1 = s1 * h2f(ch[lane + 64]);
    fwht128(f0, f1);
  }

  // fp16 segments and stream values
  float ax0[kGQA], ax1[kGQA];
#pragma unroll
  for (int a = 0; a < kGQA; ++a) { ax0[a] = 0.f; ax1[a] = 0.f; }
  for (int x = w; x < n_x; x += 4) {
    float v0, v1;
    int mpos;
    extra_kv(p, b, g, x, true, cb, sg, v0, v1, mpos);
#pragma unroll
    for (int a = 0; a < kGQA; ++a) {
      const float e = sx[a][x];
      ax0[a] += e * v0;
      ax1[a] += e * v1;
    }
  }
#pragma unroll
  for (int a = 0; a < kGQA; ++a) {
    red[w][a][lane] = ax0[a];
    red[w][a][lane + 64] = ax1[a];
  }
  __syncthreads();
  {
    const int a = w;
    const float t0 = red[0][a][lane] + red[1][a][lane] + red[2][a][lane] + red[3][a][lane];
    const float t1 = red[0][a][lane + 64] + red[1][a][lane + 64] + red[2][a][lane + 64] +
                     red[3][a][lane + 64];
    const float inv_l = 1.0f / Ls[a];
    uint16_t* o = p.out + ((int64_t)b * p.H + g * kGQA + a) * kHD;
    o[lane] = f2h((f0 + t0) * inv_l);
    o[lane + 64] = f2h((f1 + t1) * inv_l);
  }
}

inline int choose_splits(const shard_decode_args* a, int NB) {
  if (a->n_splits > 0) return ((a->n_splits + 7) / 8) * 8;
  const int HG = a->n_kv_heads / NB;
  int want = (256 + HG * a->batch - 1) / (HG * a->batch);
  int max_useful = (a->n_comp + kTile - 1) / kTile;
  if (want > max_useful) want = max_useful;
  if (want < 1) want = 1;
  want = ((want + 7) / 8) * 8;
  if (want > 1024) want = 1024;
  return want;
}

constexpr int kNB = 2;

template <int KS>
int launch_split(const SplitParams& sp, dim3 grid, hipStream_t s) {
  hipLaunchKernelGGL((k_decode_split<KS, kNB>), grid, dim3(kThreads), 0, s, sp);
  return 0;
}

}  // namespace shard

using namespace shard;

extern "C" {

size_t shard_decode_attn_workspace(const shard_decode_args* a) {
  if (!a || a->batch <= 0 || a->n_q_heads <= 0) return 0;
  const int ns = choose_splits(a, kNB);
  return (size_t)a->batch * a->n_q_heads * ns * (kHD + 2) * sizeof(float);
}

int shard_decode_attn(const shard_decode_args* a, void* workspace, size_t workspace_bytes,
                      void* stream) {
  if (!a || !a->q || !a->inv_freq || !a->k_coeffs || !a->k_coeff_scale || !a->k_basis ||
      !a->k_mean || !a->v_idx || !a->v_codebook || !a->v_ch || !a->out)
    return SHARD_ERR_ARG;
  if (a->batch <= 0 || a->n_comp <= 0) return SHARD_ERR_ARG;
  if (a->head_dim != kHD || a->n_q_heads != kGQA * a->n_kv_heads || a->n_kv_heads % kNB != 0)
    return SHARD_ERR_SHAPE;
  if (a->rank <= 0 || a->rank % 32 != 0 || a->rank > 192) return SHARD_ERR_SHAPE;
  const int n_x = a->n_sink + a->n_win + a->n_dec + a->n_stream;
  if (n_x > kMaxExtra) return SHARD_ERR_SHAPE;
  if ((a->n_sink && (!a->sink_k || !a->sink_v)) || (a->n_win && (!a->win_k || !a->win_v)) ||
      (a->n_dec && (!a->dec_k || !a->dec_v)) ||
      (a->n_stream && (!a->s_kidx || !a->s_vidx || !a->s_knorm || !a->s_vnorm || !a->s_signs ||
                       !a->s_codebook)))
    return SHARD_ERR_ARG;
  const int ns = choose_splits(a, kNB);
  if (ns > 1024) return SHARD_ERR_SHAPE;
  if (!workspace || workspace_bytes < shard_decode_attn_workspace(a)) return SHARD_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;

  float* ws = (float*)workspace;
  const int64_t nm = (int64_t)a->batch * a->n_q_heads * ns;
  SplitParams sp;
  sp.B = a->batch; sp.H = a->n_q_heads; sp.G = a->n_kv_heads; sp.rank = a->rank;
  sp.n_comp = a->n_comp; sp.cstart = a->compress_start; sp.pos_q = a->pos_q;
  sp.n_splits = ns;
  int chunk = (a->n_comp + ns - 1) / ns;
  chunk = ((chunk + kTile - 1) / kTile) * kTile;
  sp.chunk = chunk;
  sp.q = a->q; sp.inv_freq = a->inv_freq; sp.coef = a->k_coeffs; sp.cs = a->k_coeff_scale;
  sp.basis = a->k_basis; sp.mean = a->k_mean; sp.vidx = a->v_idx; sp.vcb = a->v_codebook;
  sp.mask = a->mask; sp.mask_stride = a->mask_stride; sp.n_sink = a->n_sink;
  sp.ws_m = ws; sp.ws_l = ws + nm; sp.ws_acc = ws + 2 * nm;

  dim3 grid((unsigned)(ns * (a->n_kv_heads / kNB)), (unsigned)a->batch);
  switch (a->rank / 16) {
    case 2: launch_split<2>(sp, grid, s); break;
    case 4: launch_split<4>(sp, grid, s); break;
    case 6: launch_split<6>(sp, grid, s); break;
    case 8: launch_split<8>(sp, grid, s); break;
    case 10: launch_split<10>(sp, grid, s); break;
    case 12: launch_split<12>(sp, grid, s); break;
    default: return SHARD_ERR_SHAPE;
  }
  SHARD_LAUNCH_CHECK("shard_decode_attn split");

  CombineParams cp;
  cp.B = a->batch; cp.H = a->n_q_heads; cp.G = a->n_kv_heads; cp.n_comp = a->n_comp;
  cp.n_splits = ns; cp.q = a->q; cp.vch = a->v_ch;
  cp.sink_k = a->sink_k; cp.sink_v = a->sink_v; cp.n_sink = a->n_sink;
  cp.win_k = a->win_k; cp.win_v = a->win_v; cp.n_win = a->n_win;
  cp.dec_k = a->dec_k; cp.dec_v = a->dec_v; cp.n_dec = a->n_dec; cp.dec_stride = a->dec_stride;
  cp.s_kidx = a->s_kidx; cp.s_vidx = a->s_vidx; cp.s_knorm = a->s_knorm; cp.s_vnorm = a->s_vnorm;
  cp.s_signs = a->s_signs; cp.s_cb = a->s_codebook; cp.n_stream = a->n_stream;
  cp.mask = a->mask; cp.mask_stride = a->mask_stride;
  cp.ws_m = sp.ws_m; cp.ws_l = sp.ws_l; cp.ws_acc = sp.ws_acc; cp.out = a->out;
  hipLaunchKernelGGL(k_decode_combine, dim3((unsigned)a->n_kv_heads, (unsigned)a->batch),
                     dim3(kThreads), 0, s, cp);
  SHARD_LAUNCH_CHECK("shard_decode_attn combine");
  return SHARD_OK;
}

}  // extern "C"
