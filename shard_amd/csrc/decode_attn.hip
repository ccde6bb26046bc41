// Fused decode attention over Shard's compressed KV cache, written for gfx950.
//
// One split launch + one merge launch per layer-step.  Two split kernels
// compute the same partial rows; shard_decode_attn picks one by the work per CU.
//
//   k_decode_split (row-split)  grid = (n_splits * n_kv, B), 256-thread
//     workgroups, two per CU, 4 query heads per kv head; one kv head x a chunk
//     of compressed tokens, walked 32 tokens at a time.  The 4 waves share each
//     tile: wave P rebuilds rows of the 16 RoPE pairs [16 P, 16 P + 16) (basis
//     operand in VGPRs), the partial scores meet in LDS, then a shared online
//     softmax and VQ value sum.  The last split of each head first runs the
//     extra tokens (at most 2048) into one more partial row per query head.
//   k_decode_tok (token-tiled)  grid = n_splits * n_kv * query groups * B,
//     512-thread workgroups, one per CU, 1, 2 or 4 query heads per workgroup;
//     the kv head's basis operand image sits in LDS and each wave takes whole
//     tiles (all 128 rows) of the split by a static map (results do not depend
//     on wave timing), with its own softmax state.
//     Every split owns a run of cost units (a compressed tile costs 3, a tile
//     of 32 extra tokens 1), so any number of extra tokens spreads over the
//     last splits.  The waves merge once at the end.
//   Per compressed tile, both:
//     1. rebuild the no-RoPE keys on chip with MFMA 32x32x16 f16:
//          16 K_n[rows, tok] = Basis'[rows, r] . coef[r, tok] + 16 mean
//        (coefficients: packed nibbles turned into exact fp16 integers by a
//        magic-number trick; the mean is one more k-step times a constant 1).
//        Keys never reach HBM.
//     2. rotate each (c, d) pair by its RoPE phase and dot with q on a second
//        MFMA (rows = query heads) - the relative-delta identity of
//        attention.py:3-6 in the row-split kernel, the equivalent absolute
//        form (q_rope rotated by the tile phase) in the token-tiled one.
//     3. online softmax (fp32, base 2) and the VQ values sum_t p_t cb[idx_t]
//        (rotated space) with the codebook in LDS.
//   Each workgroup applies ch and ONE inverse Hadamard to its VQ sum (both
//   linear, so they commute with the merge), adds the plain-basis sum of its
//   extra tokens and writes per (query head, split) the running max m, the
//   sum l and the 128-dim accumulator to the workspace.
//   k_decode_merge  grid = (n_q x slices, B): the log-sum-exp weighted sum
//     of the partial rows, normalized, written as fp16.
#include <algorithm>
#include <mutex>
#include <stdio.h>

#include "common.h"
#include "merge.h"

namespace shard {

constexpr int kThreads = 256;
constexpr int kTile = 32;         // tokens per MFMA tile
constexpr int kHD = 128;          // head_dim
constexpr int kGQA = 4;           // query heads per kv head
constexpr int kMaxExtra = 2048;   // sink + window + decode + stream tokens per call
constexpr int kMaxSplits = 1024;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyTau = 8.f;   // softmax numerators stay below 2^kLazyTau (lazily moved max)
constexpr int kBufWord3 = 0x00020000;  // buffer resource word 3: raw, unswizzled access (gfx9)
// rope tables of the per-layer operands (k_decode_prepare): in-tile column
// phases, the per-tile step, and the token-tiled kernel's two tile-offset tables
constexpr int kRopeEntries = 32 * 64 + 64 + 2 * 32 * 64;
constexpr int kRopeT2 = 32 * 64 + 64;       // (cos, sin)(32 b theta), b < 32
constexpr int kRopeT1 = kRopeT2 + 32 * 64;  // (cos, sin)(1024 a theta), a < 32
constexpr int kTokMaxTiles = 32 * 32;       // tiles per token-tiled chunk the tables cover
constexpr int kTokMaxRank = 256;            // the token-tiled kernel (the row-split one: 192)
#ifndef SHARD_SPLIT_PER_XCD
#define SHARD_SPLIT_PER_XCD 1
#endif
constexpr bool kSplitPerXcd = SHARD_SPLIT_PER_XCD;
// Row-split launches in two classes whose (batch row, kv head) groups fill
// the 8 XCDs evenly put every split of a group on one XCD and run the group's
// merge workgroups there too, so the merge reads the partial rows that XCD's
// L2 wrote (8K, batch 1: 13.86 -> 13.51 us).  SHARD_KV_XCD=0 keeps the split
// order of the other launches.
#ifndef SHARD_KV_XCD
#define SHARD_KV_XCD 1
#endif

// The fp16 segments around the compressed span, in attention-mask order:
// sink [0, n_sink), window, decode tokens, then the 8-bit stream (dequantized
// to fp16 rows as tokens arrive).
struct ExtraSegs {
  const uint16_t *sink_k, *sink_v;
  const uint16_t *win_k, *win_v;
  const uint16_t *dec_k, *dec_v;
  const uint16_t *s_k, *s_v;
  int32_t n_sink, n_win, n_dec, dec_stride, n_stream, n_x;
  // when set, the stream tokens of the call are the first *n_stream_dev of the
  // n_stream the launch was planned for (read at run time)
  const int32_t* n_stream_dev;
};

// The extra tokens of the call: n_x, less the planned stream rows past the
// device stream count when there is one.
__device__ __forceinline__ int extras_now(const ExtraSegs& s) {
  if (!s.n_stream_dev) return s.n_x;
  return s.n_x - s.n_stream + min(max(*s.n_stream_dev, 0), s.n_stream);
}

struct SplitParams {
  int32_t B, H, G, rank, n_comp, cstart, pos_q, n_splits;
  const int64_t* pos_q_dev;  // when set, pos_q is read from device memory
  // Token ranges: splits [0, n_first) cover `chunk` tokens each, the others
  // `chunk2` (two_class: the first and the second workgroup of each CU).
  int32_t chunk, chunk2, n_first, two_class;
  int32_t nsp;   // partial rows per (batch row, query head): n_splits (+1 with extra tokens)
  ExtraSegs xs;  // processed by the last split of each head before its compressed tiles
  const uint16_t* q;
  const float* inv_freq;
  const uint8_t* coef;
  const uint4* op;          // per-layer A operands (k_decode_prepare)
  const float2* rope;       // per-layer rotation tables (k_decode_prepare)
  const uint8_t* vidx;
  const uint16_t* vcb;
  const uint16_t* vch;
  const float* mask;
  int64_t mask_stride;
  int32_t n_sink;
  float* ws_m;
  float* ws_l;
  float* ws_acc;
  // kv_xcd (two_class launches whose (batch row, kv head) groups fill the 8
  // XCDs evenly): every split of a group on one XCD
  int32_t kv_xcd;
};

// 2^x for the online softmax, where x <= 0 (a difference from the running
// maximum): the hardware v_exp_f32 alone.  exp2f adds a range reduction that
// keeps full precision for results below 2^-126; such weights are below the
// fp32 resolution of a sum that holds at least one weight of 1.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// (x & m) | (y & ~m) in one VALU op; the compiler would emit and + or for
// literal masks (a three-operand op takes one literal at most).
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t x, uint32_t y) {
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(m), "v"(x), "v"(y));
  return r;
}

// 8 packed nibbles (n0 in bits 0-3 ... n7 in bits 28-31) -> 8 fp16 values in
// element order (n0, n4, n1, n5, n2, n6, n3, n7).  A nibble dropped into the
// mantissa of 1024.0 (0x6400) reads as 1024 + n from bits 0-3 of a half and
// as 1024 + 16 n from bits 4-7, both exact.  The basis operand carries 16 x the
// even ranks' entries (elements 0, 1, 4, 5) and 1 x the odd ranks' (2, 3, 6,
// 7), so rank r contributes 16 A'(r) (n - 8) plus a constant:
//   even: 16 A' (1024 + n) = 16 A' (n - 8) + 16512 A'
//   odd:     A' (1024 + 16 n) = 16 A' (n - 8) + 1152 A'
// and the mean k-step carries 16 mean minus those constants (k_decode_prepare),
// so the MFMA yields 16 K.  Five VALU ops per 8 values.  The offsets put the
// fp32 partial sums near 10^4 |A'|, whose rounding (about 1e-3 |A'|) stays
// below the fp16 rounding of the rotated keys.
__device__ __forceinline__ half8 nib8_to_mfma(uint32_t x) {
  const uint32_t x8 = x >> 8;
  const uint32_t m0 = 0x000F000Fu, m1 = 0x00F000F0u, magic = 0x64006400u;
  const uint4 r = make_uint4(bfi(m0, x, magic), bfi(m1, x, magic), bfi(m0, x8, magic),
                             bfi(m1, x8, magic));
  return __builtin_bit_cast(half8, r);
}

// element e of a converted dword holds nibble nib_perm(e)
__device__ __forceinline__ constexpr int nib_perm(int e) { return ((e & 1) << 2) | (e >> 1); }

// Wave-local row rho (0..31) of the MFMA tile -> head dim: rows 0..15 are the
// first components c of pairs 16P+rho, rows 16..31 the second components d.
__device__ __forceinline__ int row_dim(int P, int rho) {
  return rho < 16 ? 16 * P + rho : 64 + 16 * P + (rho - 16);
}

template <int KS>
__device__ __forceinline__ void load_coef(const uint8_t* rowp, bool valid, uint32_t (&cw)[KS]) {
  if (valid) {
    if constexpr (KS % 4 == 0) {
#pragma unroll
      for (int s = 0; s < KS; s += 4) {
        const uint4 v = *(const uint4*)(rowp + 4 * s);
        cw[s] = v.x; cw[s + 1] = v.y; cw[s + 2] = v.z; cw[s + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < KS; s += 2) {
        const uint2 v = *(const uint2*)(rowp + 4 * s);
        cw[s] = v.x; cw[s + 1] = v.y;
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < KS; ++s) cw[s] = 0x88888888u;  // nibble 8 -> coefficient 0
  }
}

// Per-layer constant operands (shard_decode_prepare), in HBM after compression:
//   op   uint4 [G][4 P][KS+1][64 lanes]: the MFMA A operand of wave P of head g,
//        k-steps 0..KS-1 = A'(r) = fp16(basis * coeff_scale) in the nibble order
//        of the coefficient dwords, times 16 for even ranks r (see
//        nib8_to_mfma); k-step KS = C = 16 mean - 16512 sum_{r even} A'(r)
//        - 1152 sum_{r odd} A'(r) as 16 bf16 parts (a bf16 MFMA against a
//        constant-1 operand), which cancels the 1024 offsets of the nibble
//        encoding:
//          16 sum_r A'(r)(n_r - 8) + 16 mean = C + sum_{r even} 16 A'(r)(1024 + n_r)
//                                              + sum_{r odd} A'(r)(1024 + 16 n_r)
//        The greedy split (each part the bf16 rounding of what remains) holds
//        C to fp32 precision at any magnitude the fp32 accumulators hold (fp16
//        parts would stop at 16 x 65504); the relative rounding of the sums
//        does not depend on the layer's scale.
//   rope float2 [32][64] = (cos, sin)(col * theta_i) for the token column inside
//        a tile, then float2 [64] = (cos, sin)(32 * theta_i), the per-tile step,
//        then the tile-offset tables of the token-tiled kernel: float2 [32][64] =
//        (cos, sin)(32 b theta_i) and float2 [32][64] = (cos, sin)(1024 a theta_i)
//        (tile k of a chunk is 32 (32 a + b) tokens from its start).
// Head pairs (hp = 1, head_dim-64 layers): G counts pairs of kv heads; pair g
// is one 128-dim head whose dims are [head 2g dims 0-31, head 2g+1 dims 0-31,
// head 2g dims 32-63, head 2g+1 dims 32-63], so that RoPE pairs (d, d + 32 of
// a 64-dim head) sit 64 apart as in a 128-dim head; the basis and mean rows
// are read in that order and inv_freq has 32 entries.
__device__ __forceinline__ int pair_row(int g, int vd) {
  return (2 * g + ((vd >> 5) & 1)) * 64 + 32 * (vd >> 6) + (vd & 31);
}

__global__ void k_decode_prepare(const uint16_t* __restrict__ basis, const uint16_t* __restrict__ cs,
                                 const uint16_t* __restrict__ mean, const float* __restrict__ inv_freq,
                                 int G, int rank, int hp, uint4* __restrict__ op, float2* __restrict__ rope) {
  const int KS = rank / 16;
  const int64_t n_op = (int64_t)G * 4 * (KS + 1) * 64;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_op + kRopeEntries; i += stride) {
    if (i < n_op) {
      const int lane = (int)(i % 64);
      const int s = (int)((i / 64) % (KS + 1));
      const int P = (int)((i / (64 * (KS + 1))) % 4);
      const int g = (int)(i / (64 * (KS + 1) * 4));
      const int col = lane & 31, hh = lane >> 5;
      const int row = hp ? pair_row(g, row_dim(P, col)) : g * kHD + row_dim(P, col);
      half8 v;
      uint16_t cb[8];  // the constant k-step's bf16 parts
      if (s < KS) {
        const int r0 = 8 * (KS * hh + s);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int r = r0 + nib_perm(e);
          const half_t a = (half_t)(h2f(basis[(int64_t)row * rank + r]) * h2f(cs[r]));
          v[e] = (e & 2) ? a : (half_t)(16.f * (float)a);  // elements 2, 3, 6, 7: odd ranks
        }
      } else {
        double c = 16.0 * (double)h2f(mean[row]);
        for (int r = 0; r < rank; ++r)
          c -= ((r & 1) ? 1152.0 : 16512.0) *
               (double)(float)(half_t)(h2f(basis[(int64_t)row * rank + r]) * h2f(cs[r]));
        // greedy split into 16 bf16 parts (8 per lane half), largest first
        for (int part = 0; part < 16; ++part) {
          const __bf16 h = (__bf16)(float)c;
          if (part >> 3 == hh) cb[part & 7] = __builtin_bit_cast(uint16_t, h);
          c -= (double)(float)h;
        }
      }
      op[i] = s < KS ? __builtin_bit_cast(uint4, v) : __builtin_bit_cast(uint4, cb);
    } else {
      const int k = (int)(i - n_op);
      const int fm = hp ? 31 : 63;  // pair -> inv_freq entry
      float sn, cn;
      if (k < 32 * 64) {
        sincosf((float)(k / 64) * inv_freq[k % 64 & fm], &sn, &cn);
      } else if (k < 32 * 64 + 64) {
        sincosf((float)kTile * inv_freq[(k - 32 * 64) & fm], &sn, &cn);
      } else {
        const int k2 = k - (32 * 64 + 64);  // tile-offset tables
        const int tab = k2 / (32 * 64), e = (k2 / 64) % 32, pi = k2 % 64;
        sincosf((float)(tab == 0 ? kTile * e : kTile * 32 * e) * inv_freq[pi & fm], &sn, &cn);
      }
      rope[k] = make_float2(cn, sn);
    }
  }
}

// A 32-bit load from a global address held as an integer (a row pointer
// broadcast from another lane): a global load, not a flat one, so the wait for
// it does not hold back LDS accesses.
__device__ __forceinline__ uint32_t ld_global_u32(uint64_t addr) {
  return *(const __attribute__((address_space(1))) uint32_t*)addr;
}

// Row x of the extra tokens (sink, window, decode, stream) of kv head g in
// batch row b (HD dims per row, G kv heads), and its column in the attention
// mask (the compressed span sits between the sink and the window).  *next =
// the element distance from this row to the same row of kv head g + 1: a
// segment's rows of one head are contiguous, stream rows hold the kv heads of
// a token side by side.
template <int HD = kHD>
__device__ __forceinline__ const uint16_t* extra_row(const ExtraSegs& s, int B, int G, int n_comp,
                                                     int b, int g, int x, bool v, int* mpos,
                                                     int* next = nullptr) {
  const int e1 = s.n_sink, e2 = e1 + s.n_win, e3 = e2 + s.n_dec;
  const int64_t bg = (int64_t)b * G + g;
  const uint16_t* base;
  int64_t row;
  int seg;
  if (x < e1) {
    base = v ? s.sink_v : s.sink_k;
    row = bg * s.n_sink + x;
    seg = s.n_sink;
  } else if (x < e2) {
    base = v ? s.win_v : s.win_k;
    row = bg * s.n_win + (x - e1);
    seg = s.n_win;
  } else if (x < e3) {
    base = v ? s.dec_v : s.dec_k;
    row = bg * s.dec_stride + (x - e2);
    seg = s.dec_stride;
  } else {
    base = v ? s.s_v : s.s_k;
    row = ((int64_t)(x - e3) * B + b) * G + g;
    seg = 1;
  }
  *mpos = x < e1 ? x : x + n_comp;
  if (next) *next = HD * seg;
  return base + row * HD;
}

// One butterfly stage at element stride 2*HL = lane stride HL.
template <int HL>
__device__ __forceinline__ void fwht_lane_stage(float& x0, float& x1, int l) {
  const float p0 = xor_lane<HL>(x0), p1 = xor_lane<HL>(x1);
  x0 = (l & HL) ? p0 - x0 : x0 + p0;
  x1 = (l & HL) ? p1 - x1 : x1 + p1;
}

// Butterflies over 128 values held as (2l, 2l+1) in lane l (Sylvester order).
// HALVES: two transforms of 64 (lanes 0-31 and 32-63), the stage across the
// halves left out and the scale 1/sqrt(64).
template <bool HALVES = false>
__device__ __forceinline__ void fwht128_pairs(float& x0, float& x1) {
  const int l = (int)lane_id();
  {
    const float a = x0, c = x1;
    x0 = a + c;
    x1 = a - c;
  }
  fwht_lane_stage<1>(x0, x1, l);
  fwht_lane_stage<2>(x0, x1, l);
  fwht_lane_stage<4>(x0, x1, l);
  fwht_lane_stage<8>(x0, x1, l);
  fwht_lane_stage<16>(x0, x1, l);
  if constexpr (!HALVES) fwht_lane_stage<32>(x0, x1, l);
  const float s = HALVES ? 0.125f : 0.08838834764831845f;  // 1/sqrt(64), 1/sqrt(128)
  x0 *= s;
  x1 *= s;
}

#ifndef SHARD_DECODE_TG
#define SHARD_DECODE_TG 1
#endif
#ifndef SHARD_SPLIT_BIAS
#define SHARD_SPLIT_BIAS 1
#endif
// With two workgroups per CU, the first-dispatched one runs a tile in about
// 1.15 us and the second in about 2.05 us while both are resident, and the
// second finishes its set-up about 1.3 tiles later (measured on MI355X at 8K
// and 32K).  Equal finishing times then give the first one
//   ta = 0.47 + 0.64 N  tiles  of every N = ta + tb.
// SHARD_SPLIT_BIAS=0 keeps even chunks.
constexpr bool kSplitBias = SHARD_SPLIT_BIAS;
// 32-token tiles a row-split workgroup processes side by side, one per group of
// 4 waves.  The default is 1: two 256-thread workgroups per CU, with the
// unequal chunks above.  SHARD_DECODE_TG=2 builds one 512-thread workgroup per
// CU working two tiles at once, which avoids the younger workgroup's tail but
// runs the two waves of each SIMD in the same phase; it measured slower on
// MI355X (19.2 vs 18.4 us at 8K) and is kept as a build option only.
constexpr int kTG = SHARD_DECODE_TG;
static_assert(kTG == 1 || kTG == 2, "SHARD_DECODE_TG must be 1 or 2");

// Extra tokens (sink, window, decode, stream; fp16 rows) of kv head g, run by
// the last split workgroup of the head before its compressed tiles, with NW
// waves.  Per pass of 32 NW tokens: scores on MFMA (rows = the kGQA query
// heads, k = head dims, columns = the wave's 32 tokens), online softmax per
// head (wave h < kGQA owns head h), values accumulated lane-per-dim pair.
// Writes partial row n_splits of each query head, in the plain (not rotated)
// basis.
template <int NW>
struct XtLds {
  float xsc[kGQA][32 * NW];     // scores of the pass (base 2)
  float xpw[32 * NW][kGQA];     // softmax numerators, [token][head]
  float2 xred[NW][kGQA][64];    // per-wave value sums
  float xal[kGQA];              // rescale of the running sums
};

template <int NW>
__device__ __forceinline__ void decode_extras_tail(const SplitParams& p, const int g, const int b,
                                                   XtLds<NW>& L) {
  constexpr int XT = 32 * NW;  // tokens per pass
  constexpr int XV = XT / 64;  // softmax values per lane
  auto& xsc = L.xsc;
  auto& xpw = L.xpw;
  auto& xred = L.xred;
  auto& xal = L.xal;

  const int tid = threadIdx.x, lane = tid & 63, col = lane & 31, hh = lane >> 5;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n_x = extras_now(p.xs);
  const float sc = kLog2e * 0.08838834764831845f;  // log2(e) / sqrt(128)

  half8 Aq[8];
  {
    const uint16_t* qv = p.q + ((int64_t)b * p.H + g * kGQA + min(col, kGQA - 1)) * kHD + 8 * hh;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const uint4 v4 = *(const uint4*)(qv + 16 * st);
      Aq[st] = __builtin_bit_cast(half8, col < kGQA ? v4 : make_uint4(0u, 0u, 0u, 0u));
    }
  }
  float m_run = -INFINITY, l_run = 0.f;  // softmax state of head w (w < kGQA)
  float2 acc[kGQA];
#pragma unroll
  for (int h = 0; h < kGQA; ++h) acc[h] = make_float2(0.f, 0.f);

  for (int x0 = 0; x0 < n_x; x0 += XT) {
    const int xt = min(x0 + 32 * w + col, n_x - 1);  // clamped: rows past n_x are masked
    int mpos;
    const uint16_t* krow = extra_row(p.xs, p.B, p.G, p.n_comp, b, g, xt, false, &mpos);
    const uint16_t* vrow = extra_row(p.xs, p.B, p.G, p.n_comp, b, g, xt, true, &mpos);
    half8 Bk[8];
#pragma unroll
    for (int st = 0; st < 8; ++st) Bk[st] = __builtin_bit_cast(half8, *(const uint4*)(krow + 16 * st + 8 * hh));
    const float madd = p.mask ? p.mask[(int64_t)b * p.mask_stride + mpos] * kLog2e : 0.f;
    uint32_t vx[32];
    const uint64_t vb = (uint64_t)vrow;
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)vb, t);
      const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(vb >> 32), t);
      vx[t] = ld_global_u32((((uint64_t)hi << 32) | lo) + 4 * lane);
    }
    float16v sacc = {};
#pragma unroll
    for (int st = 0; st < 8; ++st) sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aq[st], Bk[st], sacc, 0, 0, 0);
    if (hh == 0) {
      const bool valid = x0 + 32 * w + col < n_x;
#pragma unroll
      for (int i = 0; i < kGQA; ++i) xsc[i][32 * w + col] = valid ? sacc[i] * sc + madd : -INFINITY;
    }
    __syncthreads();
    if (w < kGQA) {  // wave w: online softmax of head w over the pass
      float s[XV];
      float mx = -INFINITY;
#pragma unroll
      for (int k = 0; k < XV; ++k) {
        s[k] = xsc[w][lane + 64 * k];
        mx = fmaxf(mx, s[k]);
      }
      const float m_new = fmaxf(m_run, wave64_reduce(mx, OpMax()));
      const float al = m_new == -INFINITY ? 1.f : fast_exp2(m_run - m_new);
      float ps = 0.f;
#pragma unroll
      for (int k = 0; k < XV; ++k) {
        const float pk = s[k] == -INFINITY ? 0.f : fast_exp2(s[k] - m_new);
        ps += pk;
        xpw[lane + 64 * k][w] = pk;
      }
      l_run = l_run * al + wave64_reduce(ps, OpAdd());
      m_run = m_new;
      if (lane == 0) xal[w] = al;
    }
    __syncthreads();
    const float4 al4 = *(const float4*)xal;
    acc[0].x *= al4.x; acc[0].y *= al4.x;
    acc[1].x *= al4.y; acc[1].y *= al4.y;
    acc[2].x *= al4.z; acc[2].y *= al4.z;
    acc[3].x *= al4.w; acc[3].y *= al4.w;
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      const float4 pw = *(const float4*)&xpw[32 * w + t][0];
      const half2v hv = __builtin_bit_cast(half2v, vx[t]);
      const float v0 = (float)hv[0], v1 = (float)hv[1];
      acc[0].x += pw.x * v0; acc[0].y += pw.x * v1;
      acc[1].x += pw.y * v0; acc[1].y += pw.y * v1;
      acc[2].x += pw.z * v0; acc[2].y += pw.z * v1;
      acc[3].x += pw.w * v0; acc[3].y += pw.w * v1;
    }
  }
#pragma unroll
  for (int h = 0; h < kGQA; ++h) xred[w][h][lane] = acc[h];
  __syncthreads();
  if (w < kGQA) {
    const int h = w;
    float2 t = xred[0][h][lane];
#pragma unroll
    for (int u = 1; u < NW; ++u) {
      const float2 a = xred[u][h][lane];
      t.x += a.x;
      t.y += a.y;
    }
    const int64_t widx = ((int64_t)b * p.H + g * kGQA + h) * p.nsp + p.n_splits;
    *(float2*)(p.ws_acc + widx * kHD + 2 * lane) = t;
    if (lane == 0) {
      p.ws_m[widx] = m_run;
      p.ws_l[widx] = l_run;
    }
  }
}

template <int KS, int TG>
__global__ __launch_bounds__(256 * TG, TG == 1 ? 2 : 1)
void k_decode_split(const SplitParams p) {
  constexpr int NT = 256 * TG;    // threads
  constexpr int TT = kTile * TG;  // tokens per iteration: one tile per group of 4 waves
  constexpr int NQ = kGQA;        // query heads of the workgroup's kv head
  constexpr int VT = 4;           // V-stage tokens per thread per iteration
  constexpr int TS = TT / VT;     // V-stage token subsets
  static_assert(TS * 32 == NT, "V stage: 32 dim groups x TS token subsets");
  static_assert(NQ * TT <= NT, "softmax: at most one entry per thread");

  __shared__ __align__(16) float sp[TG][4][NQ][kTile];  // per-wave partial scores
  __shared__ __align__(16) half_t pp16[NQ][TT];         // softmax numerators (fp16)
  __shared__ __align__(16) float alpha_s[NQ];           // rescale factors of the iteration
  __shared__ __align__(16) uint2 cbl[256];              // VQ codebook (4 x fp16 per entry)
  __shared__ __align__(16) float2 phq[64];              // (cos, sin)(pos_q * theta_i)
  __shared__ __align__(16) float2 phb[64];              // (cos, sin)(delta of the chunk start)
  __shared__ __align__(16) float2 phs[64];              // (cos, sin)(TT * theta_i)
  __shared__ __align__(16) float red[NT][17];           // end-of-chunk reduction

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int P = wv & 3;     // pair slice of the wave (16 RoPE pairs)
  const int grp = wv >> 2;  // tile of the iteration the wave works on
  const int col = lane & 31;
  const int hh = lane >> 5;

  // ---- block -> (kv head, split).  The dispatcher deals blocks to the 8
  // XCDs in turn (block id mod 8).  With n_splits % 8 == 0 all heads of one
  // split get block ids congruent mod 8, so they share one XCD and its L2
  // fetches the split's coefficient rows (read by every head) once; otherwise
  // consecutive blocks are consecutive heads of one split.
  //
  // two_class (exactly two workgroups per CU): the dispatcher fills one slot
  // of every CU with the first 256 workgroups and the second slot with the
  // next 256.  The older workgroup of a CU gets issue priority, so splits
  // [0, n_first) go to the first class with longer chunks and the second class
  // gets shorter ones; both then finish together.  Each class holds half the
  // splits of every (batch row, kv head).
  const int HG = p.G;
  const int bid = blockIdx.x;
  int hg, split, b;
  if (p.kv_xcd) {
    // every workgroup of a (batch row, kv head) group on one XCD (block id
    // mod 8): group x + 8 gi on XCD x, its splits of each class in one run
    const int L = blockIdx.y * gridDim.x + bid;  // dispatch order
    const int c = L >> 8, j = L & 255;
    const int r = j >> 3;
    const int grp_i = (j & 7) + 8 * (r / p.n_first);
    split = c * p.n_first + r % p.n_first;
    b = grp_i / HG;
    hg = grp_i % HG;
  } else if (p.two_class) {
    const int L = blockIdx.y * gridDim.x + bid;  // dispatch order
    const int c = L >> 8, j = L & 255;
    const int slot = j >> 3;
    hg = slot % HG;
    const int q = (slot / HG) * 8 + (j & 7);
    b = q / p.n_first;
    split = c * p.n_first + q % p.n_first;
  } else {
    if (kSplitPerXcd && (p.n_splits & 7) == 0) {
      const int slot = bid >> 3;
      hg = slot % HG;
      split = (slot / HG) * 8 + (bid & 7);
    } else {
      hg = bid % HG;
      split = bid / HG;
    }
    b = blockIdx.y;
  }
  // The last split of each head runs the extra tokens first (its compressed
  // chunk is shorter by their cost), so their cold loads overlap the other
  // workgroups' set-up instead of trailing the kernel.
  __shared__ __align__(16) XtLds<4 * TG> xt;
  if (split == p.n_splits - 1 && p.xs.n_x > 0) decode_extras_tail<4 * TG>(p, hg, b, xt);

  // ---- loads that feed LDS and the q operand go out first: the first barrier
  // waits for these only, not for the tile and basis loads behind them.
  const int pos_q = p.pos_q_dev ? (int)p.pos_q_dev[0] : p.pos_q;
  const uint2 cb_v = tid < 256 ? *(const uint2*)(p.vcb + 4 * tid) : make_uint2(0u, 0u);
  const float th_v = tid < 192 ? p.inv_freq[tid & 63] : 0.f;
  uint2 q_lo[2], q_hi[2];
  {
    const uint16_t* qv = p.q + ((int64_t)b * p.H + hg * NQ + min(col, NQ - 1)) * kHD;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int d0 = 16 * P + 8 * jj + 4 * hh;
      q_lo[jj] = *(const uint2*)(qv + d0);
      q_hi[jj] = *(const uint2*)(qv + d0 + 64);
    }
  }
  const int t_begin = split < p.n_first ? split * p.chunk
                                         : p.n_first * p.chunk + (split - p.n_first) * p.chunk2;
  int t_end = t_begin + (split < p.n_first ? p.chunk : p.chunk2);
  if (t_end > p.n_comp) t_end = p.n_comp;
  if (t_end <= t_begin) {
    // no compressed tokens (a last split that only holds the extra tokens):
    // the empty partial row is m = -inf, l = 0, acc = 0; skip the set-up
    if (tid < 64 * NQ) {
      const int64_t widx = ((int64_t)b * p.H + hg * NQ + wv) * p.nsp + split;
      *(float2*)(p.ws_acc + widx * kHD + 2 * lane) = make_float2(0.f, 0.f);
      if (lane == 0) {
        p.ws_m[widx] = -INFINITY;
        p.ws_l[widx] = 0.f;
      }
    }
    return;
  }

  // ---- first iteration's loads go out before the setup work.  Token indices
  // are clamped to the chunk (no divergent loads); rows past the chunk end get
  // -inf scores and zero weights.
  const int64_t coef_row_bytes = p.rank / 2;
  const int rowb = KS * 4;  // bytes per lane-half of a coefficient row
  const uint8_t* coef_b = p.coef + (int64_t)b * p.n_comp * coef_row_bytes + rowb * hh;
  const int vG = tid & 31;
  const int vts = tid >> 5;
  const uint8_t* vidx_b = p.vidx + (((int64_t)b * p.G + hg) * p.n_comp) * 32 + vG;
  const int t_last = t_end > t_begin ? t_end - 1 : t_begin;
  auto load_tile = [&](int t0, uint32_t (&cw_)[KS], uint32_t (&vc_)[VT]) {
    const int tc = min(t0 + kTile * grp + col, t_last);
    load_coef<KS>(coef_b + (int64_t)tc * coef_row_bytes, true, cw_);
#pragma unroll
    for (int m = 0; m < VT; ++m) vc_[m] = vidx_b[(int64_t)min(t0 + VT * vts + m, t_last) * 32];
  };
  uint32_t cwA[KS], vcA[VT], cwB[KS], vcB[VT];
  if (t_begin < t_end) load_tile(t_begin, cwA, vcA);

  // ---- per-layer constant operands: coalesced 16-byte loads
  half8 Ab[KS + 1];
  {
    const uint4* opp = p.op + ((int64_t)(hg * 4 + P) * (KS + 1)) * 64 + lane;
#pragma unroll
    for (int s = 0; s <= KS; ++s) Ab[s] = __builtin_bit_cast(half8, opp[s * 64]);
  }
  int pr[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) pr[i] = 16 * P + 8 * (i >> 2) + 4 * hh + (i & 3);
  float2 rc[8], r32[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    rc[i] = p.rope[col * 64 + pr[i]];  // (cos, sin)(col * theta)
    r32[i] = p.rope[32 * 64 + pr[i]];  // (cos, sin)(32 * theta)
  }

  if (tid < 256) cbl[tid] = cb_v;
  if (tid < 192) {
    const int k = tid >> 6;  // 0: q position, 1: chunk start delta, 2: iteration step
    const float x = k == 0 ? (float)pos_q * th_v
                  : k == 1 ? (float)(p.cstart + t_begin - pos_q) * th_v
                           : (float)TT * th_v;
    float sn, cn;
    sincosf(x, &sn, &cn);
    (k == 0 ? phq : k == 1 ? phb : phs)[tid & 63] = make_float2(cn, sn);
  }
  __syncthreads();

  // q_n = undo-RoPE(q_rope, pos_q): a = q_lo cos + q_hi sin, b = q_hi cos - q_lo sin
  half8 Aq[2];
  {
    float a_[8], b_[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { a_[i] = 0.f; b_[i] = 0.f; }
    if (col < NQ) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const uint2 lo4 = q_lo[jj], hi4 = q_hi[jj];
        const half2v l0 = __builtin_bit_cast(half2v, lo4.x), l1 = __builtin_bit_cast(half2v, lo4.y);
        const half2v h0 = __builtin_bit_cast(half2v, hi4.x), h1 = __builtin_bit_cast(half2v, hi4.y);
        const float lo[4] = {(float)l0[0], (float)l0[1], (float)l1[0], (float)l1[1]};
        const float hi[4] = {(float)h0[0], (float)h0[1], (float)h1[0], (float)h1[1]};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const float2 cq = phq[pr[4 * jj + m]];
          a_[4 * jj + m] = lo[m] * cq.x + hi[m] * cq.y;
          b_[4 * jj + m] = hi[m] * cq.x - lo[m] * cq.y;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      Aq[0][e] = (half_t)a_[e];
      Aq[1][e] = (half_t)b_[e];
    }
  }

  // ---- relative phase of this lane's token at the first iteration:
  // phi = delta(chunk start) * theta + (32 grp + col) * theta; advanced by
  // TT * theta per iteration
  float ph_c[8], ph_s[8];
  float2 rstep[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float2 bb = phb[pr[i]];
    float c = bb.x * rc[i].x - bb.y * rc[i].y;
    float s = bb.y * rc[i].x + bb.x * rc[i].y;
    if (grp) {
      const float c2 = c * r32[i].x - s * r32[i].y;
      s = s * r32[i].x + c * r32[i].y;
      c = c2;
    }
    ph_c[i] = c * 0.0625f;  // the rebuilt keys come out 16x: fold 1/16 in (exact)
    ph_s[i] = s * 0.0625f;
    rstep[i] = phs[pr[i]];
  }
  bf16x8 one8;  // the B operand of the constant k-step: 1 in all 16 k-elements
#pragma unroll
  for (int e = 0; e < 8; ++e) one8[e] = (__bf16)1.f;

  // ---- softmax-stage state: thread tid < NQ * TT owns (head tid / TT, token tid % TT)
  float m_run = -INFINITY, l_part = 0.f;
  const float sc = kLog2e * rsqrtf((float)kHD);

  float vacc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int e = 0; e < 4; ++e) vacc[a][e] = 0.f;

  auto tile = [&](const int t0, const uint32_t (&cw)[KS], const uint32_t (&vc)[VT]) {
    // 1. 16 x the no-RoPE keys of the wave's 32 rows for the group's 32 tokens
    //    (fp32): constant (k-step KS, times 1) + basis . coefficients
    const float16v zero16 = {};
    float16v acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, Ab[KS]), one8,
                                                          zero16, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ab[s], nib8_to_mfma(cw[s]), acc, 0, 0, 0);

    // 2. rotate pairs by phi(t, i), then dot with q_n on MFMA
    float16v sacc;
    {
      half8 b0, b1;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float c = acc[i], d = acc[i + 8];
        b0[i] = (half_t)(c * ph_c[i] - d * ph_s[i]);
        b1[i] = (half_t)(d * ph_c[i] + c * ph_s[i]);
      }
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aq[0], b0, zero16, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aq[1], b1, sacc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float c = ph_c[i] * rstep[i].x - ph_s[i] * rstep[i].y;
      const float s = ph_s[i] * rstep[i].x + ph_c[i] * rstep[i].y;
      ph_c[i] = c;
      ph_s[i] = s;
    }
    // rows of sacc: 8*(i/4) + 4*hh + (i%4) = query head; column = token col
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 8 * (i >> 2) + 4 * hh + (i & 3);
      if (row < NQ) sp[grp][P][row][col] = sacc[i];
    }
    __syncthreads();

    // the value operands of 3b (codebook entries of the thread's VT tokens,
    // read-only LDS) go out before the softmax, so their latency overlaps it
    half2v c2v[VT / 2][4];
#pragma unroll
    for (int u = 0; u < VT / 2; ++u) {
      const uint2 ca = cbl[vc[2 * u]], cb = cbl[vc[2 * u + 1]];
      c2v[u][0] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(cb.x, ca.x, 0x05040100u));
      c2v[u][1] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(cb.x, ca.x, 0x07060302u));
      c2v[u][2] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(cb.y, ca.y, 0x05040100u));
      c2v[u][3] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(cb.y, ca.y, 0x07060302u));
    }

    // 3a. online softmax over the iteration's TT tokens (base 2, scores scaled
    //     by log2e/sqrt(D)); a head's tokens fill one wave (TT = 64) or half
    if (tid < NQ * TT) {
      const int qr = tid / TT, tt = tid % TT;
      const int tok = t0 + tt;
      float s = -INFINITY;
      if (tok < t_end) {
        const int gg = tt >> 5, c = tt & 31;
        s = sp[gg][0][qr][c] + sp[gg][1][qr][c] + sp[gg][2][qr][c] + sp[gg][3][qr][c];
        s *= sc;
        if (p.mask) s += p.mask[(int64_t)b * p.mask_stride + p.n_sink + tok] * kLog2e;
      }
      // the reference max m_run moves (with the rescale of l and of the value
      // sums) only when a score exceeds it by more than kLazyTau: numerators
      // stay below 2^kLazyTau and most tiles skip the cross-lane max
      float al = 1.f;
      if (__builtin_amdgcn_ballot_w64(s > m_run + kLazyTau) != 0) {
        const float tmax = TT == 64 ? wave64_reduce(s, OpMax()) : half32_reduce(s, OpMax());
        const float m_new = fmaxf(m_run, tmax);
        al = (m_new == -INFINITY) ? 1.f : fast_exp2(m_run - m_new);
        l_part *= al;
        m_run = m_new;
      }
      const float pv = (s == -INFINITY) ? 0.f : fast_exp2(s - m_run);
      l_part += pv;
      pp16[qr][tt] = (half_t)pv;
      if (tt == 0) alpha_s[qr] = al;
    }
    __syncthreads();

    // 3b. VQ values (dot2 over token pairs, fp32 accumulation):
    //     vacc[q][e] = alpha * vacc + sum_t p[q,t] * cb[idx[t,G]][e]
    {
      const float4 al4 = *(const float4*)&alpha_s[0];
      const float alv[4] = {al4.x, al4.y, al4.z, al4.w};
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int e = 0; e < 4; ++e) vacc[a][e] *= alv[a];
      uint32_t pq[4][VT / 2];
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const uint32_t* src = (const uint32_t*)&pp16[a][VT * vts];
#pragma unroll
        for (int u = 0; u < VT / 2; ++u) pq[a][u] = src[u];
      }
#pragma unroll
      for (int u = 0; u < VT / 2; ++u) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const half2v p2 = __builtin_bit_cast(half2v, pq[a][u]);
#pragma unroll
          for (int e = 0; e < 4; ++e) vacc[a][e] = __builtin_amdgcn_fdot2(p2, c2v[u][e], vacc[a][e], false);
        }
      }
    }
  };

  for (int t0 = t_begin; t0 < t_end; t0 += 2 * TT) {
    // ping-pong buffers: the next iteration's loads are in flight during this one
    load_tile(t0 + TT, cwB, vcB);
    tile(t0, cwA, vcA);
    if (t0 + TT < t_end) {
      load_tile(t0 + 2 * TT, cwA, vcA);
      tile(t0 + TT, cwB, vcB);
    }
  }

  // ---- chunk epilogue: (m, l) per query head and the reduced accumulators
  if (tid < NQ * TT) {
    const float l = TT == 64 ? wave64_reduce(l_part, OpAdd()) : half32_reduce(l_part, OpAdd());
    if (tid % TT == 0) {
      const int64_t widx = ((int64_t)b * p.H + hg * NQ + tid / TT) * p.nsp + split;
      p.ws_m[widx] = m_run;
      p.ws_l[widx] = l;
    }
  }
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[tid][4 * a + e] = vacc[a][e];
  __syncthreads();
  // thread (vG, i): value i = 4 a + e of dim group vG, summed over the TS subsets
  __shared__ __align__(16) float racc[NQ][kHD];
  for (int i = tid >> 5; i < 16; i += NT / 32) {
    float s = red[vG][i];
#pragma unroll
    for (int u = 1; u < TS; ++u) s += red[32 * u + vG][i];
    racc[i >> 2][4 * vG + (i & 3)] = s;
  }
  __syncthreads();
  // wave h < NQ: ch and one inverse FWHT of query head h, so the partial row is
  // in the plain basis (the FWHT is linear and commutes with the merge)
  if (wv < NQ) {
    const uint32_t ch2 = *(const uint32_t*)(p.vch + ((int64_t)b * p.G + hg) * kHD + 2 * lane);
    const half2v chh = __builtin_bit_cast(half2v, ch2);
    const float2 rv = *(const float2*)&racc[wv][2 * lane];
    float x0 = rv.x * (float)chh[0], x1 = rv.y * (float)chh[1];
    fwht128_pairs(x0, x1);
    const int qh = hg * NQ + wv;
    *(float2*)(p.ws_acc + (((int64_t)b * p.H + qh) * p.nsp + split) * kHD + 2 * lane) = make_float2(x0, x1);
  }
}

// --------------------------------------------------------------------------
// Token-tiled split kernel: each wave rebuilds all 128 rows of its own tiles.
// --------------------------------------------------------------------------
// One 512-thread workgroup (8 waves, 2 per SIMD) per CU owns one kv head x a
// range of tiles.  The head's basis operand image (4 row blocks x (KS + 1)
// k-steps, 52 KB at rank 192) sits in LDS; the 32-token tiles p, p + 4,
// p + 8, ... go to SIMD p, whose two waves (p and p + 4) alternate over them
// (3 to 2 for the first-dispatched wave in splits of 64 tiles or more), and
// each wave works through its tiles with no workgroup barrier: per tile it
// unpacks the coefficients once, runs the 4 x (KS + 1) rebuild MFMAs with A
// from LDS, rotates, scores, and keeps its own online softmax and VQ value
// sums.  The waves merge once, after the loop, in a fixed order.  The
// tile-to-wave map is static (not claimed from a counter), so a call's result
// does not depend on the timing of the waves: repeated calls give the same
// bits.
//
// Tiles: the split's compressed tiles first, then its extra tiles (sink,
// window, decode and stream tokens as fp16 rows), round robin over the waves
// and with the same softmax state: scores against
// q_rope on MFMA, values lane-per-dim-pair in the plain basis.  The host
// spreads the extra tiles over the last splits (a compressed tile counts as 3
// cost units, an extra tile as 1), so any number of extra tokens runs on many
// workgroups.
//
// RoPE: undo-RoPE at pos_q followed by the relative rotation (pos_t - pos_q) of
// the reference (attention.py:3-6, 74-79) is the rotation of q_rope by -pos_t
// (pos_q cancels), so the score of token t is q_rope . R(pos_t theta) k_t with
// k_t the no-RoPE key.  For token t0 + col of a tile, pos_t theta = phi0 +
// col theta: the in-tile part is a constant per lane (table rc, with the 1/16 of
// the rebuilt keys folded in) and the tile part rotates q instead,
//   q . R(phi0 + phic) k = (R(-phi0) q) . (R(phic) k),
// one rotation of the query heads per tile (lane = pair).  phi0 of tile k of
// the split is its first token's phase composed with the per-layer tables
// (32 (k mod 32)) theta and (1024 (k / 32)) theta.
//
// Score layout (32x32 MFMA, rows = query heads): element i < 4 of lane half
// hh holds head 4 hh + i of token col = lane % 32.
//
// Epilogue: the 8 waves' states merge in LDS; per query head the VQ part (in
// the Hadamard-rotated basis) is scaled by ch and rotated back with one FWHT,
// the extra tokens' part (plain basis) added, and one partial row (m, l,
// acc[128]) written per (batch row, query head, split).  The FWHT is linear, so
// it commutes with the log-sum-exp merge of k_decode_merge.
//
// Head pairs (HP, head_dim-64 layers): kv heads 2g and 2g + 1 run as one
// 128-dim head g (G counts the pairs).  The rebuilt keys come from the pair's
// operand image (k_decode_prepare, hp = 1: dims [2g low, 2g+1 low, 2g high,
// 2g+1 high], RoPE pairs 64 apart); a query head reads its 64-dim q into its
// own head's pairs and zeros into the other's, so its scores are against its
// own head's keys, softmax scale 1/sqrt(64).  The V indices of the two heads
// (16 bytes per token each, in their own rows) form the 32 subvectors, the
// fp16 rows of the extra tokens are read per head, ch and the plain-basis
// sums are the two heads' 64 dims side by side, and the inverse Hadamard runs
// per 64 dims.  A query head keeps its own head's 64 dims (the first 64 of its
// partial row); the other half of its value sums is discarded.
constexpr int kTokWaves = 8;
constexpr int kTokThreads = 64 * kTokWaves;
constexpr int kShareMinTiles = 64;  // splits with fewer tiles give both waves of a SIMD equal shares

struct TokParams {
  int32_t B, H, G, QG, n_comp, cstart;  // QG: groups of NQ query heads per kv head
  int32_t n_ct, n_xt;      // compressed tiles (32 tokens each) and extra tiles
  int32_t n_splits, per_u; // splits per (batch row, kv head); cost units per split
  ExtraSegs xs;
  const uint16_t* q;
  const float* inv_freq;
  const uint8_t* coef;
  const uint4* op;
  const float2* rope;
  const uint8_t* vidx;
  const uint16_t* vcb;
  const uint16_t* vch;
  const float* mask;
  int64_t mask_stride;
  int32_t n_sink;
  float* ws_m;
  float* ws_l;
  float* ws_acc;
};

#ifndef SHARD_RC_PAD
#define SHARD_RC_PAD 8  // rows of 40 dwords: the two lane halves (pairs 4 apart) read other banks
#endif
template <int KS, int NQ>
struct TokLds {
  union {
    uint4 A[4][KS + 1][64];             // basis operand image of the kv head
    struct {                            // end-of-split merge (after the tile loops)
      float r[kTokWaves][NQ][kHD];      // value sums, rotated basis
      float pl[kTokWaves][NQ][kHD];     // value sums, plain basis (extra tokens)
      float m[kTokWaves][NQ];
      float l[kTokWaves][NQ];
    } red;
  } u;
  uint2 cb[256];                        // VQ codebook, 4 x fp16 per entry
  uint32_t rc[64][32 + SHARD_RC_PAD];   // [pair][col]: fp16 (cos, sin)(col theta) / 16
  uint16_t qr[kTokWaves][NQ + 1][2][64];  // per wave: R(-phi0) q (fp16, score k order); row NQ = 0
  uint16_t pa[kTokWaves][NQ + 1][32];     // per wave: fp16 numerators [head][token]; row NQ stays 0
  float xp[kTokWaves][32][NQ + 1];        // per wave: numerators of an extra tile, [token][head]
};

// Position in the score MFMA's k order (16 rb + 8 hh + e) of pair i, where the
// rebuild MFMA puts pair 16 rb + 8 (e / 4) + 4 hh + e % 4 in element e of lane half hh.
__device__ __forceinline__ int pair_k(int i) {
  const int pl = i & 15;
  return (i & ~15) + 8 * ((pl >> 2) & 1) + 4 * (pl >> 3) + (pl & 3);
}

template <int KS, int NQ, bool HP>
__global__ __launch_bounds__(kTokThreads, 1)
void k_decode_tok(const TokParams p) {
  static_assert(NQ >= 1 && NQ <= 4, "query heads per workgroup");
  constexpr int NW = kTokWaves;
  constexpr int NE = NQ < 4 ? NQ : 4;  // score elements holding heads, per lane half
  __shared__ __align__(16) TokLds<KS, NQ> L;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31;
  const int hh = lane >> 5;

  // ---- block -> (kv head, query group, batch row, split).  A kv head's
  // query heads are split into QG groups of NQ (4, 3, 2 or 1), each its own
  // workgroup.  The dispatcher deals blocks to the 8 XCDs in turn (block id
  // mod 8); with B n_splits % 8 == 0 the heads of one (batch row, split)
  // share an XCD, whose L2 then fetches the split's coefficient rows (read by
  // every head) once.
  const int HG = p.G * p.QG;
  const int bid = blockIdx.x;
  int vh, pair;  // vh = kv head * QG + query group; pair = b * n_splits + split
  if (((p.B * p.n_splits) & 7) == 0) {
    const int slot = bid >> 3;
    vh = slot % HG;
    pair = (slot / HG) * 8 + (bid & 7);
  } else {
    vh = bid % HG;
    pair = bid / HG;
  }
  const int hg = vh / p.QG;          // kv head
  const int qh0 = vh * NQ;           // first query head of the group
  const int b = pair / p.n_splits;
  const int split = pair - b * p.n_splits;

  // ---- the split's tiles.  Cost units: a compressed tile 3, an extra tile 1;
  // split s covers units [s per_u, (s + 1) per_u), compressed tile j belongs to
  // the split holding unit 3 j, extra tile x to the one holding unit 3 n_ct + x.
  const int uc = 3 * p.n_ct;
  const int u0 = split * p.per_u, u1 = min(u0 + p.per_u, uc + p.n_xt);
  const int ct0 = min((u0 + 2) / 3, p.n_ct), ct1 = min((u1 + 2) / 3, p.n_ct);
  const int xt0 = min(max(u0 - uc, 0), p.n_xt), xt1 = min(max(u1 - uc, 0), p.n_xt);
  const int n_c = ct1 > ct0 ? ct1 - ct0 : 0;
  const int n_x = xt1 > xt0 ? xt1 - xt0 : 0;
  const int n_xact = extras_now(p.xs);  // extra tokens of the call (<= 32 n_xt)

  // ---- raw buffers of the split's coefficient rows and V indices: rows past
  // the compressed span read as zeros (coefficient -8, centroid 0: finite;
  // their scores are set to -inf), and the offsets of a tile are one base +
  // immediates
  const int coef_row_bytes = 8 * KS;  // rank / 2
  const int r0 = 32 * ct0;
  const int n_rows = min(32 * ct1, p.n_comp) > r0 ? min(32 * ct1, p.n_comp) - r0 : 0;
  const __amdgpu_buffer_rsrc_t rcoef = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.coef + ((int64_t)b * p.n_comp + r0) * coef_row_bytes), (short)0,
      n_rows * coef_row_bytes, kBufWord3);
  // head pairs: each head of the pair has its own rows (16 bytes per token),
  // read through a buffer of its own (rvidx: the first head, rvidx2: the second)
  const uint8_t* vbase = HP ? p.vidx + (2 * ((int64_t)b * p.G + hg) * p.n_comp + r0) * 16
                            : p.vidx + (((int64_t)b * p.G + hg) * p.n_comp + r0) * 32;
  const __amdgpu_buffer_rsrc_t rvidx =
      __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, n_rows * (HP ? 16 : 32), kBufWord3);
  const __amdgpu_buffer_rsrc_t rvidx2 = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(vbase + (HP ? (int64_t)p.n_comp * 16 : 0)), (short)0, HP ? n_rows * 16 : 0, kBufWord3);
  // the additive mask row of batch row b: no mask reads as 0 (zero-length buffer)
  const int64_t n_keys = (int64_t)p.n_sink + p.n_comp + p.xs.n_x;
  const __amdgpu_buffer_rsrc_t rmask = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.mask ? p.mask + (int64_t)b * p.mask_stride : p.ws_m), (short)0,
      p.mask ? (int)(n_keys * 4) : 0, kBufWord3);
  // V stage on MFMA 16x16x32 f16: rows = query heads (NQ of 16 used), columns
  // = 16 subvectors, k = the tile's 32 tokens.  Lane (vn = lane % 16, vt =
  // lane / 16) holds tokens 8 vt .. 8 vt + 7 of subvector vn + 16 jg, jg = 0, 1.
  const int vn = lane & 15, vt = lane >> 4;
  auto load_vidx = [&](int k, uint32_t (&vi_)[16]) {
    if constexpr (HP) {
      const int voff = (32 * k + 8 * vt) * 16 + vn;
#pragma unroll
      for (int m = 0; m < 16; ++m)
        vi_[m] = __builtin_amdgcn_raw_buffer_load_b8((m >> 3) ? rvidx2 : rvidx, voff + 16 * (m & 7), 0, 0);
    } else {
      const int voff = (32 * k + 8 * vt) * 32 + vn;
#pragma unroll
      for (int m = 0; m < 16; ++m)
        vi_[m] = __builtin_amdgcn_raw_buffer_load_b8(rvidx, voff + 32 * (m & 7) + 16 * (m >> 3), 0, 0);
    }
  };
  const float2* t2tab = p.rope + kRopeT2 + lane;  // lane = pair
  const float2* t1tab = p.rope + kRopeT1 + lane;
  auto load_tile = [&](int k, uint32_t (&cw_)[KS], float2& f2, float2& f1) {
    const int kc = min(k, kTokMaxTiles - 1);  // a tile past the split: any valid entry (unused)
    f2 = t2tab[64 * (kc & 31)];
    f1 = t1tab[64 * (kc >> 5)];
    const int coff = (32 * k + col) * coef_row_bytes + KS * 4 * hh;
    if constexpr (KS % 4 == 0) {
#pragma unroll
      for (int s = 0; s < KS; s += 4) {
        const uint4 v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rcoef, coff + 4 * s, 0, 0));
        cw_[s] = v.x; cw_[s + 1] = v.y; cw_[s + 2] = v.z; cw_[s + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < KS; s += 2) {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rcoef, coff + 4 * s, 0, 0));
        cw_[s] = v.x; cw_[s + 1] = v.y;
      }
    }
  };
  // ---- the wave's compressed tiles (a static map: the result does not depend
  // on wave timing).  Waves p and p + 4 share a SIMD, whose arbiter favours
  // the first-dispatched one (w < 4): measured at 5.8K vs 7.7K clocks per tile
  // while both run.  SIMD p takes tiles p, p + 4, p + 8, ... (its j-th at
  // p + 4 j).  In a split of at least kShareMinTiles tiles the favoured wave
  // takes 3 of every 5 (j = 0, 2, 4 mod 5) and its partner 2 (j = 1, 3), so
  // the two finish closer together; shorter splits alternate (j even / odd).
  const int wp = w & 3;
  const bool w_old = w < 4;
  const bool uneven = n_c >= kShareMinTiles;
  auto tile_of = [&](int m) {  // index of this wave's m-th compressed tile
    int j;
    if (uneven) j = w_old ? 5 * (m / 3) + 2 * (m % 3) : 5 * (m >> 1) + 2 * (m & 1) + 1;
    else j = 2 * m + (w_old ? 0 : 1);
    return wp + 4 * j;
  };
  uint32_t cwA[KS], cwB[KS];
  float2 fA2, fA1, fB2, fB1;

  // every global load of the set-up goes out before the first LDS store, so
  // the cold misses overlap (one round trip instead of one per copy step)
  constexpr int kNA = 4 * (KS + 1) * 64;                       // uint4 of the image
  constexpr int kPA = (kNA + kTokThreads - 1) / kTokThreads;   // per thread
  constexpr int kPR = 32 * 64 / kTokThreads;                   // rope entries per thread
  uint4 av[kPA];
  float2 rv[kPR];
  {
    const uint4* src = p.op + (int64_t)hg * kNA;
#pragma unroll
    for (int j = 0; j < kPA; ++j) {
      const int i = tid + kTokThreads * j;
      av[j] = i < kNA ? src[i] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int j = 0; j < kPR; ++j) rv[j] = p.rope[tid + kTokThreads * j];
  }
  const uint2 cbv = tid < 256 ? *(const uint2*)(p.vcb + 4 * tid) : make_uint2(0u, 0u);
  const float th = p.inv_freq[HP ? (lane & 31) : lane];
  // head pairs: query heads per kv head; a query head's kv head is 2 hg + its half
  const int gq = HP ? p.H / (2 * p.G) : 1;
  uint16_t qlo[NQ], qhi[NQ];
  if constexpr (HP) {  // pairs 0..31: the pair's first head, 32..63 its second
    const uint16_t* qv = p.q + ((int64_t)b * p.H + qh0) * 64 + (lane & 31);
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      const bool mine = (((qh0 + h) / gq) & 1) == hh;
      qlo[h] = mine ? qv[h * 64] : (uint16_t)0;
      qhi[h] = mine ? qv[h * 64 + 32] : (uint16_t)0;
    }
  } else {
    const uint16_t* qv = p.q + ((int64_t)b * p.H + qh0) * kHD;
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      qlo[h] = qv[h * kHD + lane];
      qhi[h] = qv[h * kHD + 64 + lane];
    }
  }
  // the first tile's coefficients queue behind the set-up's loads: those are
  // needed first (the LDS stores before the barrier), the tile after it
  if (tile_of(0) < n_c) load_tile(tile_of(0), cwA, fA2, fA1);
  {
    uint4* dst = &L.u.A[0][0][0];
#pragma unroll
    for (int j = 0; j < kPA; ++j) {
      const int i = tid + kTokThreads * j;
      if (i < kNA) dst[i] = av[j];
    }
#pragma unroll
    for (int j = 0; j < kPR; ++j) {  // rope table [col][pair] -> rc[pair][col] / 16, fp16 pairs
      const int i = tid + kTokThreads * j;
      half2v hcs;
      hcs[0] = (half_t)(rv[j].x * 0.0625f);
      hcs[1] = (half_t)(rv[j].y * 0.0625f);
      L.rc[i & 63][i >> 6] = __builtin_bit_cast(uint32_t, hcs);
    }
  }
  if (tid < 256) L.cb[tid] = cbv;
  for (int i = tid; i < NW * 64; i += kTokThreads) {  // zero row NQ of each wave's rotated-q slot
    const int ww = i >> 6, k = i & 63;
    ((uint32_t*)&L.qr[ww][NQ][0][0])[k] = 0u;
  }

  // ---- per-lane pair state (lane = pair i): q_rope of the query heads, the
  // phase of the split's first compressed token
  float qa[NQ], qb[NQ];
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    qa[h] = h2f(qlo[h]);
    qb[h] = h2f(qhi[h]);
  }
  float bs_c, bs_s;
  sincosf((float)(p.cstart + r0) * th, &bs_s, &bs_c);
  const int kq = pair_k(lane);  // this lane's slot in the rotated-q rows
  int pr[8];                    // rc rows of this lane: pairs 16 rb + pr[i]
#pragma unroll
  for (int i = 0; i < 8; ++i) pr[i] = 8 * (i >> 2) + 4 * hh + (i & 3);
  const int qrow = min(col, NQ);  // rows >= NQ of the score MFMA read the zero row
  bf16x8 one8;  // the B operand of the constant k-step (bf16 parts of the image)
#pragma unroll
  for (int e = 0; e < 8; ++e) one8[e] = (__bf16)1.f;
  __syncthreads();

  const float sc = kLog2e * rsqrtf(HP ? 64.f : (float)kHD);
  float m_run[NE], l_part[NE];
  float4v vacc[2][4];  // [subvector group][component]: rows (heads) 4 vt + i, column vn
  float2 xacc[NQ];
#pragma unroll
  for (int i = 0; i < NE; ++i) {
    m_run[i] = -INFINITY;
    l_part[i] = 0.f;
  }
#pragma unroll
  for (int h = 0; h < NQ; ++h) xacc[h] = make_float2(0.f, 0.f);
#pragma unroll
  for (int jg = 0; jg < 2; ++jg)
#pragma unroll
    for (int e = 0; e < 4; ++e) vacc[jg][e] = float4v{0.f, 0.f, 0.f, 0.f};
  // the rescale of the value sums by the rows' softmax factors: row 4 vt + i
  // holds a head only for vt = 0, i < NQ (other rows are zero)
  auto rescale_v = [&](const float (&al)[NQ]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = al[i < NQ ? i : NQ - 1];
#pragma unroll
      for (int jg = 0; jg < 2; ++jg)
#pragma unroll
        for (int e = 0; e < 4; ++e) vacc[jg][e][i] *= a;
    }
  };

  // Online softmax of one tile's scores (lanes: token col; element i of lane
  // half hh: head 4 hh + i) with a lazily moved reference max.  The numerators
  // are 2^(s - m_run); m_run moves (with the rescale of l and of the value
  // sums) only when some score of the tile exceeds it by more than kLazyTau,
  // so every numerator stays below 2^kLazyTau (exact range for fp16) and most
  // tiles skip the cross-lane max and the rescale.  The partial rows carry
  // m_run as their max, so the merge is unchanged.  Returns whether m_run
  // moved (wave-uniform); then al[h] holds head h's rescale factor.  Stores
  // the numerators through put(row, pv), row NQ for lanes that hold no head
  // (every lane stores: no branch).
  auto softmax = [&](const float (&sv)[NE], int n_valid, int mpos, float (&al)[NQ], auto put) {
    const bool tok_ok = col < n_valid;
    const float madd = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rmask, 4 * mpos, 0, 0));
    float s[NE];
    bool over = false;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int h = 4 * hh + i;
      s[i] = (tok_ok && h < NQ) ? sv[i] * sc + madd * kLog2e : -INFINITY;
      over |= s[i] > m_run[i] + kLazyTau;
    }
    const bool moved = __builtin_amdgcn_ballot_w64(over) != 0;
    if (moved) {
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        const float m_new = fmaxf(m_run[i], half32_reduce(s[i], OpMax()));
        const float a = m_new == -INFINITY ? 1.f : fast_exp2(m_run[i] - m_new);
        l_part[i] *= a;
        m_run[i] = m_new;
#pragma unroll
        for (int hf = 0; hf < (NQ > 4 ? 2 : 1); ++hf)
          if (4 * hf + i < NQ) al[4 * hf + i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 32 * hf));
      }
    }
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int h = 4 * hh + i;
      const float pv = s[i] == -INFINITY ? 0.f : fast_exp2(s[i] - m_run[i]);
      l_part[i] += pv;
      put(h < NQ ? h : NQ, pv);
    }
    return moved;
  };

  // ---- one compressed tile (relative index k) on this wave
  auto tile = [&](const int k, const uint32_t (&cw)[KS], const float2 f2, const float2 f1) {
    const int t0 = 32 * (ct0 + k);
    uint32_t vi[16];  // V indices of the tile: needed at its end
    load_vidx(k, vi);
    // 1. q rotated by -phi0 of this tile -> the wave's qr slot (lane = pair)
    float ph_c = bs_c * f2.x - bs_s * f2.y;
    float ph_s = bs_s * f2.x + bs_c * f2.y;
    {
      const float c = ph_c * f1.x - ph_s * f1.y;
      ph_s = ph_s * f1.x + ph_c * f1.y;
      ph_c = c;
    }
#pragma unroll
    for (int h = 0; h < NQ; ++h) {
      L.qr[w][h][0][kq] = f2h(qa[h] * ph_c + qb[h] * ph_s);
      L.qr[w][h][1][kq] = f2h(qb[h] * ph_c - qa[h] * ph_s);
    }
    // 2. rebuild, k-step major: per k-step one converted coefficient operand
    //    feeds the 4 row blocks' independent accumulators.  The A operands
    //    stream from LDS through a ring of kRing registers, kRing reads ahead
    //    of the MFMA that consumes them (the order is pinned: the scheduler
    //    otherwise sinks each read to its MFMA and waits for it there).
    const float16v zero16 = {};
    float16v sacc = zero16;
    constexpr int kRing = 8;
    constexpr int NA = 4 * (KS + 1);  // A operands per tile, in (k-step, block) order
    auto a_at = [&](int j) {
      const int s = j >> 2, rb = j & 3;
      return __builtin_bit_cast(half8, L.u.A[rb][s == 0 ? KS : s - 1][lane]);
    };
    half8 ring[kRing];
#pragma unroll
    for (int j = 0; j < kRing; ++j) ring[j] = a_at(j);
    __builtin_amdgcn_sched_group_barrier(0x100, kRing, 0);
    float16v acc[4];
#pragma unroll
    for (int s = 0; s <= KS; ++s) {
      const half8 bs = s == 0 ? half8{} : nib8_to_mfma(cw[s - 1]);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const int j = 4 * s + rb;
        const half8 a = ring[j % kRing];
        if (j + kRing < NA) ring[j % kRing] = a_at(j + kRing);
        if (s == 0)  // the constant k-step: bf16 parts
          acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), one8, zero16, 0, 0, 0);
        else
          acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bs, acc[rb], 0, 0, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (j + kRing < NA) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        half8 b0, b1;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const half2v rr = __builtin_bit_cast(half2v, L.rc[16 * rb + pr[i]][col]);
          const float c = acc[rb][i], d = acc[rb][i + 8];
          // c cos - d sin, d cos + c sin: fp32 products and sums, one fp16 rounding
          b0[i] = (half_t)__builtin_fmaf(c, (float)rr[0], -__builtin_fmaf(d, (float)rr[1], 0.0f));
          b1[i] = (half_t)__builtin_fmaf(d, (float)rr[0], __builtin_fmaf(c, (float)rr[1], 0.0f));
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const half8 qa8 = *(const half8*)&L.qr[w][qrow][0][16 * rb + 8 * hh];
        const half8 qb8 = *(const half8*)&L.qr[w][qrow][1][16 * rb + 8 * hh];
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qa8, b0, sacc, 0, 0, 0);
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qb8, b1, sacc, 0, 0, 0);
      }
    }
    // 3. the value operands of step 4 (codebook lookups, read-only LDS) go out
    //    before the softmax, so their latency overlaps it: B_e = component e of
    //    the codebook entries of the lane's 8 tokens in subvector vn + 16 jg
    uint4 bw[2][4];
#pragma unroll
    for (int jg = 0; jg < 2; ++jg) {
      uint2 en[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) en[t] = L.cb[vi[8 * jg + t]];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        bw[jg][e].x = __builtin_amdgcn_perm(e < 2 ? en[1].x : en[1].y, e < 2 ? en[0].x : en[0].y, sel);
        bw[jg][e].y = __builtin_amdgcn_perm(e < 2 ? en[3].x : en[3].y, e < 2 ? en[2].x : en[2].y, sel);
        bw[jg][e].z = __builtin_amdgcn_perm(e < 2 ? en[5].x : en[5].y, e < 2 ? en[4].x : en[4].y, sel);
        bw[jg][e].w = __builtin_amdgcn_perm(e < 2 ? en[7].x : en[7].y, e < 2 ? en[6].x : en[6].y, sel);
      }
    }
    //    online softmax of the query heads over the tile
    float sv[NE], al[NQ];
#pragma unroll
    for (int i = 0; i < NE; ++i) sv[i] = sacc[i];
    const bool moved = softmax(sv, p.n_comp - t0, p.n_sink + t0 + col, al,
                               [&](int row, float pv) { L.pa[w][row][col] = f2h(pv); });
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // 4. VQ values of the tile on MFMA: A = the numerators of the query heads
    //    (row vn, tokens 8 vt ..), B as above
    if (moved) rescale_v(al);
    const half8 pa8 = __builtin_bit_cast(half8, *(const uint4*)&L.pa[w][vn < NQ ? vn : NQ][8 * vt]);
#pragma unroll
    for (int jg = 0; jg < 2; ++jg)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        vacc[jg][e] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa8, __builtin_bit_cast(half8, bw[jg][e]),
                                                             vacc[jg][e], 0, 0, 0);
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // pa is rewritten by the next tile
  };

  // ---- one extra tile (relative index x): fp16 K (RoPE applied) and V rows
  half8 Aq[8];  // rows = query heads (rows >= NQ zero), k = head dims; loaded at the first extra tile
  bool aq_loaded = false;
  auto xtile = [&](const int x) {
    if (!aq_loaded) {
      if constexpr (HP) {  // k chunk st: 16 dims of slot st / 2 = (first low, second low, first high, second high)
        const int qh = qh0 + min(col, NQ - 1);
        const int own = (qh / gq) & 1;
        const uint16_t* qv = p.q + ((int64_t)b * p.H + qh) * 64 + 8 * hh;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
          const int slot = st >> 1;
          const bool use = col < NQ && (slot & 1) == own;
          const uint4 v4 = use ? *(const uint4*)(qv + 32 * (slot >> 1) + 16 * (st & 1))
                               : make_uint4(0u, 0u, 0u, 0u);
          Aq[st] = __builtin_bit_cast(half8, v4);
        }
      } else {
        const uint16_t* qv = p.q + ((int64_t)b * p.H + qh0 + min(col, NQ - 1)) * kHD + 8 * hh;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
          const uint4 v4 = *(const uint4*)(qv + 16 * st);
          Aq[st] = __builtin_bit_cast(half8, col < NQ ? v4 : make_uint4(0u, 0u, 0u, 0u));
        }
      }
      aq_loaded = true;
    }
    const int n_xtok = n_xact;
    const int x0 = 32 * (xt0 + x);
    const int xt = min(x0 + col, n_xtok - 1);  // clamped: tokens past n_x are masked
    int mp;
    half8 Bk[8];
    uint32_t vx[32];
    if constexpr (HP) {
      // rows of the pair's first head (kv head 2 hg, 64 dims); the second's
      // are nx elements on.  V: lanes 32..63 hold the second head's row.
      int nx;
      const uint16_t* krow = extra_row<64>(p.xs, p.B, 2 * p.G, p.n_comp, b, 2 * hg, xt, false, &mp, &nx);
      const uint16_t* vrow = extra_row<64>(p.xs, p.B, 2 * p.G, p.n_comp, b, 2 * hg, xt, true, &mp) +
                             (hh ? nx : 0);
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        const int slot = st >> 1;
        Bk[st] = __builtin_bit_cast(
            half8, *(const uint4*)(krow + ((slot & 1) ? nx : 0) + 32 * (slot >> 1) + 16 * (st & 1) + 8 * hh));
      }
      const uint64_t vb = (uint64_t)vrow;
#pragma unroll
      for (int t = 0; t < 32; ++t) {
        const uint32_t lo0 = __builtin_amdgcn_readlane((uint32_t)vb, t);
        const uint32_t hi0 = __builtin_amdgcn_readlane((uint32_t)(vb >> 32), t);
        const uint32_t lo1 = __builtin_amdgcn_readlane((uint32_t)vb, 32 + t);
        const uint32_t hi1 = __builtin_amdgcn_readlane((uint32_t)(vb >> 32), 32 + t);
        const uint64_t row = hh ? (((uint64_t)hi1 << 32) | lo1) : (((uint64_t)hi0 << 32) | lo0);
        vx[t] = ld_global_u32(row + 4 * (lane & 31));
      }
    } else {
      const uint16_t* krow = extra_row(p.xs, p.B, p.G, p.n_comp, b, hg, xt, false, &mp);
      const uint16_t* vrow = extra_row(p.xs, p.B, p.G, p.n_comp, b, hg, xt, true, &mp);
#pragma unroll
      for (int st = 0; st < 8; ++st) Bk[st] = __builtin_bit_cast(half8, *(const uint4*)(krow + 16 * st + 8 * hh));
      const uint64_t vb = (uint64_t)vrow;
#pragma unroll
      for (int t = 0; t < 32; ++t) {
        const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)vb, t);
        const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(vb >> 32), t);
        vx[t] = ld_global_u32((((uint64_t)hi << 32) | lo) + 4 * lane);
      }
    }
    float16v sacc = {};
#pragma unroll
    for (int st = 0; st < 8; ++st) sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aq[st], Bk[st], sacc, 0, 0, 0);
    float sv[NE], al[NQ];
#pragma unroll
    for (int i = 0; i < NE; ++i) sv[i] = sacc[i];
    const bool moved = softmax(sv, n_xtok - x0, mp, al, [&](int row, float pv) { L.xp[w][col][row] = pv; });
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (moved) {
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        xacc[h].x *= al[h];
        xacc[h].y *= al[h];
      }
      rescale_v(al);
    }
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      const half2v hv = __builtin_bit_cast(half2v, vx[t]);
      const float v0 = (float)hv[0], v1 = (float)hv[1];
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        const float pt = L.xp[w][t][h];
        xacc[h].x += pt * v0;
        xacc[h].y += pt * v1;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");  // xp is rewritten by the next tile
  };

  // compressed tiles tile_of(0), tile_of(1), ... (increasing): ping-pong, the
  // next tile's loads fly during the current one
  int k = tile_of(0);
  for (int m = 0; k < n_c; m += 2) {
    const int kb = tile_of(m + 1);
    if (kb < n_c) load_tile(kb, cwB, fB2, fB1);
    tile(k, cwA, fA2, fA1);
    if (kb >= n_c) break;
    k = tile_of(m + 2);
    if (k < n_c) load_tile(k, cwA, fA2, fA1);
    tile(kb, cwB, fB2, fB1);
  }
  // extra tiles w, w + NW, ... (those holding tokens of this call)
  for (int x = w; x < n_x && 32 * (xt0 + x) < n_xact; x += NW) xtile(x);

  // ---- merge the waves; per query head: ch, one inverse FWHT, plain part
#pragma unroll
  for (int i = 0; i < NE; ++i) l_part[i] = half32_reduce(l_part[i], OpAdd());
  __syncthreads();  // every wave is done with the image the merge buffer overlays
  if (vt == 0) {  // rows 0..3 of the value sums: head i, subvector vn + 16 jg
#pragma unroll
    for (int i = 0; i < NQ; ++i)
#pragma unroll
      for (int jg = 0; jg < 2; ++jg)
        *(float4*)&L.u.red.r[w][i][4 * (vn + 16 * jg)] =
            make_float4(vacc[jg][0][i], vacc[jg][1][i], vacc[jg][2][i], vacc[jg][3][i]);
  }
#pragma unroll
  for (int h = 0; h < NQ; ++h) *(float2*)&L.u.red.pl[w][h][2 * lane] = xacc[h];
  if (col == 0) {
#pragma unroll
    for (int i = 0; i < NE; ++i)
      if (4 * hh + i < NQ) {
        L.u.red.m[w][4 * hh + i] = m_run[i];
        L.u.red.l[w][4 * hh + i] = l_part[i];
      }
  }
  __syncthreads();
  const uint32_t ch2 = *(const uint32_t*)(p.vch + ((int64_t)b * p.G + hg) * kHD + 2 * lane);
  const half2v chh = __builtin_bit_cast(half2v, ch2);
  for (int h = w; h < NQ; h += NW) {
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, L.u.red.m[ww][h]);
    float r0v = 0.f, r1v = 0.f, p0 = 0.f, p1 = 0.f, l = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float mw = L.u.red.m[ww][h];
      const float wt = mw == -INFINITY ? 0.f : exp2f(mw - M);
      const float2 rvv = *(const float2*)&L.u.red.r[ww][h][2 * lane];
      const float2 pvv = *(const float2*)&L.u.red.pl[ww][h][2 * lane];
      r0v += wt * rvv.x; r1v += wt * rvv.y;
      p0 += wt * pvv.x; p1 += wt * pvv.y;
      l += wt * L.u.red.l[ww][h];
    }
    r0v *= (float)chh[0];
    r1v *= (float)chh[1];
    fwht128_pairs<HP>(r0v, r1v);
    const int64_t widx = ((int64_t)b * p.H + qh0 + h) * p.n_splits + split;
    if (HP) {  // the query head's own head: its 64 dims first in the row
      if (hh == (((qh0 + h) / gq) & 1))
        *(float2*)(p.ws_acc + widx * kHD + 2 * (lane & 31)) = make_float2(r0v + p0, r1v + p1);
    } else {
      *(float2*)(p.ws_acc + widx * kHD + 2 * lane) = make_float2(r0v + p0, r1v + p1);
    }
    if (lane == 0) {
      p.ws_m[widx] = M;
      p.ws_l[widx] = l;
    }
  }
}

// Which split kernel runs.  The row-split kernel takes query groups of 4 and
// at most kMaxExtra extra tokens; the token-tiled kernel takes every supported
// shape.  Automatic choice by the work per CU: the token-tiled kernel has the
// higher tile throughput but a longer set-up, so it takes over from 9
// head-tiles per CU (measured on MI355X, row-split vs token-tiled, us per
// call: batch 1 x 8K (7.9 per CU) 14.5-14.6 vs 14.8; 1 x 10K (9.9) 16.2 vs
// 15.3; 1 x 12K 18.0 vs 17.7; 2 x 8K 20.5 vs 17.9; 1 x 16K 19.4-19.8 vs 17.8).
constexpr int kTokMinHeadTilesPerCU = 9;

inline int device_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
  }
  return n;
}

inline int64_t n_extra(const shard_decode_args* a) {
  return (int64_t)a->n_sink + a->n_win + a->n_dec + a->n_stream;
}

// The token-tiled kernel's kv heads: head_dim-64 layers run their kv heads in
// pairs (one 128-dim head per pair).
inline bool head_pairs(const shard_decode_args* a) { return a->head_dim == 64; }
inline int tok_g(const shard_decode_args* a) {
  return head_pairs(a) ? a->n_kv_heads / 2 : a->n_kv_heads;
}

// head_dim 128, or 64 with an even number of kv heads; up to 64 query heads
// per kernel kv head, in groups of NQ (4, 3, 2 or 1: the largest dividing the
// count) per workgroup
inline bool tok_supported(const shard_decode_args* a) {
  if ((a->head_dim != kHD && a->head_dim != 64) || a->n_kv_heads <= 0 || a->n_q_heads <= 0 ||
      a->n_q_heads % a->n_kv_heads)
    return false;
  // the value stage reads 4-value subvectors from a 256-row codebook in LDS
  if ((a->v_group != 0 && a->v_group != 4) || (a->v_codebook_n != 0 && a->v_codebook_n != 256))
    return false;
  if (head_pairs(a) && (a->n_kv_heads & 1)) return false;
  const int g = a->n_q_heads / tok_g(a);
  return g <= 64 && a->rank > 0 && a->rank % 32 == 0 && a->rank <= kTokMaxRank;
}

inline int tok_nq(const shard_decode_args* a) {
  const int g = a->n_q_heads / tok_g(a);
  return g % 4 == 0 ? 4 : g % 3 == 0 ? 3 : g % 2 == 0 ? 2 : 1;
}

inline bool split_supported(const shard_decode_args* a) {
  return a->head_dim == kHD && a->n_q_heads == kGQA * a->n_kv_heads && a->rank > 0 &&
         a->rank % 32 == 0 && a->rank <= 192 && n_extra(a) <= kMaxExtra;
}

// The row-split kernel runs every extra token in its last split, one pass of
// 128 after another; beyond this many the token-tiled kernel, which spreads
// them over splits, is faster (measured at 8K: 18.6 vs 18.8 us with 268 extra
// tokens, 23.3 vs 21.9 with 468, 34.3 vs 22.7 with 1,068).
constexpr int kRowSplitMaxExtraAuto = 256;

// kernel = 1 asks for the row-split kernel; a call it cannot take (query
// groups other than 4, more than kMaxExtra extra tokens: the reference appends
// stream tokens without limit, cache.py:156-181) runs on the token-tiled one.
inline bool use_tok(const shard_decode_args* a) {
  if (a->kernel == 2) return true;
  if (a->kernel == 1) return !split_supported(a);
  if (!split_supported(a) || n_extra(a) > kRowSplitMaxExtraAuto) return true;
  const int64_t tiles = (int64_t)((a->n_comp + kTile - 1) / kTile) * a->n_kv_heads * a->batch;
  return tiles >= (int64_t)kTokMinHeadTilesPerCU * device_cus();
}

// Row-split kernel: splits per (batch row, kv head), two workgroups per CU.
inline int split_count(const shard_decode_args* a) {
  const int max_useful = (a->n_comp + kTile - 1) / kTile;
  int want = a->n_splits > 0 ? a->n_splits
                             : (kTG == 1 ? 2 : 1) * device_cus() / (a->n_kv_heads * a->batch);
  if (want > max_useful) want = max_useful;
  if (want < 1) want = 1;
  if (want > kMaxSplits) want = kMaxSplits;
  return want;
}

// Token-tiled kernel: the split count and the cost units per split.
struct TokPlan {
  int n_ct, n_xt, ns, per_u;
};

inline TokPlan tok_plan(const shard_decode_args* a) {
  TokPlan w;
  w.n_ct = (a->n_comp + kTile - 1) / kTile;
  w.n_xt = (int)((n_extra(a) + kTile - 1) / kTile);
  const int64_t U = 3LL * w.n_ct + w.n_xt;
  // one 8-wave workgroup per CU: n_splits x (kv heads x query groups) x batch
  // workgroups fill the CUs once
  const int G = tok_g(a);
  const int qg = a->n_q_heads / G / tok_nq(a);
  int64_t want = a->n_splits > 0 ? a->n_splits
                                 : std::max(1, device_cus() / std::max(1, G * qg * a->batch));
  want = std::min<int64_t>(std::max<int64_t>(want, 1), std::max<int64_t>(U, 1));
  int64_t per = (U + want - 1) / want;
  per = std::min<int64_t>(per, 3LL * kTokMaxTiles);  // compressed tiles per split: phase tables
  w.per_u = (int)std::max<int64_t>(per, 1);
  w.ns = (int)((U + w.per_u - 1) / w.per_u);
  return w;
}

template <int KS>
void launch_tok(const TokParams& tp, int nq, bool hp, dim3 grid, hipStream_t s) {
  if (hp) {  // head pairs: an even number of query heads per pair, groups of 2, 3 or 4
    switch (nq) {
      case 2: hipLaunchKernelGGL((k_decode_tok<KS, 2, true>), grid, dim3(kTokThreads), 0, s, tp); break;
      case 3: hipLaunchKernelGGL((k_decode_tok<KS, 3, true>), grid, dim3(kTokThreads), 0, s, tp); break;
      default: hipLaunchKernelGGL((k_decode_tok<KS, 4, true>), grid, dim3(kTokThreads), 0, s, tp); break;
    }
    return;
  }
  switch (nq) {
    case 1: hipLaunchKernelGGL((k_decode_tok<KS, 1, false>), grid, dim3(kTokThreads), 0, s, tp); break;
    case 2: hipLaunchKernelGGL((k_decode_tok<KS, 2, false>), grid, dim3(kTokThreads), 0, s, tp); break;
    case 3: hipLaunchKernelGGL((k_decode_tok<KS, 3, false>), grid, dim3(kTokThreads), 0, s, tp); break;
    default: hipLaunchKernelGGL((k_decode_tok<KS, 4, false>), grid, dim3(kTokThreads), 0, s, tp); break;
  }
}

int launch_merge(const shard_decode_args* a, const float* ws, int nsp, hipStream_t s,
                 int kv_nq = 0) {
  const int64_t nm = (int64_t)a->batch * a->n_q_heads * nsp;
  MergeParams mp;
  mp.H = a->n_q_heads; mp.nsp = nsp; mp.hd = a->head_dim;
  mp.kv_nq = kv_nq;
  mp.ws_m = ws; mp.ws_l = ws + nm; mp.ws_acc = ws + 2 * nm; mp.out = a->out;
  launch_partial_merge(mp, a->batch, s);
  SHARD_LAUNCH_CHECK("shard_decode_attn merge");
  return SHARD_OK;
}

// Token-tiled split kernel + merge for one decode call (arguments checked by the caller).
int decode_attn_tok(const shard_decode_args* a, float* ws, hipStream_t s) {
  const TokPlan pl = tok_plan(a);
  const int nq = tok_nq(a);
  const int64_t nm = (int64_t)a->batch * a->n_q_heads * pl.ns;
  const bool hp = head_pairs(a);
  TokParams tp;
  tp.B = a->batch; tp.H = a->n_q_heads; tp.G = tok_g(a); tp.n_comp = a->n_comp;
  tp.QG = a->n_q_heads / tp.G / nq;
  tp.cstart = a->compress_start;
  tp.n_ct = pl.n_ct; tp.n_xt = pl.n_xt; tp.n_splits = pl.ns; tp.per_u = pl.per_u;
  tp.xs.sink_k = a->sink_k; tp.xs.sink_v = a->sink_v;
  tp.xs.win_k = a->win_k; tp.xs.win_v = a->win_v;
  tp.xs.dec_k = a->dec_k; tp.xs.dec_v = a->dec_v;
  tp.xs.s_k = a->s_k; tp.xs.s_v = a->s_v;
  tp.xs.n_sink = a->n_sink; tp.xs.n_win = a->n_win; tp.xs.n_dec = a->n_dec;
  tp.xs.dec_stride = a->dec_stride; tp.xs.n_stream = a->n_stream;
  tp.xs.n_x = (int32_t)n_extra(a);
  tp.xs.n_stream_dev = a->n_stream_dev;
  tp.q = a->q; tp.inv_freq = a->inv_freq; tp.coef = a->k_coeffs;
  tp.op = (const uint4*)a->prep;
  tp.rope = (const float2*)((const char*)a->prep + (size_t)tp.G * 4 * (a->rank / 16 + 1) * 64 * sizeof(uint4));
  tp.vidx = a->v_idx; tp.vcb = a->v_codebook; tp.vch = a->v_ch;
  tp.mask = a->mask; tp.mask_stride = a->mask_stride; tp.n_sink = a->n_sink;
  tp.ws_m = ws; tp.ws_l = ws + nm; tp.ws_acc = ws + 2 * nm;
  const dim3 grid((unsigned)((int64_t)pl.ns * tp.G * tp.QG * a->batch));
  switch (a->rank / 16) {
    case 2: launch_tok<2>(tp, nq, hp, grid, s); break;
    case 4: launch_tok<4>(tp, nq, hp, grid, s); break;
    case 6: launch_tok<6>(tp, nq, hp, grid, s); break;
    case 8: launch_tok<8>(tp, nq, hp, grid, s); break;
    case 10: launch_tok<10>(tp, nq, hp, grid, s); break;
    case 12: launch_tok<12>(tp, nq, hp, grid, s); break;
    case 14: launch_tok<14>(tp, nq, hp, grid, s); break;
    case 16: launch_tok<16>(tp, nq, hp, grid, s); break;
    default: return SHARD_ERR_SHAPE;
  }
  SHARD_LAUNCH_CHECK("shard_decode_attn token-tiled kernel");
  return launch_merge(a, ws, pl.ns, s);
}

}  // namespace shard

using namespace shard;

static size_t shard_decode_prepare_op_bytes(int32_t G, int32_t rank) {
  return (size_t)G * 4 * (rank / 16 + 1) * 64 * sizeof(uint4);
}

extern "C" {

size_t shard_decode_prepare_bytes(int32_t n_kv_heads, int32_t rank) {
  if (n_kv_heads <= 0 || rank <= 0 || rank % 32 != 0) return 0;
  return shard_decode_prepare_op_bytes(n_kv_heads, rank) + kRopeEntries * sizeof(float2);
}

int shard_decode_prepare(const uint16_t* k_basis, const uint16_t* k_coeff_scale,
                         const uint16_t* k_mean, const float* inv_freq, int32_t n_kv_heads,
                         int32_t head_dim, int32_t rank, void* out, size_t out_bytes,
                         void* stream) {
  if (!k_basis || !k_coeff_scale || !k_mean || !inv_freq || !out || n_kv_heads <= 0)
    return SHARD_ERR_ARG;
  if ((head_dim != kHD && head_dim != 64) || rank <= 0 || rank % 32 != 0 || rank > kTokMaxRank)
    return SHARD_ERR_SHAPE;
  const int hp = head_dim == 64;  // head pairs: one operand image per two kv heads
  if (hp && (n_kv_heads & 1)) return SHARD_ERR_SHAPE;
  const int G = hp ? n_kv_heads / 2 : n_kv_heads;
  if (out_bytes < shard_decode_prepare_bytes(G, rank)) return SHARD_ERR_WORKSPACE;
  hipStream_t s = (hipStream_t)stream;
  uint4* op = (uint4*)out;
  float2* rope = (float2*)((char*)out + shard_decode_prepare_op_bytes(G, rank));
  const int64_t total = (int64_t)G * 4 * (rank / 16 + 1) * 64 + kRopeEntries;
  hipLaunchKernelGGL(k_decode_prepare, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                     k_basis, k_coeff_scale, k_mean, inv_freq, G, rank, hp, op, rope);
  SHARD_LAUNCH_CHECK("shard_decode_prepare");
  return SHARD_OK;
}

int shard_decode_supported(const shard_decode_args* a) {
  return a && tok_supported(a) ? 1 : 0;
}

size_t shard_decode_attn_workspace(const shard_decode_args* a) {
  if (!a || a->batch <= 0 || a->n_q_heads <= 0 || a->n_comp <= 0 || !tok_supported(a)) return 0;
  if (use_tok(a)) {
    const TokPlan pl = tok_plan(a);
    return (size_t)a->batch * a->n_q_heads * pl.ns * (kHD + 2) * sizeof(float);
  }
  const int nsp = split_count(a) + (n_extra(a) > 0 ? 1 : 0);
  return (size_t)a->batch * a->n_q_heads * nsp * (kHD + 2) * sizeof(float);
}

}  // extern "C"

static int decode_attn_check(const shard_decode_args* a) {
  if (!a || !a->q || !a->inv_freq || !a->k_coeffs || !a->prep || !a->v_idx || !a->v_codebook ||
      !a->v_ch || !a->out)
    return SHARD_ERR_ARG;
  if (a->batch <= 0 || a->n_comp <= 0) return SHARD_ERR_ARG;
  if (a->n_sink < 0 || a->n_win < 0 || a->n_dec < 0 || a->n_stream < 0) return SHARD_ERR_ARG;
  if (a->kernel < 0 || a->kernel > 2) return SHARD_ERR_ARG;
  // a device stream count bounds the stream by n_stream; the mask row would
  // have to follow the count, so the two do not go together
  if (a->n_stream_dev && (a->mask || !a->n_stream)) return SHARD_ERR_ARG;
  if ((a->n_sink && (!a->sink_k || !a->sink_v)) || (a->n_win && (!a->win_k || !a->win_v)) ||
      (a->n_dec && (!a->dec_k || !a->dec_v || a->dec_stride < a->n_dec)) ||
      (a->n_stream && (!a->s_k || !a->s_v)))
    return SHARD_ERR_ARG;
  if (!tok_supported(a) || n_extra(a) > (int64_t)INT32_MAX / 4) return SHARD_ERR_SHAPE;
  if (((uintptr_t)a->q & 15) || ((uintptr_t)a->out & 3)) return SHARD_ERR_ARG;  // vector accesses
  return SHARD_OK;
}

// One decode call on a checked `a` with a workspace of shard_decode_attn_workspace(a) bytes.
static int decode_attn_run(const shard_decode_args* a, void* workspace, hipStream_t s) {
  if (use_tok(a)) return decode_attn_tok(a, (float*)workspace, s);

  const int n_x = (int)n_extra(a);
  const int ns = split_count(a);
  const int nsp = ns + (n_x > 0 ? 1 : 0);
  float* ws = (float*)workspace;
  const int64_t nm = (int64_t)a->batch * a->n_q_heads * nsp;
  SplitParams sp;
  sp.B = a->batch; sp.H = a->n_q_heads; sp.G = a->n_kv_heads; sp.rank = a->rank;
  sp.n_comp = a->n_comp; sp.cstart = a->compress_start; sp.pos_q = a->pos_q;
  sp.pos_q_dev = a->pos_q_dev;
  sp.n_splits = ns;
  // Compressed tiles per split, in whole 32-token tiles.  The last split of
  // each head also runs the extra tokens (an extra token costs about half a
  // compressed one), so the tiles are spread over the splits as if there were
  // n_x / 64 more of them and the last split takes what remains.
  const int n_tiles = (a->n_comp + kTile - 1) / kTile;
  const int x_cost = (n_x + 63) / 64;
  const int cap = n_tiles + x_cost;
  const int chunk_tiles = (cap + ns - 1) / ns;
  sp.chunk = ((chunk_tiles + kTG - 1) / kTG) * kTG * kTile;
  sp.chunk2 = sp.chunk;
  sp.n_first = ns;
  sp.two_class = 0;
  const int half = ns / 2;
  // the class split and both block orders assume 256 CUs (two classes of 256 workgroups)
  if (kTG == 1 && kSplitBias && device_cus() == 256 && (int64_t)ns * a->n_kv_heads * a->batch == 512 &&
      ns % 2 == 0 && 32 % a->n_kv_heads == 0 && n_tiles >= 2 * ns) {
    // first class: ta tiles per split, second class: tb (the last split also
    // runs the extra tokens, counted as x_cost tiles)
    const int ta = (97 * half + 64 * cap) / (100 * half);  // round(0.47 + 0.64 cap / half)
    const int tb = (cap - half * ta + half - 1) / half;
    if (ta >= 1 && tb >= 1) {
      sp.chunk = ta * kTile;
      sp.chunk2 = tb * kTile;
      sp.n_first = half;
      sp.two_class = 1;
    }
  }
  sp.nsp = nsp;
  sp.xs.sink_k = a->sink_k; sp.xs.sink_v = a->sink_v;
  sp.xs.win_k = a->win_k; sp.xs.win_v = a->win_v;
  sp.xs.dec_k = a->dec_k; sp.xs.dec_v = a->dec_v;
  sp.xs.s_k = a->s_k; sp.xs.s_v = a->s_v;
  sp.xs.n_sink = a->n_sink; sp.xs.n_win = a->n_win; sp.xs.n_dec = a->n_dec;
  sp.xs.dec_stride = a->dec_stride; sp.xs.n_stream = a->n_stream; sp.xs.n_x = n_x;
  sp.xs.n_stream_dev = a->n_stream_dev;
  sp.q = a->q; sp.inv_freq = a->inv_freq; sp.coef = a->k_coeffs;
  sp.op = (const uint4*)a->prep;
  sp.rope = (const float2*)((const char*)a->prep + shard_decode_prepare_op_bytes(a->n_kv_heads, a->rank));
  sp.vidx = a->v_idx; sp.vcb = a->v_codebook; sp.vch = a->v_ch;
  sp.mask = a->mask; sp.mask_stride = a->mask_stride; sp.n_sink = a->n_sink;
  sp.ws_m = ws; sp.ws_l = ws + nm; sp.ws_acc = ws + 2 * nm;
  sp.kv_xcd = SHARD_KV_XCD && sp.two_class && (a->batch * a->n_kv_heads) % 8 == 0;

  dim3 grid((unsigned)(ns * a->n_kv_heads), (unsigned)a->batch);
  switch (a->rank / 16) {
    case 2: hipLaunchKernelGGL((k_decode_split<2, kTG>), grid, dim3(256 * kTG), 0, s, sp); break;
    case 4: hipLaunchKernelGGL((k_decode_split<4, kTG>), grid, dim3(256 * kTG), 0, s, sp); break;
    case 6: hipLaunchKernelGGL((k_decode_split<6, kTG>), grid, dim3(256 * kTG), 0, s, sp); break;
    case 8: hipLaunchKernelGGL((k_decode_split<8, kTG>), grid, dim3(256 * kTG), 0, s, sp); break;
    case 10: hipLaunchKernelGGL((k_decode_split<10, kTG>), grid, dim3(256 * kTG), 0, s, sp); break;
    case 12: hipLaunchKernelGGL((k_decode_split<12, kTG>), grid, dim3(256 * kTG), 0, s, sp); break;
    default: return SHARD_ERR_SHAPE;
  }
  SHARD_LAUNCH_CHECK("shard_decode_attn row-split kernel");
  return launch_merge(a, ws, nsp, s, sp.kv_xcd ? kGQA : 0);
}

// ---- scratch of shard_decode_attn_noalloc: the partial rows (m, l, acc) of
// every (batch row, query head, split), in one device array per GPU that is
// never freed.  Host code uses the per-device address that
// hipGetSymbolAddress returns, never the array's own name (on the host that
// name is a stand-in, not a device address).
static __device__ __align__(256) unsigned char scratch[SHARD_DECODE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch_dev[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of `scratch` on the current device, looked up on the first
// call there.
static int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_last_error("shard_decode_attn_noalloc hipGetDevice", e);
    return SHARD_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_last_text("shard_decode_attn_noalloc: device index beyond 63");
    return SHARD_ERR_ARG;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_last_error("shard_decode_attn_noalloc hipGetSymbolAddress", e);
      return SHARD_ERR_HIP;
    }
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return SHARD_OK;
}

extern "C" {

int shard_decode_attn(const shard_decode_args* a, void* workspace, size_t workspace_bytes,
                      void* stream) {
  const int st = decode_attn_check(a);
  if (st != SHARD_OK) return st;
  const size_t need = shard_decode_attn_workspace(a);
  if (!workspace || workspace_bytes < need) {
    char msg[128];
    snprintf(msg, sizeof(msg), "shard_decode_attn: workspace of %zu bytes, the call needs %zu",
             workspace ? workspace_bytes : (size_t)0, need);
    set_last_text(msg);
    return SHARD_ERR_WORKSPACE;
  }
  return decode_attn_run(a, workspace, (hipStream_t)stream);
}

int shard_decode_attn_noalloc(const shard_decode_args* a, void* stream) {
  const int st = decode_attn_check(a);
  if (st != SHARD_OK) return st;
  const size_t need = shard_decode_attn_workspace(a);
  if (need > SHARD_DECODE_NOALLOC_SCRATCH_BYTES) {
    char msg[160];
    snprintf(msg, sizeof(msg),
             "shard_decode_attn_noalloc: the call needs %zu workspace bytes, more than the %zu of "
             "its scratch (fewer splits or a smaller batch fit)",
             need, (size_t)SHARD_DECODE_NOALLOC_SCRATCH_BYTES);
    set_last_text(msg);
    return SHARD_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  const int sa = scratch_address(&ws);
  if (sa != SHARD_OK) return sa;
  return decode_attn_run(a, ws, (hipStream_t)stream);
}

}  // extern "C"
