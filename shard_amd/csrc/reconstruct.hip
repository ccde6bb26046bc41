// Full fp16 reconstruction of the compressed cache for unfused consumers
// (_ensure_dequant, cache.py:87-124) and the stream dequantizer
// (_dequant_stream, cache.py:243-279).  Off the decode hot path: used on the
// first decode step (compression happens inside it), for q_len > 1 extends and
// for callers that read layer.keys / layer.values.
#include "common.h"

namespace shard {

constexpr int kRcTok = 32;   // tokens per block

// K: block = (b, 32-token tile, kv head g); 256 threads = 32 tokens x 8 lanes,
// each lane owns HD / 16 RoPE pairs of its token.  The head's basis rows and
// the tile's coefficients are staged in LDS.
template <int HD>
__global__ __launch_bounds__(256)
void k_reconstruct_k(const uint8_t* __restrict__ coef, const uint16_t* __restrict__ cs,
                     const uint16_t* __restrict__ basis, const uint16_t* __restrict__ mean,
                     const float* __restrict__ inv_freq, int B, int G, int rank, int n_comp,
                     int cstart, uint16_t* __restrict__ k_out) {
  constexpr int kRcHD = HD;
  extern __shared__ __align__(16) unsigned char smem[];
  uint16_t* cf = (uint16_t*)smem;                  // [kRcTok][rank] fp16(nib*cs)
  uint16_t* bb = cf + kRcTok * rank;               // [HD][rank] basis rows of head g
  const int tid = threadIdx.x;
  const int g = blockIdx.y, b = blockIdx.z;
  const int t0 = blockIdx.x * kRcTok;
  const int row_bytes = rank / 2;
  for (int i = tid; i < kRcTok * rank; i += 256) {
    const int tt = i / rank, r = i - tt * rank;
    const int t = t0 + tt;
    uint16_t v = 0;
    if (t < n_comp) {
      const uint8_t byte = coef[((int64_t)b * n_comp + t) * row_bytes + (r >> 1)];
      const int nib = (r & 1) ? (byte >> 4) : (byte & 15);
      // fp16(nib - 8) * fp16(cs) rounded to fp16, as the reference's fp16 multiply
      v = f2h((float)(nib - 8) * h2f(cs[r]));
    }
    cf[i] = v;
  }
  for (int i = tid; i < kRcHD * rank; i += 256)
    bb[i] = basis[(int64_t)g * kRcHD * rank + i];
  __syncthreads();
  const int tt = tid >> 3, part = tid & 7;
  const int t = t0 + tt;
  if (t >= n_comp) return;
  const uint16_t* cr = cf + tt * rank;
  const int pos = cstart + t;
  constexpr int PL = HD / 16;  // pairs per lane
#pragma unroll 1
  for (int u = 0; u < PL; ++u) {
    const int i = part * PL + u;  // pair index 0 .. HD/2 - 1
    float c = 0.f, d = 0.f;
    const uint16_t* b0 = bb + i * rank;
    const uint16_t* b1 = bb + (i + HD / 2) * rank;
    for (int r = 0; r < rank; ++r) {
      const float cv = h2f(cr[r]);
      c += cv * h2f(b0[r]);
      d += cv * h2f(b1[r]);
    }
    // recon = fp16(coeffs @ basis^T) + mean, both fp16
    const float cm = h2f(f2h(h2f(f2h(c)) + h2f(mean[g * kRcHD + i])));
    const float dm = h2f(f2h(h2f(f2h(d)) + h2f(mean[g * kRcHD + i + HD / 2])));
    // reapply_rope: k*cos + rotate_half(k)*sin with fp32 phase fl(pos*theta)
    float sn, csn;
    sincosf(__fmul_rn((float)pos, inv_freq[i]), &sn, &csn);
    uint16_t* o = k_out + (((int64_t)b * G + g) * n_comp + t) * kRcHD;
    o[i] = f2h(__fsub_rn(__fmul_rn(cm, csn), __fmul_rn(dm, sn)));
    o[i + HD / 2] = f2h(__fadd_rn(__fmul_rn(dm, csn), __fmul_rn(cm, sn)));
  }
}

// V: one wave per (b, g, t): fp16(hadamard(cb[idx] * ch)), fp32 math;
// subvectors of gs = 2^lg values (D / gs indices per token), a codebook of
// cbn rows (an index past it reads its last row), head dim D = 64 E
// (element i = lane + 64 k).
template <int E>
__global__ void k_reconstruct_v(const uint8_t* __restrict__ vidx, const uint16_t* __restrict__ vcb,
                                const uint16_t* __restrict__ vch, int64_t rows, int G, int n_comp,
                                int lg, int cbn, uint16_t* __restrict__ v_out) {
  constexpr int D = 64 * E;
  const int l = (int)lane_id();
  const int gs = 1 << lg;
  int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t r = wave; r < rows; r += nw) {  // r = (b*G + g)*n_comp + t
    const int64_t bg = r / n_comp;
    const uint8_t* ix = vidx + r * (D >> lg);
    const uint16_t* ch = vch + bg * D;
    float x[E];
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const int d = l + 64 * k;
      const int e = min((int)ix[d >> lg], cbn - 1);
      x[k] = __fmul_rn(h2f(vcb[gs * e + (d & (gs - 1))]), h2f(ch[d]));
    }
    wave_fwht<E>(x, D);
#pragma unroll
    for (int k = 0; k < E; ++k) v_out[r * D + l + 64 * k] = f2h_opaque(x[k]);
  }
}

// Stream rows: fp16(fp16(hadamard(cb[idx] (+ QJL term)) * signs) * norm), one
// wave per row of D = 64 E elements (element i = lane + 64 k).
template <int E>
__global__ void k_stream_dequant(const uint8_t* __restrict__ idx, const uint16_t* __restrict__ norm,
                                 const uint8_t* __restrict__ qsign,
                                 const uint16_t* __restrict__ qscale, int64_t rows,
                                 const float* __restrict__ signs, const float* __restrict__ cb,
                                 uint16_t* __restrict__ y) {
  constexpr int D = 64 * E;
  const int l = (int)lane_id();
  int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
  int64_t nw = ((int64_t)gridDim.x * blockDim.x) >> 6;
  for (int64_t r = wave; r < rows; r += nw) {
    float x[E];
#pragma unroll
    for (int k = 0; k < E; ++k) x[k] = cb[idx[r * D + l + 64 * k]];
    if (qsign) {  // QJL: cb[idx] + (2 s - 1) * scale (streaming.py:76-77)
      const float sc = h2f(qscale[r]);
#pragma unroll
      for (int k = 0; k < E; ++k) x[k] = __fadd_rn(x[k], qsign[r * D + l + 64 * k] ? sc : -sc);
    }
    wave_fwht<E>(x, D);
    const float n = h2f(norm[r]);
    // fp16(fp16(x * sign) * norm): the sign flip is exact, the product of two
    // fp16 values is exact in fp32, so each line rounds exactly twice like torch
#pragma unroll
    for (int k = 0; k < E; ++k)
      y[r * D + l + 64 * k] = f2h_opaque(h2f(f2h(mul_sign(x[k], signs[l + 64 * k]))) * n);
  }
}

}  // namespace shard

using namespace shard;

extern "C" {

int shard_kv_reconstruct(const shard_decode_args* a, uint16_t* k_out, uint16_t* v_out,
                         void* stream) {
  if (!a || !a->k_coeffs || !a->k_coeff_scale || !a->k_basis || !a->k_mean || !a->v_idx ||
      !a->v_codebook || !a->v_ch || !a->inv_freq || !k_out || !v_out)
    return SHARD_ERR_ARG;
  if (a->batch <= 0 || a->n_comp <= 0 || a->n_kv_heads <= 0) return SHARD_ERR_ARG;
  const int hd = a->head_dim;
  // the tile's fp16 coefficients and the head's basis rows in LDS: up to
  // 160 KB (rank 512 at head_dim 128, 284 at 256)
  const size_t lds = (size_t)(kRcTok + hd) * (a->rank > 0 ? a->rank : 0) * sizeof(uint16_t);
  if ((hd != 64 && hd != 128 && hd != 256) || a->rank <= 0 || (a->rank & 1) || lds > 160 * 1024)
    return SHARD_ERR_SHAPE;
  const int gs = a->v_group ? a->v_group : 4, cbn = a->v_codebook_n ? a->v_codebook_n : 256;
  const int lg = gs == 1 ? 0 : gs == 2 ? 1 : gs == 4 ? 2 : gs == 8 ? 3 : -1;
  if (lg < 0 || cbn < 1 || cbn > 256) return SHARD_ERR_SHAPE;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)((a->n_comp + kRcTok - 1) / kRcTok), (unsigned)a->n_kv_heads,
            (unsigned)a->batch);
  auto launch_k = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, a->k_coeffs, a->k_coeff_scale, a->k_basis,
                       a->k_mean, a->inv_freq, a->batch, a->n_kv_heads, a->rank, a->n_comp,
                       a->compress_start, k_out);
  };
  const int64_t rows = (int64_t)a->batch * a->n_kv_heads * a->n_comp;
  const dim3 vgrid(grid_cap((rows + 3) / 4, 16384));
  auto launch_v = [&](auto kern) {
    hipLaunchKernelGGL(kern, vgrid, dim3(256), 0, s, a->v_idx, a->v_codebook, a->v_ch, rows,
                       a->n_kv_heads, a->n_comp, lg, cbn, v_out);
  };
  if (lds > 64 * 1024) {  // LDS beyond the default dynamic limit (160 KB per CU on gfx950)
    const void* kern = hd == 64 ? reinterpret_cast<const void*>(&k_reconstruct_k<64>)
                     : hd == 128 ? reinterpret_cast<const void*>(&k_reconstruct_k<128>)
                                 : reinterpret_cast<const void*>(&k_reconstruct_k<256>);
    const hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      set_last_error("shard_kv_reconstruct LDS attribute", e);
      return SHARD_ERR_HIP;
    }
  }
  if (hd == 64) {
    launch_k(k_reconstruct_k<64>);
    launch_v(k_reconstruct_v<1>);
  } else if (hd == 128) {
    launch_k(k_reconstruct_k<128>);
    launch_v(k_reconstruct_v<2>);
  } else {
    launch_k(k_reconstruct_k<256>);
    launch_v(k_reconstruct_v<4>);
  }
  SHARD_LAUNCH_CHECK("shard_kv_reconstruct");
  return SHARD_OK;
}

int shard_stream_dequant_qjl(const uint8_t* idx, const uint16_t* norm, const uint8_t* qsign,
                             const uint16_t* qscale, int64_t rows, int32_t hd, const float* signs,
                             const float* codebook, uint16_t* y, void* stream) {
  if (!idx || !norm || !signs || !codebook || !y || rows <= 0) return SHARD_ERR_ARG;
  if ((qsign == nullptr) != (qscale == nullptr)) return SHARD_ERR_ARG;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(grid_cap((rows + 3) / 4, 16384)), block(256);
  switch (hd) {
    case 64: hipLaunchKernelGGL(k_stream_dequant<1>, grid, block, 0, s, idx, norm, qsign, qscale, rows, signs, codebook, y); break;
    case 128: hipLaunchKernelGGL(k_stream_dequant<2>, grid, block, 0, s, idx, norm, qsign, qscale, rows, signs, codebook, y); break;
    case 256: hipLaunchKernelGGL(k_stream_dequant<4>, grid, block, 0, s, idx, norm, qsign, qscale, rows, signs, codebook, y); break;
    default: return SHARD_ERR_SHAPE;
  }
  SHARD_LAUNCH_CHECK("shard_stream_dequant");
  return SHARD_OK;
}

int shard_stream_dequant(const uint8_t* idx, const uint16_t* norm, int64_t rows, int32_t hd,
                         const float* signs, const float* codebook, uint16_t* y, void* stream) {
  return shard_stream_dequant_qjl(idx, norm, nullptr, nullptr, rows, hd, signs, codebook, y, stream);
}

}  // extern "C"
