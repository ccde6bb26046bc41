/*
 * shard_hip.h — C ABI of libshard_hip.so, the MI355X (gfx950) kernels of the
 * compressed-KV attention path.
 *
 * Conventions (every entry point):
 *   - plain device pointers (HBM), element counts and strides; no torch types;
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream); all work
 *     is enqueued on it, nothing synchronizes the host;
 *   - fp16 tensors are passed as uint16_t* (IEEE binary16 bit patterns);
 *   - return 0 on success, a negative SHARD_ERR_* code otherwise; nothing is
 *     allocated inside: scratch memory comes in through `workspace`, sized by
 *     the matching *_workspace() query (shard_decode_attn_noalloc alone uses
 *     a static device array of the library instead, see its declaration);
 *   - entry points are stateless and re-entrant (no mutable globals; calls of
 *     shard_decode_attn_noalloc share its array and must not overlap).
 *
 * Each declaration names the reference code (bhengubv/shard, src/shard/...)
 * whose role it takes over.
 */
#ifndef SHARD_HIP_H
#define SHARD_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SHARD_OK 0
#define SHARD_ERR_ARG (-1)       /* null pointer, negative or zero size */
#define SHARD_ERR_SHAPE (-2)     /* shape the kernels do not support */
#define SHARD_ERR_HIP (-3)       /* a HIP launch or runtime call failed */
#define SHARD_ERR_WORKSPACE (-4) /* workspace missing or too small */

/* Library version string, e.g. "shard_hip 0.1.0 gfx950". */
const char* shard_version(void);

/* Human-readable text of the last HIP error seen on this thread ("" if none). */
const char* shard_last_error(void);

/* sizeof(shard_decode_args) as compiled into the library (ABI check for bindings). */
size_t shard_decode_args_size(void);

/* ------------------------------------------------------------------------
 * Prefill compression: keys
 * ------------------------------------------------------------------------ */

/* PCA projection GEMM on MFMA: C[m, n] (fp32) = A[m, k] (fp16) . Bt[n, k]^T (fp16).
 * A row-major with row stride lda (elements), Bt row-major (n rows of k),
 * C row-major with row stride ldc.  k % 16 == 0, n % 32 == 0 (one launch per
 * 256 columns: ranks above 256 take several).
 * Replaces the projection GEMM of _compress_k, cache.py:392
 * ((flat - mean) @ (basis_q * scale)). */
int shard_pca_project(const uint16_t* a, int64_t m, int32_t k, int64_t lda,
                      const uint16_t* bt, int32_t n, float* c, int64_t ldc,
                      void* stream);

/* The same projection with fp32 operands, as the reference computes it
 * (cache.py:389-392: (flat - mean) @ (basis_q.float() * scale.float()), fp32):
 * C[m, n] = A[m, k] (fp32) . Bt[n, k]^T (fp32) on v_mfma_f32_32x32x2_f32,
 * fp32 sums.  k % 8 == 0, n % 32 == 0 (one launch per 256 columns),
 * lda % 4 == 0, a and bt 16-byte aligned.  The path Cache.compress takes. */
int shard_pca_project_f32(const float* a, int64_t m, int32_t k, int64_t lda,
                          const float* bt, int32_t n, float* c, int64_t ldc,
                          void* stream);

/* The fp16 projection with its front end fused (the fp16 operand of
 * shard_k_prepare is never written): C[b * n_comp + t, j] =
 *   sum_k fp16(undo_rope(k)[.., col(k)]) * btp[j, k] - bias[j]
 * for the post-RoPE keys k (B, n_kv, seq, 128) fp16 at positions start + t,
 * undone with phases[(t, i)] = (cos, sin) of shard_rope_phases (the arithmetic
 * of shard_k_prepare), in the permuted k order of the header of csrc/pca.hip
 * (btp = the basis columns in that order, n rows of n_kv * 128; the host
 * permutes them once); bias (n, nullable) = mean . basis stands for the
 * centring.  hd == 128, n % 32 == 0, n <= 256; k, phases, btp 16-byte aligned.
 * Replaces undo_rope + (flat - mean) @ basis of cache.py:370-392 on the fp16
 * path. */
int shard_pca_project_rope(const uint16_t* k, int32_t batch, int32_t n_kv, int32_t seq,
                           int32_t hd, int32_t start, int32_t n_comp,
                           const float* phases, const uint16_t* btp, int32_t n,
                           const float* bias, float* c, int64_t ldc, void* stream);

/* (cos, sin)(fl((start + t) * inv_freq[i])) as float pairs, out (n, hd2, 2):
 * the phases of rope_cos_sin (rope.py:13-18) that undo_rope uses. */
int shard_rope_phases(int32_t start, int32_t n, int32_t hd2, const float* inv_freq,
                      float* out, void* stream);

/* Prefill K preparation fused with the projection input: reads post-RoPE keys
 * k (B, n_kv, T, hd) fp16, undoes RoPE at positions start+t with fp32 phases
 * fl(pos * inv_freq[i]) (rope.py:13-24), subtracts mean[n_kv*hd] (fp32) and
 * writes the fp16 row-major matrix out[(b*n_comp + t), n_kv*hd] for tokens
 * t in [0, n_comp).  Replaces undo_rope + permute/reshape + (flat - mean) of
 * cache.py:370-376 (as the fp16 GEMM operand).  hd is a multiple of 8 and at
 * most 512; k and out are 8-byte aligned (rows move as 4-half vectors). */
int shard_k_prepare(const uint16_t* k, int32_t batch, int32_t n_kv, int32_t seq,
                    int32_t hd, int32_t start, int32_t n_comp,
                    const float* inv_freq, const float* mean, uint16_t* out,
                    void* stream);

/* shard_k_prepare writing the centred rows in fp32 (no fp16 rounding): the
 * (flat - mean) operand of cache.py:392 as the reference holds it.  out is
 * 16-byte aligned. */
int shard_k_prepare_f32(const uint16_t* k, int32_t batch, int32_t n_kv, int32_t seq,
                        int32_t hd, int32_t start, int32_t n_comp,
                        const float* inv_freq, const float* mean, float* out,
                        void* stream);

/* Integer chain of the key coefficients, bit-exact with the reference:
 *   per column c with bits[c] > 0: lo = min, rng = max(max - lo, 1e-6),
 *     code = clamp(rint(clamp((x - lo) / rng, 0, 1) * L), 0, L), L = 2^bits - 1,
 *     y = code / L * rng + lo;  columns with bits[c] == 0 give y = 0
 *     (quantize_group / dequantize_group values, rope.py:95-161);
 *   cs = max(max |y|, 1e-6) / 7;  q = clamp(rint(y / cs), -7, 7)
 *     (cache.py:416-419);
 *   packed[i] = ((q[2i] + 8) & 15) | ((q[2i+1] + 8) & 15) << 4 over the
 *     row-major (n_rows, keep) matrix; an odd count is padded with a zero
 *     value (high nibble 8)
 *     (int4_pack, triton_kernels.py:648-682).
 * proj: (n_rows, keep) fp32 row-major.  Outputs: packed ((n_rows*keep+1)/2),
 * coeff_scale (keep, fp32), lo/rng (keep, fp32, nullable), codes
 * ((n_rows, keep) uint8 group codes, nullable). */
size_t shard_int4_quant_pack_workspace(int64_t n_rows, int32_t keep);
int shard_int4_quant_pack(const float* proj, int64_t n_rows, int32_t keep,
                          const int32_t* bits, uint8_t* packed, float* coeff_scale,
                          float* lo, float* rng, uint8_t* codes,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Prefill compression: values
 * ------------------------------------------------------------------------ */

/* Normalized fast Walsh-Hadamard transform over the last dim d (power of two,
 * 2..1024) of `rows` fp32 rows; bit-exact with hadamard(), cache.py:10-19
 * (butterflies h = 1, 2, 4, ... then one IEEE division by fp32(sqrt(d))).
 * y may alias x. */
int shard_fwht(const float* x, float* y, int64_t rows, int32_t d, void* stream);

/* V encoder front half (vq_encode, cache.py:41-46 after hadamard, cache.py:402):
 * v fp16 (bh, seq, hd) -> v_rot = hadamard(fp32(v)); ch = max(max_t |v_rot|, 1e-8)
 * per (bh, channel); x = v_rot / ch written as fp32 (bh*seq*hd/g, g) subvectors;
 * ch also written as fp16 (bh, hd).  Uses workspace for the fp32 channel max.
 * v must be aligned to hd/32 bytes with v_bh_stride a multiple of hd/64, and
 * x_out to hd/16 bytes (rows move as hd/64-element vectors). */
size_t shard_vq_prepare_workspace(int64_t bh, int32_t hd);
int shard_vq_prepare(const uint16_t* v, int64_t bh, int64_t seq, int32_t hd,
                     int64_t v_bh_stride, float* x_out, float* ch_f32,
                     uint16_t* ch_f16, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Nearest-centroid assignment: idx[i] = argmin_k sum_j (x[i,j] - c[k,j])^2 with
 * the squared differences summed in fp32 in j order without FMA, first index
 * on ties.  d <= 8, k <= 1024.  Replaces vq_assign, triton_kernels.py:689-746
 * (whose CPU fallback is cdist(...).argmin, triton_kernels.py:733-734).  The
 * unfused sum is this library's reading of the kernel's `dist += diff * diff`,
 * which Triton's default fp fusion may contract into an FMA. */
int shard_vq_assign(const float* x, int64_t n, int32_t d, const float* centroids,
                    int32_t k, int32_t* idx, void* stream);

/* The same assignment for 4-dim rows and k = 32, 64, ..., 256 centroids
 * through a candidate table built once per codebook (the same replacement of
 * triton_kernels.py:689-746; the reference's k-means calls it every
 * iteration, cache.py:26-27).  The table cuts the box [lo, hi]^4 into
 * nbins^4 cells (nbins <= 32) and lists for each cell, in index order, the
 * centroids that can be the answer for some row in it (a rigorous bound on
 * the fp32 distance drops the others); a row in the box is decided by the
 * direct distances to its cell's list.  Rows outside the box, non-finite rows
 * and rows of cells with more than 32 candidates are finished by a direct
 * scan of every centroid, so every result equals shard_vq_assign's (the scan
 * suits the few rows normalized data leaves to it; rows not normalized to
 * the box belong with shard_vq_assign).  The box must satisfy hi > lo and
 * max(|lo|, |hi|) <= 64 (hi - lo); normalized subvectors (shard_vq_prepare's
 * x, in [-1, 1]) take lo = -1, hi = 1.
 * table: shard_vq_table_bytes(k, nbins) bytes, 16-byte aligned.
 * shard_vq_assign_table takes the build's k, nbins, lo and hi (a table built
 * with other values decides nothing: every row takes the direct scan) and a
 * 16-byte aligned workspace of shard_vq_assign_table_workspace(n) bytes (per
 * wave of the launch, a count and a region of the rows it left undecided);
 * n < 2^31. */
size_t shard_vq_table_bytes(int32_t k, int32_t nbins);
/* shard_vq_prepare's first half (cache.py:43-44: the FWHT's per-(bh,
 * channel) max |.|, clamped): ch_f32 (bh, hd), optional ch_f16 and ch_rcp
 * (the scales' correctly rounded reciprocals, for shard_vq_encode_table);
 * the same workspace as shard_vq_prepare. */
int shard_vq_scales(const uint16_t* v, int64_t bh, int64_t seq, int32_t hd,
                    int64_t v_bh_stride, float* ch_f32, uint16_t* ch_f16, float* ch_rcp,
                    void* workspace, size_t workspace_bytes, void* stream);
/* vq_encode against a given codebook (cache.py:41-52 with the k-means step
 * replaced by one assignment, triton_kernels.py:689-746): the normalized
 * subvectors of shard_vq_prepare are formed in registers from V (hd = 128,
 * 8-byte aligned rows, v_bh_stride % 4 == 0) and assigned through a table
 * of those centroids (built for the box [lo, hi]^4; lo = -1, hi = 1 holds
 * every normalized row), without writing them out: idx (bh * seq * 32)
 * equals shard_vq_assign_table(shard_vq_prepare(v).x).  ch_f32 / ch_rcp from
 * shard_vq_scales; workspace shard_vq_encode_table_workspace(bh * seq * 32)
 * bytes, 16-byte aligned (the undecided rows and their values). */
size_t shard_vq_encode_table_workspace(int64_t n_rows);
int shard_vq_encode_table(const uint16_t* v, int64_t bh, int64_t seq, int32_t hd,
                          int64_t v_bh_stride, const float* ch_f32, const float* ch_rcp,
                          const float* centroids, int32_t k, const void* table,
                          size_t table_bytes, int32_t nbins, float lo, float hi, int32_t* idx,
                          void* workspace, size_t workspace_bytes, void* stream);
int shard_vq_table_build(const float* centroids, int32_t k, float lo, float hi,
                         int32_t nbins, void* table, size_t table_bytes, void* stream);
size_t shard_vq_assign_table_workspace(int64_t n);
int shard_vq_assign_table(const float* x, int64_t n, const float* centroids, int32_t k,
                          const void* table, size_t table_bytes, int32_t nbins, float lo,
                          float hi, int32_t* idx, void* workspace, size_t workspace_bytes,
                          void* stream);

/* One k-means update (cache.py:28-38) given assignments idx: new_c[k] = mean of
 * the rows assigned to k (empty clusters keep c[k]); also writes
 * max |new_c - c| to *max_delta (device fp32).  Sums are accumulated per
 * centroid in increasing row order, so the result is deterministic.
 * workspace: shard_kmeans_update_workspace_d(n, k, d) bytes (per-block
 * counts of the counting sort and the rows' sorted copy);
 * shard_kmeans_update_workspace(n, k) is the size for rows of up to 8 values. */
size_t shard_kmeans_update_workspace_d(int64_t n, int32_t k, int32_t d);
size_t shard_kmeans_update_workspace(int64_t n, int32_t k);
int shard_kmeans_update(const float* x, int64_t n, int32_t d, const int32_t* idx,
                        const float* centroids, int32_t k, float* new_centroids,
                        float* max_delta, void* workspace, size_t workspace_bytes,
                        void* stream);

/* ------------------------------------------------------------------------
 * Decode stream (8-bit Lloyd-Max, per token)
 * ------------------------------------------------------------------------ */

/* Per-token quantizer, bit-exact with _stream_append's _unit (cache.py:207-213)
 * + quantize_per_token (streaming.py:59-72, qjl off):
 *   t = fp32(x); n = max(||t||, 1e-8) with torch-CPU's 8-lane summation order;
 *   r = hadamard(t / n * signs); idx = bucketize(r, codebook) clamped, then the
 *   nearer of (idx-1, idx) by |cb - r| in fp32 (ties to idx); norm = fp16(n).
 * Optional `deq` (nullable, (rows, hd) fp16) receives the token as the
 * reference dequantizes it, fp16(fp16(hadamard(cb[idx]) * signs) * norm)
 * (cache.py:275-278, streaming.py:74-79), bit-exact.
 * x: (rows, hd) fp16 contiguous, hd in {64, 128, 256}; codebook sorted, n_codes <= 256. */
int shard_stream_quant(const uint16_t* x, int64_t rows, int32_t hd,
                       const float* signs, const float* codebook, int32_t n_codes,
                       uint8_t* idx, uint16_t* norm, uint16_t* deq, void* stream);

/* Stream dequantizer, bit-exact with _dequant_stream / dequantize_per_token
 * (cache.py:275-278, streaming.py:74-79, qjl off):
 *   y = fp16(fp16(hadamard(codebook[idx]) * signs) * norm)
 * idx (rows, hd) uint8, norm (rows) fp16 -> y (rows, hd) fp16; hd in {64, 128, 256}. */
int shard_stream_dequant(const uint8_t* idx, const uint16_t* norm, int64_t rows, int32_t hd,
                         const float* signs, const float* codebook, uint16_t* y,
                         void* stream);

/* shard_stream_quant with the 1-bit QJL residual (quantize_per_token with
 * qjl=True, streaming.py:67-70; stored by cache.py:234-240):
 *   res = r - codebook[idx] (fp32); qsign (rows, hd) uint8 = res >= 0;
 *   qscale (rows) fp16 = fp16(mean |res|), the sum in torch CPU's order for a
 *   contiguous fp32 row (element i into accumulator (i/8) % 4, lane i % 8, in
 *   increasing i; accumulators then lanes added in order), divided by hd;
 *   `deq` includes the residual: fp16(fp16(hadamard(codebook[idx] + (2 qsign - 1)
 *   qscale) * signs) * norm) (streaming.py:74-79, cache.py:275-278).
 * qsign and qscale are both null (exactly shard_stream_quant) or both set. */
int shard_stream_quant_qjl(const uint16_t* x, int64_t rows, int32_t hd,
                           const float* signs, const float* codebook, int32_t n_codes,
                           uint8_t* idx, uint16_t* norm, uint8_t* qsign, uint16_t* qscale,
                           uint16_t* deq, void* stream);

/* One decode token's K and V in one launch: shard_stream_quant_qjl on k and on
 * v (rows each), with the same signs and codebook, as _stream_append quantizes
 * both per token (cache.py:207-215).  The QJL outputs are nullable in pairs. */
int shard_stream_quant_kv(const uint16_t* k, const uint16_t* v, int64_t rows, int32_t hd,
                          const float* signs, const float* codebook, int32_t n_codes,
                          uint8_t* k_idx, uint16_t* k_norm, uint16_t* k_deq,
                          uint8_t* v_idx, uint16_t* v_norm, uint16_t* v_deq,
                          uint8_t* k_qsign, uint16_t* k_qscale, uint8_t* v_qsign,
                          uint16_t* v_qscale, void* stream);

/* The decode step's front end for one layer, in one launch: RoPE of q and k
 * exactly as transformers' apply_rotary_pos_emb computes it in fp16 (each
 * product and the sum rounded to fp16), then the rotated k and v appended to
 * the stream as shard_stream_quant_kv does.  Replaces the patched forward's
 * apply_rotary_pos_emb + update(k, v) of a streaming layer
 * (attention.py:376-381, cache.py:193-241).
 *   q (B, n_q_heads, hd), k and v (B, n_kv_heads, hd): fp16; cos and sin fp16
 *   rows of hd, batch row b at b * cos_stride (0: one row shared by the batch,
 *   as transformers passes it when the positions are the same)
 *   q_rope (B, n_q_heads, hd) fp16 out; the k_* / v_* outputs are the rows of
 *   this token in the stream buffers (codes, norms, fp16 rows; QJL nullable).
 * hd = 64, 128 or 256. */
int shard_rope_stream_append(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                             const uint16_t* cos, const uint16_t* sin, int64_t cos_stride,
                             int32_t batch,
                             int32_t n_q_heads, int32_t n_kv_heads, int32_t hd,
                             uint16_t* q_rope, const float* signs, const float* codebook,
                             int32_t n_codes, uint8_t* k_idx, uint16_t* k_norm, uint16_t* k_deq,
                             uint8_t* v_idx, uint16_t* v_norm, uint16_t* v_deq,
                             uint8_t* k_qsign, uint16_t* k_qscale, uint8_t* v_qsign,
                             uint16_t* v_qscale, void* stream);

/* shard_rope_stream_append with the token's stream row read from device
 * memory: the k_* / v_* outputs are the stream buffers' first rows, and the
 * token goes to row *row_dev of them (rows of B n_kv_heads entries), written
 * only when 0 <= *row_dev < row_cap (the buffers' rows).  No counterpart in
 * the reference; it lets one captured HIP graph append every decode step's
 * token while the stream grows (with shard_decode_args.n_stream_dev). */
int shard_rope_stream_append_dev(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* cos, const uint16_t* sin, int64_t cos_stride,
                                 int32_t batch, int32_t n_q_heads, int32_t n_kv_heads, int32_t hd,
                                 uint16_t* q_rope, const float* signs, const float* codebook,
                                 int32_t n_codes, uint8_t* k_idx, uint16_t* k_norm,
                                 uint16_t* k_deq, uint8_t* v_idx, uint16_t* v_norm,
                                 uint16_t* v_deq, uint8_t* k_qsign, uint16_t* k_qscale,
                                 uint8_t* v_qsign, uint16_t* v_qscale, const int32_t* row_dev,
                                 int32_t row_cap, void* stream);

/* shard_stream_dequant with the QJL residual term (streaming.py:76-77):
 * codebook[idx] + (2 qsign - 1) * qscale before the inverse Hadamard.
 * qsign (rows, hd) uint8 and qscale (rows) fp16 both null or both set. */
int shard_stream_dequant_qjl(const uint8_t* idx, const uint16_t* norm, const uint8_t* qsign,
                             const uint16_t* qscale, int64_t rows, int32_t hd,
                             const float* signs, const float* codebook, uint16_t* y,
                             void* stream);

/* ------------------------------------------------------------------------
 * Fused decode attention over the compressed cache
 * ------------------------------------------------------------------------ */

/* Arguments of one decode-attention call (one layer, one query token per row).
 * Layouts (B = batch, H = n_q_heads, G = n_kv_heads, D = head_dim, 128 or 64):
 *   q            (B, H, D) fp16, post-RoPE at position pos_q
 *   inv_freq     (D/2) fp32
 *   k_coeffs     (B*n_comp, rank/2) packed int4 (row-major, low nibble first)
 *   k_coeff_scale (rank) fp16;  k_basis (G*D, rank) fp16;  k_mean (G*D) fp16
 *   v_idx        (B, G, n_comp, D/4) uint8;  v_codebook (256, 4) fp16
 *   v_ch         (B, G, D) fp16
 *   sink_k/v     (B, G, n_sink, D) fp16;  win_k/v (B, G, n_win, D) fp16
 *   dec_k/v      (B, G, dec_stride, D) fp16, first n_dec tokens valid
 *   s_k/s_v      (>= n_stream, B, G, D) fp16: the 8-bit stream tokens as the
 *                reference dequantizes them (cache.py:275-278), written by
 *                shard_stream_quant's `deq` output when each token is appended
 *   mask         additive fp32, row b at mask + b*mask_stride, indexed in the
 *                reference's concatenation order [sink, comp, win, dec, stream]
 *                (nullable)
 *   out          (B, H, D) fp16
 * H / G (query heads per kv head) is at most 64 (128 / D up to 32 at D = 64):
 * the token-tiled kernel takes them in groups of 4, 3, 2 or 1 (the largest
 * that divides the count) per workgroup.  rank must be a multiple of 32
 * (<= 256; the row-split kernel takes <= 192, larger ranks run token-tiled);
 * pad coefficients and basis with zeros otherwise.  head_dim 64
 * needs an even G: the kernel runs kv heads 2j and 2j+1 as one 128-dim head
 * (the token-tiled kernel; `prep` from shard_decode_prepare with head_dim
 * 64), every layout above with D = 64 as it stands.  Any number of sink, window, decode and stream tokens (the
 * reference appends without limit, cache.py:156-181).  The softmax and all
 * sums run in fp32.
 * Replaces fused_attention_compressed (attention.py:270-343) with its
 * compressed_scores (18-81) and _v_weighted_sum_compressed (83-121), and the
 * flash-mixing of fused_attention_compressed_full (183-267). */
typedef struct shard_decode_args {
  int32_t batch, n_q_heads, n_kv_heads, head_dim;
  int32_t rank, n_comp, compress_start, pos_q;
  const uint16_t* q;
  const float* inv_freq;
  const uint8_t* k_coeffs;
  const uint16_t* k_coeff_scale;
  const uint16_t* k_basis;
  const uint16_t* k_mean;
  const void* prep;          /* shard_decode_prepare output of this layer */
  const uint8_t* v_idx;
  const uint16_t* v_codebook;
  const uint16_t* v_ch;
  const uint16_t* sink_k;
  const uint16_t* sink_v;
  int32_t n_sink;
  const uint16_t* win_k;
  const uint16_t* win_v;
  int32_t n_win;
  const uint16_t* dec_k;
  const uint16_t* dec_v;
  int32_t n_dec, dec_stride;
  const uint16_t* s_k;
  const uint16_t* s_v;
  int32_t n_stream, _pad0;
  const float* mask;
  int64_t mask_stride;
  uint16_t* out;
  int32_t n_splits; /* 0 = choose automatically */
  int32_t kernel;   /* split kernel: 0 = automatic, 1 = row-split (4 waves share a
                     * tile; 4 query heads per kv head, <= 2048 extra tokens;
                     * a call outside that runs on the token-tiled kernel),
                     * 2 = token-tiled (each wave owns whole tiles; every shape) */
  /* nullable device int64: when set, the kernel reads pos_q from it (the
   * reference's cache_position[-1], attention.py:383) and `pos_q` is ignored,
   * so the caller needs no host read-back of the position */
  const int64_t* pos_q_dev;
  /* nullable device int32: when set, the call attends over the first
   * min(*n_stream_dev, n_stream) stream rows, read at run time; n_stream then
   * bounds the count and sizes the work plan, so one captured HIP graph serves
   * every decode step while the stream grows.  No counterpart in the
   * reference (its counts are host integers).  Not together with `mask`. */
  const int32_t* n_stream_dev;
  /* V codebook shape (v_codebook is v_codebook_n x v_group fp16, v_idx holds
   * head_dim / v_group indices per token): 0 means the default 4 and 256.
   * shard_decode_attn takes group 4 with a 256-row codebook (pad a smaller
   * one with rows no index names); shard_kv_reconstruct takes groups 1, 2, 4
   * and 8 and 1..256 rows (cache.py:41-61: any Cache(v_vq_group_size,
   * v_vq_codebook_size) this build accepts). */
  int32_t v_group, v_codebook_n;
} shard_decode_args;

/* Per-layer constant operands of shard_decode_attn, computed once after a
 * layer is compressed (they depend only on its basis, scales, mean and RoPE
 * frequencies): the MFMA operand image of fp16(k_basis * k_coeff_scale) with
 * the mean folded in, and the in-tile RoPE rotation tables.  `out` holds
 * shard_decode_prepare_bytes(n_kv_heads, rank) bytes (head_dim 64:
 * shard_decode_prepare_bytes(n_kv_heads / 2, rank), one image per pair of kv
 * heads) and is passed to shard_decode_attn as args->prep.  head_dim 128, or
 * 64 with n_kv_heads even; rank % 32 == 0, rank <= 256.  The mean and the
 * nibble offsets fold into one constant k-step per key dim, C = 16 mean -
 * 16512 sum_{even r} A'(r) - 1152 sum_{odd r} A'(r) with A' = fp16(basis *
 * coeff_scale), held as 16 bf16 parts (a bf16 MFMA k-step): any finite C. */
size_t shard_decode_prepare_bytes(int32_t n_kv_heads, int32_t rank);
int shard_decode_prepare(const uint16_t* k_basis, const uint16_t* k_coeff_scale,
                         const uint16_t* k_mean, const float* inv_freq, int32_t n_kv_heads,
                         int32_t head_dim, int32_t rank, void* out, size_t out_bytes,
                         void* stream);

/* 1 when shard_decode_attn takes the shapes in `args` (head_dim 128 with up
 * to 64 query heads per kv head, or head_dim 64 with an even number of kv
 * heads and up to 32 query heads per kv head; rank a multiple of 32 up to 256;
 * V subvectors of 4 values from a 256-row codebook), else 0: the caller then
 * rebuilds fp16 K/V (shard_kv_reconstruct) and runs
 * plain attention, as the reference's unfused path does (attention.py:411). */
int shard_decode_supported(const shard_decode_args* args);

/* Workspace bytes of one call with these arguments (0: unsupported shape).
 * The size depends on every count (batch, context, extra tokens, n_splits,
 * kernel), so ask again whenever one changes. */
size_t shard_decode_attn_workspace(const shard_decode_args* args);
int shard_decode_attn(const shard_decode_args* args, void* workspace,
                      size_t workspace_bytes, void* stream);

/* shard_decode_attn without a workspace argument and without any allocation:
 * the partial rows go to a device array of the library,
 * SHARD_DECODE_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same kernels and results as shard_decode_attn; a call whose
 * shard_decode_attn_workspace(args) exceeds the scratch returns
 * SHARD_ERR_WORKSPACE (shard_last_error says by how much).  Runs on the
 * current device, whose scratch every call shares: calls that overlap on one
 * GPU (two streams, two threads) race on it.  Nothing in it needs clearing
 * between calls (every split writes its whole partial row). */
#define SHARD_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)8 << 20)
int shard_decode_attn_noalloc(const shard_decode_args* args, void* stream);

/* Full fp16 reconstruction of the compressed segment for unfused consumers,
 * _ensure_dequant (cache.py:87-124), using the compressed-segment fields of
 * `args` (q, out and the fp16 segments are ignored):
 *   K: fp16(fp16(sum_r fp16(nib*cs) * basis) + mean), then RoPE re-applied at
 *      positions compress_start + t with fp32 phases fl(pos*theta), fp16 out;
 *   V: fp16(hadamard(cb[idx] * ch)) (hadamard in fp32, bit-exact), for
 *      subvectors of args->v_group values (1, 2, 4 or 8) from a codebook of
 *      args->v_codebook_n rows (<= 256; 0 means 4 and 256).
 * k_out / v_out: (B, G, n_comp, D) fp16 contiguous.  D = 64, 128 or 256; any
 * even rank whose (32 + D) x rank fp16 staging fits 160 KB of LDS (rank <= 512
 * at D = 128), so layers the fused call does not take (rank above 256) decode
 * through it. */
int shard_kv_reconstruct(const shard_decode_args* args, uint16_t* k_out,
                         uint16_t* v_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SHARD_HIP_H */
