/* Benchmark-only entry points of libshard_hip.so: baselines the benchmark
 * times next to the compressed-KV path.  No product code calls them. */
#ifndef SHARD_BENCH_H
#define SHARD_BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp16 split-K GQA decode attention over uncompressed K/V (FlashDecoding
 * style), the same-GPU baseline of the compressed decode call.  q (B, 4 G, 128),
 * k and v (B, G, seq, 128), out (B, 4 G, 128), all fp16 contiguous, q / k / v
 * 16-byte aligned; scores scaled by 1/sqrt(128), no mask.  Work is split over
 * n_splits token ranges per (batch row, kv head), then merged. */
size_t shard_bench_fp16_decode_workspace(int32_t batch, int32_t n_kv_heads, int32_t n_splits);
int shard_bench_fp16_decode(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            int32_t batch, int32_t n_kv_heads, int32_t seq, int32_t n_splits,
                            uint16_t* out, void* workspace, size_t workspace_bytes,
                            void* stream);
/* The same over k / v buffers holding head_rows >= seq rows per (batch row,
 * kv head), of which the first seq are attended: k (B, G, head_rows, 128), as
 * a preallocated fp16 cache keeps them between decode steps. */
int shard_bench_fp16_decode_ld(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               int32_t batch, int32_t n_kv_heads, int32_t seq, int64_t head_rows,
                               int32_t n_splits, uint16_t* out, void* workspace,
                               size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SHARD_BENCH_H */
