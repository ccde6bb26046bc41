"""The benchmark's same-GPU fp16 baseline (shard_bench_fp16_decode: split-K
GQA decode attention over uncompressed K/V) against fp64 softmax attention on
the same fp16 inputs, to the decode bar (max-abs-err 2e-3, cosine 0.9999)."""
import numpy as np
import pytest
import torch

from tests.helpers import compare

pytestmark = pytest.mark.gpu


def _fp64_attention(q, k, v):
    """q (B, H, D), k / v (B, G, T, D) -> (B, H, D); query head h uses kv head h // (H / G)."""
    q, k, v = (x.double().numpy() for x in (q, k, v))
    B, H, D = q.shape
    G = k.shape[1]
    kk = np.repeat(k, H // G, axis=1)
    vv = np.repeat(v, H // G, axis=1)
    s = np.einsum("bhd,bhtd->bht", q, kk) / np.sqrt(D)
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bht,bhtd->bhd", p, vv)


# the merge runs 8, 4, 2 or 1 slices per query head by batch x heads, and one
# slice when the head count is not a multiple of 8: (1, 1, ...) has 4 heads
@pytest.mark.parametrize("B,G,T,n_splits", [(1, 8, 8192, 0), (1, 8, 1000, 7), (2, 4, 333, 0),
                                             (3, 2, 100, 50), (1, 8, 32, 1), (4, 8, 300, 0),
                                             (8, 8, 256, 0), (16, 8, 64, 3), (1, 1, 500, 9)])
def test_fp16_baseline_matches_fp64(cuda, B, G, T, n_splits):
    from shard_amd import ops
    g = torch.Generator().manual_seed(T + B)
    q = torch.randn(B, 4 * G, 128, generator=g).half()
    k = (torch.randn(B, G, T, 128, generator=g) * 1.5).half()
    v = torch.randn(B, G, T, 128, generator=g).half()
    print(f"[fp16 baseline] B={B} G={G} T={T} n_splits={n_splits}", flush=True)
    got = ops.bench_fp16_decode(q.to(cuda), k.to(cuda), v.to(cuda), n_splits=n_splits)
    torch.cuda.synchronize()
    want = _fp64_attention(q, k, v)
    err, cos = compare(got.cpu().float().numpy(), want)
    print(f"[fp16 baseline] max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= 2e-3 and cos >= 0.9999


@pytest.mark.parametrize("B,G,T,rows", [(2, 8, 700, 1024), (16, 8, 257, 300)])
def test_fp16_baseline_over_a_preallocated_cache(cuda, B, G, T, rows):
    """shard_bench_fp16_decode_ld: the first T of `rows` rows per head (the
    e2e fp16 baseline's preallocated cache); rows past T hold NaN and must not
    reach the result."""
    from shard_amd import ops
    g = torch.Generator().manual_seed(T)
    q = torch.randn(B, 4 * G, 128, generator=g).half()
    k = torch.full((B, G, rows, 128), float("nan")).half()
    v = torch.full((B, G, rows, 128), float("nan")).half()
    k[:, :, :T] = (torch.randn(B, G, T, 128, generator=g) * 1.5).half()
    v[:, :, :T] = torch.randn(B, G, T, 128, generator=g).half()
    got = ops.bench_fp16_decode(q.to(cuda), k.to(cuda), v.to(cuda), seq=T)
    torch.cuda.synchronize()
    want = _fp64_attention(q, k[:, :, :T].contiguous(), v[:, :, :T].contiguous())
    err, cos = compare(got.cpu().float().numpy(), want)
    print(f"[fp16 baseline ld] B={B} T={T} rows={rows}: max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= 2e-3 and cos >= 0.9999
