"""Writes the golden fixtures in this folder by running the reference in THIS
container (never on the GPU box).  Only functions that no closed form,
invariant or library routine pins are recorded here:

  lloyd_max.npz      lloyd_max_codebook(128, 8)  (streaming.py:35-51) — the
                     100th, non-converged Lloyd iterate
  lloyd_max_bits.npz lloyd_max_codebook(128, b) for b = 3..7, the widths that
                     do not converge within 100 iterations either (1 and 2
                     bits converge and are pinned by Max's table instead)
  kmeans.npz         kmeans(data, 16, 30, seed 42) on 600 x 4 fp32 rows
                     (cache.py:21-39): pre-update indices, CPU randperm init
  fused_attn.npz     fused_attention_compressed on a hand-built stub cache
                     (attention.py:270-343, non-Triton CPU branches) with
                     sink, window and an 8-bit stream: pins the reference's
                     fp16 cast points.  Same stub technique as the reference's
                     own benchmarks/kernel_test.py:178-259.

Usage:  python tests/golden/make_golden.py /root/reference [fixture ...]
        (no fixture names: write all of them)
The fixtures hold inputs and outputs only (arrays), no reference source.
"""
import os
import sys
import types

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def main(ref_root, only=()):
    sys.path.insert(0, os.path.join(ref_root, "src"))
    from shard.streaming import lloyd_max_codebook, quantize_per_token  # noqa: F401
    from shard import cache as rcache
    from shard.attention import fused_attention_compressed

    want = lambda name: not only or name in only

    # 1. Lloyd-Max codebooks
    if want("lloyd_max.npz"):
        cb = lloyd_max_codebook(128, 8).numpy().astype(np.float32)
        np.savez(os.path.join(HERE, "lloyd_max.npz"), codebook=cb, d=128, bits=8)
    if want("lloyd_max_bits.npz"):
        books = {f"cb{b}": lloyd_max_codebook(128, b).numpy().astype(np.float32)
                 for b in range(3, 8)}
        np.savez(os.path.join(HERE, "lloyd_max_bits.npz"), d=128, **books)

    # 2. k-means on small data
    if want("kmeans.npz"):
        g = torch.Generator().manual_seed(123)
        data = torch.randn(600, 4, generator=g)
        cent, idx = rcache.kmeans(data, 16, n_iter=30, seed=42)
        np.savez(os.path.join(HERE, "kmeans.npz"), data=data.numpy(), centroids=cent.numpy(),
                 idx=idx.numpy().astype(np.int64), k=16, n_iter=30, seed=42)
    if not want("fused_attn.npz"):
        return

    # 3. fused attention on a stub cache layer (B=1, 8 q heads, 2 kv heads, hd 128)
    g = torch.Generator().manual_seed(7)
    B, n_q, nkv, hd, rank, n_comp, sink, win, n_stream = 1, 8, 2, 128, 32, 40, 4, 8, 3
    start = sink
    inv_freq = 1.0 / (500000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    basis_q = torch.randint(-127, 128, (nkv * hd, rank), generator=g).to(torch.int8)
    basis_scale = (torch.rand(rank, generator=g) * 0.004 + 0.001).half()
    q4 = torch.randint(-7, 8, (B * n_comp, rank), generator=g)
    sh = (q4 + 8).to(torch.uint8).reshape(-1)
    packed = sh[0::2] | (sh[1::2] << 4)
    coeff_scale = (torch.rand(rank, generator=g) * 0.3 + 0.05).half()
    mean = (torch.randn(nkv * hd, generator=g) * 0.2).half()
    v_idx = torch.randint(0, 256, (B * nkv * n_comp * (hd // 4),), generator=g).to(torch.uint8)
    cent_h = (torch.randn(256, 4, generator=g) * 0.5).half()
    ch = (torch.rand(B * nkv, hd, generator=g) * 2 + 0.5).half()
    sink_k = torch.randn(B, nkv, sink, hd, generator=g).half()
    sink_v = torch.randn(B, nkv, sink, hd, generator=g).half()
    win_k = torch.randn(B, nkv, win, hd, generator=g).half()
    win_v = torch.randn(B, nkv, win, hd, generator=g).half()
    s_kidx = torch.randint(0, 256, (n_stream, B, nkv, hd), generator=g).to(torch.uint8)
    s_vidx = torch.randint(0, 256, (n_stream, B, nkv, hd), generator=g).to(torch.uint8)
    s_kn = (torch.rand(n_stream, B, nkv, generator=g) * 10 + 1).half()
    s_vn = (torch.rand(n_stream, B, nkv, generator=g) * 10 + 1).half()
    signs = ((torch.randint(0, 2, (hd,), generator=g) * 2 - 1).float())
    q_rope = torch.randn(B, n_q, 1, hd, generator=g).half()
    pos_q = start + n_comp + win + n_stream - 1

    gc = {
        "k_coeffs": packed, "k_coeffs_shape": (B * n_comp, rank),
        "k_coeff_scale": coeff_scale, "k_basis_q": basis_q, "k_basis_scale": basis_scale,
        "k_basis_f16": (basis_q.to(torch.float16) * basis_scale.to(torch.float16)).contiguous(),
        "k_mean": mean, "k_mean_f16": mean,
        "v_qdata": {"centroids": cent_h, "packed": v_idx, "ch_maxabs": ch,
                    "shape": (B * nkv, n_comp, hd), "group_size": 4, "bits": 8,
                    "n_orig": v_idx.numel()},
        "sink_k": sink_k, "sink_v": sink_v, "win_k": win_k, "win_v": win_v,
        "n_compress": n_comp, "batch": B, "compress_start": start,
        "signs": signs, "stream_n": n_stream * B,
        "k_idx_buf": s_kidx, "v_idx_buf": s_vidx, "k_norm_buf": s_kn, "v_norm_buf": s_vn,
    }
    cref = types.SimpleNamespace(_n_kv_heads=nkv, _stream_bits=8, _stream_qjl=False)
    layer = types.SimpleNamespace(_gpu_compressed=gc, _cache_ref=cref)
    layer._dequant_stream = types.MethodType(rcache.CacheLayer._dequant_stream, layer)
    with torch.no_grad():
        out = fused_attention_compressed(q_rope, layer, pos_q, inv_freq, None)
    np.savez(os.path.join(HERE, "fused_attn.npz"),
             q_rope=q_rope.numpy(), pos_q=pos_q, inv_freq=inv_freq.numpy(),
             k_coeffs=packed.numpy(), rank=rank, n_comp=n_comp, start=start,
             k_coeff_scale=coeff_scale.numpy(), k_basis_q=basis_q.numpy(),
             k_basis_scale=basis_scale.numpy(), k_mean=mean.numpy(), v_idx=v_idx.numpy(),
             centroids=cent_h.numpy(), ch=ch.numpy(), sink_k=sink_k.numpy(),
             sink_v=sink_v.numpy(), win_k=win_k.numpy(), win_v=win_v.numpy(),
             s_kidx=s_kidx.numpy(), s_vidx=s_vidx.numpy(), s_knorm=s_kn.numpy(),
             s_vnorm=s_vn.numpy(), signs=signs.numpy(), out=out.numpy())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", tuple(sys.argv[2:]))
