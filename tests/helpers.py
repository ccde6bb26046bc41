"""Shared test builders: random compressed layers (the stub-cache technique of
the reference's benchmarks/kernel_test.py:178-259) and conversion of an
oracle-format layer to the device format of shard_amd."""
import numpy as np
import torch

from oracle import ref


def random_layer(B=1, nkv=8, hd=128, rank=192, n_comp=512, sink=4, win=64, n_stream=0,
                 n_dec=0, seed=0, inv_freq=None, basis_amp=0.05, stream_bits=8, qjl=False,
                 v_group=4, v_codebook=256):
    """A random compressed layer in the oracle's gc format (CPU tensors); V
    subvectors of v_group values from a codebook of v_codebook rows."""
    g = torch.Generator().manual_seed(seed)
    if inv_freq is None:
        inv_freq = ref.default_inv_freq(500000.0, hd)
    basis_q = torch.randint(-127, 128, (nkv * hd, rank), generator=g).to(torch.int8)
    basis_scale = (torch.rand(rank, generator=g) * basis_amp / 127 + 1e-4).half()
    q4 = torch.randint(-7, 8, (B * n_comp, rank), generator=g)
    sh = (q4 + 8).to(torch.uint8).reshape(-1)
    packed = sh[0::2] | (sh[1::2] << 4)
    # spectrum-like decay of the coefficient scales
    coeff_scale = (torch.exp(-torch.arange(rank) / 80.0) * 0.4 + 0.01).half()
    mean = (torch.randn(nkv * hd, generator=g) * 0.2).half()
    v_idx = torch.randint(0, v_codebook, (B, nkv, n_comp, hd // v_group), generator=g).to(torch.uint8)
    cent = (torch.randn(v_codebook, v_group, generator=g) * 0.5).half()
    ch = (torch.rand(B, nkv, hd, generator=g) * 2 + 0.5).half()
    gc = {
        "k_coeffs": packed, "k_coeffs_shape": (B * n_comp, rank),
        "k_coeff_scale": coeff_scale, "k_basis_q": basis_q, "k_basis_scale": basis_scale,
        "k_basis_f16": (basis_q.to(torch.float16) * basis_scale.to(torch.float16)).contiguous(),
        "k_mean": mean, "k_mean_f16": mean,
        "v_idx_full": v_idx, "v_centroids_f16": cent, "v_ch_f16": ch,
        "v_qdata": {"centroids": cent, "idx": v_idx.reshape(-1), "ch_maxabs": ch.view(B * nkv, hd),
                    "shape": (B * nkv, n_comp, hd), "group_size": v_group},
        "sink_k": torch.randn(B, nkv, sink, hd, generator=g).half(),
        "sink_v": torch.randn(B, nkv, sink, hd, generator=g).half(),
        "win_k": torch.randn(B, nkv, win, hd, generator=g).half(),
        "win_v": torch.randn(B, nkv, win, hd, generator=g).half(),
        "n_compress": n_comp, "batch": B, "compress_start": sink,
    }
    if n_dec:
        gc["decode_k"] = torch.randn(B, nkv, n_dec, hd, generator=g).half()
        gc["decode_v"] = torch.randn(B, nkv, n_dec, hd, generator=g).half()
    if n_stream:
        cb = ref.lloyd_max_codebook(hd, stream_bits)
        signs = ref.stream_signs(5, hd)
        xk = (torch.randn(n_stream, B, nkv, hd, generator=g) * 1.5).half().numpy()
        xv = torch.randn(n_stream, B, nkv, hd, generator=g).half().numpy()
        kq = ref.quantize_stream_token(xk, signs, cb, qjl=qjl)
        vq = ref.quantize_stream_token(xv, signs, cb, qjl=qjl)
        gc.update({"signs": signs, "stream_codebook": cb, "stream_n": n_stream * B,
                   "k_idx_buf": kq[0], "v_idx_buf": vq[0], "k_norm_buf": kq[1], "v_norm_buf": vq[1]})
        if qjl:
            gc.update({"k_qsign_buf": kq[2], "v_qsign_buf": vq[2],
                       "k_qscale_buf": kq[3], "v_qscale_buf": vq[3]})
    return gc, inv_freq


def to_device(gc, device, inv_freq, nkv=8, hd=128):
    """Oracle-format gc -> shard_amd device format (cache.compress_layer's keys)."""
    from shard_amd.cache import finalize_format
    B = gc["batch"]
    n_comp = gc["n_compress"]
    n_total, rank = gc["k_coeffs_shape"]
    t = lambda x: (x if torch.is_tensor(x) else torch.from_numpy(np.ascontiguousarray(x))).to(device)
    d = {
        "k_coeffs": t(gc["k_coeffs"]).contiguous(),
        "k_coeff_scale": t(gc["k_coeff_scale"]).contiguous(),
        "k_coeffs_shape": (n_total, rank),
        "k_basis_f16": t(gc["k_basis_f16"]).contiguous(),
        "k_mean_f16": t(gc["k_mean_f16"]).contiguous(),
        "v_indices": t(gc["v_idx_full"]).reshape(B, nkv, n_comp, hd // gc["v_qdata"]["group_size"]).contiguous(),
        "v_centroids_f16": t(gc["v_centroids_f16"]).contiguous(),
        "v_ch_f16": t(gc["v_ch_f16"]).reshape(B, nkv, hd).contiguous(),
        "sink_k": t(gc["sink_k"]).contiguous(), "sink_v": t(gc["sink_v"]).contiguous(),
        "win_k": t(gc["win_k"]).contiguous(), "win_v": t(gc["win_v"]).contiguous(),
        "n_compress": n_comp, "batch": B, "compress_start": gc["compress_start"],
        "n_kv": nkv, "head_dim": hd, "rank": rank,
    }
    if "decode_k" in gc:
        d["decode_k"] = t(gc["decode_k"]).contiguous()
        d["decode_v"] = t(gc["decode_v"]).contiguous()
    if gc.get("stream_n", 0):
        q = (lambda k: gc.get(k))
        kdeq = ref.dequantize_stream_token(gc["k_idx_buf"], gc["k_norm_buf"], gc["signs"],
                                           gc["stream_codebook"], q("k_qsign_buf"), q("k_qscale_buf"))
        vdeq = ref.dequantize_stream_token(gc["v_idx_buf"], gc["v_norm_buf"], gc["signs"],
                                           gc["stream_codebook"], q("v_qsign_buf"), q("v_qscale_buf"))
        d.update({"signs": t(np.asarray(gc["signs"], np.float32)),
                  "stream_codebook": t(np.asarray(gc["stream_codebook"], np.float32)),
                  "stream_n": gc["stream_n"],
                  "k_idx_buf": t(gc["k_idx_buf"]).contiguous(),
                  "v_idx_buf": t(gc["v_idx_buf"]).contiguous(),
                  "k_norm_buf": t(gc["k_norm_buf"]).contiguous(),
                  "v_norm_buf": t(gc["v_norm_buf"]).contiguous(),
                  "k_deq_buf": t(kdeq).contiguous(), "v_deq_buf": t(vdeq).contiguous()})
    finalize_format(d, torch.as_tensor(inv_freq), device)
    return d


def compare(got, want):
    """(max abs err, cosine) of two arrays."""
    g = np.asarray(got, np.float64).reshape(-1)
    w = np.asarray(want, np.float64).reshape(-1)
    err = float(np.max(np.abs(g - w)))
    cos = float(g @ w / (np.linalg.norm(g) * np.linalg.norm(w) + 1e-300))
    return err, cos


def batch_rows(gc, rows):
    """The oracle-format layer gc restricted to the batch rows `rows` (in that
    order): per-row coefficient bytes, V indices, channel scales and fp16
    segments; the shared tables are kept.  Stream tokens are not carried."""
    assert not gc.get("stream_n", 0), "batch_rows: layers without stream tokens"
    B, n_comp = gc["batch"], gc["n_compress"]
    n_total, rank = gc["k_coeffs_shape"]
    assert n_total == B * n_comp and rank % 2 == 0
    rows = list(rows)
    idx = torch.as_tensor(rows, dtype=torch.long)
    packed = torch.as_tensor(np.asarray(gc["k_coeffs"])).reshape(B, n_comp * rank // 2)
    out = dict(gc)
    out.update({
        "k_coeffs": packed[idx].reshape(-1).contiguous(),
        "k_coeffs_shape": (len(rows) * n_comp, rank),
        "v_idx_full": gc["v_idx_full"][idx].contiguous(),
        "v_ch_f16": gc["v_ch_f16"][idx].contiguous(),
        "batch": len(rows),
    })
    out.pop("v_qdata", None)
    for k in ("sink_k", "sink_v", "win_k", "win_v", "decode_k", "decode_v"):
        if k in gc:
            out[k] = gc[k][idx].contiguous()
    return out
