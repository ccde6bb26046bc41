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
  int4_chain.npz     the K coefficient chain of _compress_k / _build_gpu_format:
                     quantize_group -> dequantize_group (rope.py:95-161) ->
                     col-max/7 scale and round/clamp (cache.py:416-419) ->
                     int4_pack (triton_kernels.py:665-676, CPU branch) on
                     2000 x 192 fp32 projections with 0/2/4/6/8-bit columns,
                     including columns whose values land exactly on .5 code
                     boundaries in either rounding step (half-even pinned).

  compress.npz       one layer of Cache.compress (cache.py:338-366): the
                     reference's own _compress_k (368-396) and _compress_v
                     (398-404) on a two-batch-row, 2-kv-head layer with RoPE'd
                     low-rank keys and outlier V channels, then the K/V
                     statements of _build_gpu_format (406-454) on the CPU (it
                     hard-codes "cuda").  torch.svd_lowrank is replaced by a
                     stub returning a fixed (S, V) (the float64 SVD of the
                     centred keys, stored in the fixture): the randomized
                     routine depends on the device RNG.  Pins the flatten
                     order, centring, DP allocation, keep-even, int8 basis,
                     fp32 projection -> group codes -> int4 chain, and the V
                     codec's Hadamard, channel scales, subvector order and
                     k-means.
  ensure_dequant.npz CacheLayer._ensure_dequant (cache.py:87-124) on a stub
                     layer (B = 2, 2 kv heads, rank 48, 3 stream
                     tokens, 2 fp16 decode tokens): the rebuilt K (int4 ->
                     basis -> mean -> view(B, n, nkv, hd) -> RoPE) and V
                     (vq_decode -> Hadamard) with the sink / window / stream /
                     decode concatenation; plus vq_decode (cache.py:54-61) alone.

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

# Column parameters (bits, lo * 8, rng * 8) whose dequantized values divided by
# col-max/7 land exactly on k + 0.5 in fp32 for two or more codes (found by
# enumerating lo, rng over multiples of 1/8).
_INT4_TIE_COLS = [(2, -60, 90), (2, -56, 36), (4, -56, 20), (4, -58, 87), (6, -62, 93),
                  (6, -60, 30), (8, -60, 102), (8, -56, 15)]


def int4_chain_inputs(n=2000, seed=11):
    """(proj (n, 192) fp32, alloc) for int4_chain.npz.

    Columns: Gaussian with varied scales and offsets (most); for each width,
    columns on the group quantizer's exact .5 boundaries (min 0, max L 2^e,
    values (j + 0.5) 2^e, which (x - lo) / rng * L maps to j + 0.5 exactly);
    columns of _INT4_TIE_COLS, filled with exact code points so the int4
    rounding meets .5 ties; a constant column and one with a range below the
    1e-6 clamp."""
    rs = np.random.default_rng(seed)
    alloc = [8] * 40 + [6] * 30 + [4] * 50 + [2] * 30 + [0] * 10 + [4] * 20 + [8] * 12
    keep = len(alloc)
    proj = (rs.standard_normal((n, keep)) * rs.uniform(0.05, 4.0, keep)
            + rs.uniform(-1.0, 1.0, keep)).astype(np.float32)
    nxt = {b: alloc.index(b) for b in (2, 4, 6, 8)}  # next unused column of each width

    def take(b):
        c = nxt[b]
        nxt[b] = alloc.index(b, c + 1)
        return c

    for b in (2, 4, 6, 8):  # stage-1 ties, two columns per width
        for e in (-3, 1):
            c = take(b)
            L = (1 << b) - 1
            j = rs.integers(0, L, n)
            x = ((j + 0.5) * 2.0 ** e).astype(np.float32)
            x[0], x[1] = 0.0, L * 2.0 ** e
            proj[:, c] = x
    for b, lo8, r8 in _INT4_TIE_COLS:  # stage-2 ties
        c = take(b)
        L = (1 << b) - 1
        lo, r = np.float32(lo8 / 8.0), np.float32(r8 / 8.0)
        codes = rs.integers(0, L + 1, n).astype(np.float32)
        codes[0], codes[1] = 0, L
        proj[:, c] = ((codes / np.float32(L)).astype(np.float32) * r).astype(np.float32) + lo
    proj[:, take(8)] = np.float32(0.75)                                 # constant column
    proj[:, take(8)] = np.float32(0.5) + rs.integers(0, 2, n).astype(np.float32) * np.float32(2e-7)
    return proj, alloc


def group_header(blob, alloc):
    """Per-column (lo, rng) fp32 from a quantize_group blob (rope.py:120-124's
    layout: int32 group count and rows, int16 (start, size, bits) per group,
    then (lo, rng) fp32 per column of the non-zero groups); zero for 0-bit
    columns."""
    import zlib
    raw = zlib.decompress(blob)
    ng = int(np.frombuffer(raw[:4], np.int32)[0])
    off, groups = 8, []
    for _ in range(ng):
        s, g, b = (int(v) for v in np.frombuffer(raw[off:off + 6], np.int16))
        groups.append((s, g, b))
        off += 6
    nz = sum(g for _, g, _ in groups)
    hdr = np.frombuffer(raw[off:off + nz * 8], np.float32).reshape(-1, 2)
    lo = np.zeros(len(alloc), np.float32)
    rng = np.zeros(len(alloc), np.float32)
    ci = 0
    for s, g, _ in groups:
        lo[s:s + g] = hdr[ci:ci + g, 0]
        rng[s:s + g] = hdr[ci:ci + g, 1]
        ci += g
    return lo, rng


def compress_inputs(seed=21, B=2, nkv=2, hd=128, T=200):
    """(k_full, v_full fp16 (B, nkv, T, hd), inv_freq fp32) for compress.npz.

    K: no-RoPE rows z diag(sigma) W^T + offset (W a random orthonormal p x p,
    sigma_i = exp(-i / 24), so a few dozen components hold the energy),
    normalized to unit per-dim std, then RoPE at positions 0..T-1 (theta
    500000), fp16.  V: N(0, 1) with two channels scaled x8, fp16."""
    g = torch.Generator().manual_seed(seed)
    p = nkv * hd
    W, _ = torch.linalg.qr(torch.randn(p, p, generator=g, dtype=torch.float64))
    sig = torch.exp(-torch.arange(p, dtype=torch.float64) / 24.0)
    z = torch.randn(B * T, p, generator=g, dtype=torch.float64)
    kn = (z * sig) @ W.T
    kn = kn / kn.std(dim=0).clamp(min=1e-12) + torch.randn(p, generator=g, dtype=torch.float64) * 0.3
    kn = kn.view(B, T, nkv, hd).permute(0, 2, 1, 3)
    inv_freq = 1.0 / (500000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    ph = torch.arange(T, dtype=torch.float64)[:, None] * inv_freq.double()[None, :]
    c, s = ph.cos(), ph.sin()
    k1, k2 = kn[..., : hd // 2], kn[..., hd // 2:]
    k_full = torch.cat([k1 * c - k2 * s, k2 * c + k1 * s], dim=-1).half()
    v = torch.randn(B, nkv, T, hd, generator=g)
    out_ch = torch.randperm(p, generator=g)[:2]
    vf = v.permute(0, 2, 1, 3).reshape(B, T, p)
    vf[:, :, out_ch] *= 8.0
    v_full = vf.view(B, T, nkv, hd).permute(0, 2, 1, 3).contiguous().half()
    return k_full.contiguous(), v_full, inv_freq


def write_compress(rcache):
    """compress.npz: see the module docstring."""
    import types
    from shard.rope import dequantize_group, unpack_nbits
    from shard.triton_kernels import int4_pack
    B, nkv, hd, T, sink, win, max_rank, cr = 2, 2, 128, 200, 4, 64, 192, 4.0
    k_full, v_full, inv_freq = compress_inputs(B=B, nkv=nkv, hd=hd, T=T)
    start, end = sink, T - win
    n_comp = end - start
    positions = torch.arange(T)[start:end]
    p = nkv * hd
    # the fixed (S, V) the svd_lowrank stub returns: the float64 SVD of the
    # centred no-RoPE keys, computed with the reference's own statements
    from shard.rope import undo_rope
    kk = undo_rope(k_full[:, :, start:end, :].float(), positions, inv_freq)
    flat = kk.permute(0, 2, 1, 3).reshape(B * n_comp, p)
    x64 = (flat - flat.mean(dim=0)).double()
    _, S64, Vh64 = torch.linalg.svd(x64, full_matrices=False)
    S_fix, V_fix = S64.float().contiguous(), Vh64.t().float().contiguous()
    stub = types.SimpleNamespace(_rope_inv_freq=inv_freq, _per_layer_dim=p, _max_rank_k=max_rank,
                                 _k_target_cr=cr, _n_kv_heads=nkv, head_dim=hd,
                                 _v_vq_group_size=4, _v_vq_codebook_size=256)
    saved = torch.svd_lowrank
    torch.svd_lowrank = lambda A, q=6, niter=2, M=None: (None, S_fix, V_fix)
    try:
        torch.manual_seed(42)  # Cache.compress seeds 42 + layer index before layer 0
        kd = rcache.Cache._compress_k(stub, k_full[:, :, start:end, :], positions, B, n_comp)
        vd = rcache.Cache._compress_v(stub, v_full[:, :, start:end, :], B)
    finally:
        torch.svd_lowrank = saved
    # _build_gpu_format's K and V statements (cache.py:412-427) on the CPU
    n_total = kd["k_n_total"]
    keep = len(kd["k_alloc"])
    coeffs = dequantize_group(kd["k_bytes"], kd["k_alloc"], n_total, "cpu")
    col_max = coeffs.abs().amax(dim=0).clamp(min=1e-6)
    coeff_scale = col_max / 7.0
    q = (coeffs / coeff_scale).round().clamp(-7, 7).to(torch.int8)
    k_coeffs = int4_pack(q)
    qd = vd["v_qdata"]
    ng = hd // qd["group_size"]
    v_idx = unpack_nbits(qd["packed"], qd["bits"], qd["n_orig"])
    v_idx_row0 = v_idx[: nkv * n_comp * ng].view(nkv, n_comp, ng).to(torch.uint8)
    k_basis_f16 = (kd["k_basis_q"][:, :keep].to(torch.float16)
                   * kd["k_scale"][:keep].to(torch.float16)).contiguous()
    lo, rng = group_header(kd["k_bytes"], kd["k_alloc"])
    np.savez_compressed(
        os.path.join(HERE, "compress.npz"),
        k_full=k_full.numpy(), v_full=v_full.numpy(), inv_freq=inv_freq.numpy(),
        sink=sink, win=win, max_rank=max_rank, k_target_cr=cr,
        svd_S=S_fix.numpy(), svd_V=V_fix.numpy(),
        k_basis_q=kd["k_basis_q"].numpy(), k_scale=kd["k_scale"].numpy(),
        k_mean=kd["k_mean"].numpy(), alloc=np.asarray(kd["k_alloc"], np.int32),
        lo=lo, rng=rng, deq=coeffs.numpy().astype(np.float32), q=q.numpy(),
        coeff_scale=coeff_scale.numpy().astype(np.float32), k_coeffs=k_coeffs.numpy(),
        k_basis_f16=k_basis_f16.numpy(),
        centroids=qd["centroids"].numpy(), v_packed=qd["packed"].numpy().astype(np.uint8),
        ch_maxabs=qd["ch_maxabs"].numpy(), v_indices_row0=v_idx_row0.numpy())


def write_ensure_dequant(rcache):
    """ensure_dequant.npz: see the module docstring."""
    import types
    g = torch.Generator().manual_seed(31)
    B, nkv, hd, rank, n_comp, sink, win, n_stream, n_dec = 2, 2, 128, 48, 37, 4, 8, 3, 2
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
    seg = lambda n: torch.randn(B, nkv, n, hd, generator=g).half()
    sink_k, sink_v, win_k, win_v, dec_k, dec_v = seg(sink), seg(sink), seg(win), seg(win), seg(n_dec), seg(n_dec)
    s_kidx = torch.randint(0, 256, (n_stream, B, nkv, hd), generator=g).to(torch.uint8)
    s_vidx = torch.randint(0, 256, (n_stream, B, nkv, hd), generator=g).to(torch.uint8)
    s_kn = (torch.rand(n_stream, B, nkv, generator=g) * 10 + 1).half()
    s_vn = (torch.rand(n_stream, B, nkv, generator=g) * 10 + 1).half()
    signs = ((torch.randint(0, 2, (hd,), generator=g) * 2 - 1).float())
    qdata = {"centroids": cent_h, "packed": v_idx, "ch_maxabs": ch, "shape": (B * nkv, n_comp, hd),
             "group_size": 4, "bits": 8, "n_orig": v_idx.numel()}
    gc = {
        "k_coeffs": packed, "k_coeffs_shape": (B * n_comp, rank), "k_coeff_scale": coeff_scale,
        "k_basis_q": basis_q, "k_basis_scale": basis_scale, "k_mean": mean,
        "v_qdata": qdata, "sink_k": sink_k, "sink_v": sink_v, "win_k": win_k, "win_v": win_v,
        "n_compress": n_comp, "batch": B, "compress_start": start,
        "signs": signs, "stream_n": n_stream * B,
        "k_idx_buf": s_kidx, "v_idx_buf": s_vidx, "k_norm_buf": s_kn, "v_norm_buf": s_vn,
        "decode_k": dec_k, "decode_v": dec_v,
    }
    cref = types.SimpleNamespace(_n_kv_heads=nkv, head_dim=hd, _rope_inv_freq=inv_freq,
                                 _stream_bits=8, _stream_qjl=False)
    layer = types.SimpleNamespace(_gpu_compressed=gc, _cache_ref=cref, _needs_decompress=True,
                                  _keys=None, _values=None)
    layer._dequant_stream = types.MethodType(rcache.CacheLayer._dequant_stream, layer)
    with torch.no_grad():
        rcache.CacheLayer._ensure_dequant(layer)
        vdec = rcache.vq_decode(qdata, "cpu")
    np.savez_compressed(
        os.path.join(HERE, "ensure_dequant.npz"),
        inv_freq=inv_freq.numpy(), rank=rank, n_comp=n_comp, start=start, batch=B,
        k_coeffs=packed.numpy(), k_coeff_scale=coeff_scale.numpy(), k_basis_q=basis_q.numpy(),
        k_basis_scale=basis_scale.numpy(), k_mean=mean.numpy(), v_idx=v_idx.numpy(),
        centroids=cent_h.numpy(), ch=ch.numpy(), sink_k=sink_k.numpy(), sink_v=sink_v.numpy(),
        win_k=win_k.numpy(), win_v=win_v.numpy(), decode_k=dec_k.numpy(), decode_v=dec_v.numpy(),
        s_kidx=s_kidx.numpy(), s_vidx=s_vidx.numpy(), s_knorm=s_kn.numpy(), s_vnorm=s_vn.numpy(),
        signs=signs.numpy(), keys=layer._keys.numpy(), values=layer._values.numpy(),
        vq_decoded=vdec.numpy())


def main(ref_root, only=()):
    sys.path.insert(0, os.path.join(ref_root, "src"))
    from shard.streaming import lloyd_max_codebook, quantize_per_token  # noqa: F401
    from shard import cache as rcache
    from shard.attention import fused_attention_compressed

    want = lambda name: not only or name in only

    # 0. int4 coefficient chain
    if want("int4_chain.npz"):
        from shard.rope import dequantize_group, quantize_group
        from shard.triton_kernels import int4_pack
        proj, alloc = int4_chain_inputs()
        n = proj.shape[0]
        blob = quantize_group(torch.from_numpy(proj), alloc)
        deq = dequantize_group(blob, alloc, n, "cpu")
        # _build_gpu_format, cache.py:416-419 (its device is hard-coded to
        # "cuda"; the four statements are run here on the CPU tensors)
        col_max = deq.abs().amax(dim=0).clamp(min=1e-6)
        coeff_scale = col_max / 7.0
        q = (deq / coeff_scale).round().clamp(-7, 7).to(torch.int8)
        packed = int4_pack(q)
        lo, rng = group_header(blob, alloc)
        np.savez_compressed(os.path.join(HERE, "int4_chain.npz"), proj=proj,
                 alloc=np.asarray(alloc, np.int32), lo=lo, rng=rng,
                 deq=deq.numpy().astype(np.float32), q=q.numpy(),
                 coeff_scale=coeff_scale.numpy().astype(np.float32), packed=packed.numpy())

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
    if want("compress.npz"):
        write_compress(rcache)
    if want("ensure_dequant.npz"):
        write_ensure_dequant(rcache)
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
