"""Op-for-op CPU restatement of the reference compressed-KV path (test oracle).

Every function cites the reference file:line it follows (paths relative to the
reference's ``src/shard/``).  Float paths use torch on the CPU in the same op
order and dtypes as the reference's non-Triton fallbacks, so fp16 cast points
are kept; the integer chains are written in numpy with every fp32 rounding
explicit (no fused multiply-add anywhere in numpy elementwise code).

Test infrastructure only: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use it as the checker; the product never imports it.

How each function is pinned (checked in ``tests/test_oracle.py``):
  hadamard            closed form: Sylvester matrix H/sqrt(d) on small d; H.H = I.
  rope helpers        rotation-matrix closed form; undo(reapply(x)) = x.
  dp_bit_allocation   exhaustive enumeration of bit vectors on tiny inputs.
  group_quant/dequant bit formulas; codes equal brute-force nearest level.
  int4_chain/pack     bit formula; the reference's own kernel_test.py:133-146
                      relation (pack == flat[0::2] | flat[1::2] << 4).
  lloyd_max_codebook  golden vectors written by importing the reference
                      (tests/golden/make_golden.py) at 3..8 bits + Lloyd
                      fixed-point residual; Max's (1960) table at 1 and 2 bits.
  stream quantize     torch.norm (library) for the norm order; brute-force
                      nearest codebook entry in fp64 away from ties.
  QJL residual        torch.mean (library) for mean_fp32_4x8's order; sign
                      against fp64; the per-token error identity
                      |r - cb - s m|^2 = |r - cb|^2 - d m^2 for the dequant term.
  vq_assign           torch.cdist(...).argmin (the reference's own fallback,
                      triton_kernels.py:733-734) and fp64 brute force.
  kmeans              golden vectors from the reference import.
  fused attention     golden vectors from the reference import on a stub cache
                      (the reference's own kernel_test.py:178-259 technique),
                      reproduced bit for bit, and exact.py's fp64 evaluation.
  compress_layer      golden vectors of the reference's _compress_k +
                      _compress_v + _build_gpu_format (svd_lowrank replaced by
                      a fixed (S, V) on both sides, ``svd=``), bit for bit.
  reconstruct_kv,     golden vectors of the reference's _ensure_dequant on a
  vq_decode           two-batch-row stub layer and of vq_decode, bit for bit.
"""
import math

import numpy as np
import torch

F32 = np.float32


# --------------------------------------------------------------------------
# Hadamard (cache.py:10-19)
# --------------------------------------------------------------------------
def hadamard(x: torch.Tensor) -> torch.Tensor:
    """Normalized butterfly WHT on the last dim; cache.py:10-19.

    Stage h pairs element i with i+h inside blocks of 2h: (a+b, a-b); then one
    true division by sqrt(d) (a Python float, so fp32(sqrt(d)) for fp32 input).
    """
    d = x.shape[-1]
    h = 1
    while h < d:
        x = x.unflatten(-1, (-1, h * 2))
        a, b = x[..., :h], x[..., h:]
        x = torch.cat([a + b, a - b], dim=-1).flatten(-2)
        h *= 2
    return x / math.sqrt(d)


def hadamard_np(x: np.ndarray) -> np.ndarray:
    """numpy fp32 restatement of cache.py:10-19 (same pairing, same rounding)."""
    x = np.asarray(x, dtype=F32).copy()
    d = x.shape[-1]
    h = 1
    while h < d:
        y = x.reshape(*x.shape[:-1], d // (2 * h), 2 * h)
        a = y[..., :h].copy()
        b = y[..., h:].copy()
        y[..., :h] = a + b
        y[..., h:] = a - b
        x = y.reshape(*x.shape)
        h *= 2
    return (x / F32(math.sqrt(d))).astype(F32)


# --------------------------------------------------------------------------
# RoPE (rope.py:8-47)
# --------------------------------------------------------------------------
def rotate_half(x):
    """rope.py:8-11: [-x[..., d/2:], x[..., :d/2]]."""
    h = x.shape[-1] // 2
    return torch.cat([-x[..., h:], x[..., :h]], dim=-1)


def rope_cos_sin(positions, inv_freq):
    """rope.py:13-18 (fp32 phases fl(theta*pos), duplicated halves)."""
    if positions.dim() == 1:
        positions = positions.unsqueeze(0)
    freqs = inv_freq[None, :, None].float() @ positions[:, None, :].float()
    emb = torch.cat([freqs.transpose(1, 2)] * 2, dim=-1)
    return emb.cos(), emb.sin()


def undo_rope(keys, positions, inv_freq):
    """rope.py:20-24."""
    cos, sin = rope_cos_sin(positions, inv_freq.to(keys.device))
    while cos.dim() < keys.dim():
        cos = cos.unsqueeze(-3)
        sin = sin.unsqueeze(-3)
    return keys * cos - rotate_half(keys) * sin


def reapply_rope(keys, positions, inv_freq):
    """rope.py:26-30."""
    cos, sin = rope_cos_sin(positions, inv_freq.to(keys.device))
    while cos.dim() < keys.dim():
        cos = cos.unsqueeze(-3)
        sin = sin.unsqueeze(-3)
    return keys * cos + rotate_half(keys) * sin


def default_inv_freq(theta: float, hd: int) -> torch.Tensor:
    """rope.py:47: 1 / theta^(arange(0, hd, 2)/hd) in fp32."""
    return 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))


# --------------------------------------------------------------------------
# DP bit allocation (rope.py:49-84)
# --------------------------------------------------------------------------
def dp_bit_allocation(variances, total_budget):
    """rope.py:49-84: groups of 64, options {0,2,4,6,8}, unit 16, drop x4."""
    GROUP, OPTIONS, DROP, UNIT = 64, [0, 2, 4, 6, 8], 4.0, 16
    v = torch.as_tensor(variances).float().cpu()
    d = v.shape[0]
    ng = (d + GROUP - 1) // GROUP
    gs = [min(GROUP, d - g * GROUP) for g in range(ng)]
    gv = [v[g * GROUP: g * GROUP + gs[g]].sum().item() for g in range(ng)]
    mu = total_budget // UNIT + 1
    INF = float("inf")
    dp = [[INF] * (mu + 1) for _ in range(ng + 1)]
    back = [[0] * (mu + 1) for _ in range(ng + 1)]
    dp[0] = [0.0] * (mu + 1)
    for g in range(ng):
        for b in range(mu + 1):
            for bits in OPTIONS:
                cost = 0 if bits == 0 else (gs[g] * bits + UNIT - 1) // UNIT
                err = gv[g] * DROP if bits == 0 else gv[g] / (3.0 * (1 << (2 * bits)))
                if b - cost < 0:
                    continue
                c = dp[g][b - cost] + err
                if c < dp[g + 1][b]:
                    dp[g + 1][b] = c
                    back[g + 1][b] = bits
    best = min(range(mu + 1), key=lambda b: dp[ng][b])
    alloc = [0] * d
    b = best
    for g in range(ng - 1, -1, -1):
        bits = back[g + 1][b]
        for i in range(g * GROUP, g * GROUP + gs[g]):
            alloc[i] = bits
        if bits > 0:
            b -= (gs[g] * bits + UNIT - 1) // UNIT
    return alloc


# --------------------------------------------------------------------------
# Group quantizer values (rope.py:95-161) and the int4 chain (cache.py:416-420)
# --------------------------------------------------------------------------
def group_quant(proj: np.ndarray, alloc):
    """Values of quantize_group (rope.py:95-125) per column.

    Returns (codes uint8 (n, keep) with 0 for 0-bit columns, lo fp32 (keep,),
    rng fp32 (keep,)).  The zlib/bit-packing container is lossless, so only the
    values matter downstream (dequantize_group, rope.py:127-161).
    """
    proj = np.asarray(proj, dtype=F32)
    n, keep = proj.shape
    codes = np.zeros((n, keep), np.uint8)
    lo = np.zeros(keep, F32)
    rng = np.zeros(keep, F32)
    for c in range(keep):
        bits = int(alloc[c])
        if bits == 0:
            continue
        col = proj[:, c]
        l = col.min()
        r = max(F32(col.max() - l), F32(1e-6))           # .clamp(min=1e-6)
        levels = F32((1 << bits) - 1)
        v = ((col - l) / r).astype(F32)
        v = np.minimum(np.maximum(v, F32(0)), F32(1))     # .clamp(0, 1)
        v = (v * levels).astype(F32)
        q = np.rint(v)                                    # torch.round: half-even
        q = np.clip(q, 0, (1 << bits) - 1).astype(np.uint8)
        codes[:, c] = q
        lo[c] = l
        rng[c] = r
    return codes, lo, rng


def group_dequant(codes: np.ndarray, lo, rng, alloc) -> np.ndarray:
    """dequantize_group values (rope.py:156-159): arr/levels*s + sh, fp32 per op."""
    n, keep = codes.shape
    out = np.zeros((n, keep), F32)
    for c in range(keep):
        bits = int(alloc[c])
        if bits == 0:
            continue
        levels = F32((1 << bits) - 1)
        a = codes[:, c].astype(F32)
        out[:, c] = ((a / levels).astype(F32) * F32(rng[c])).astype(F32) + F32(lo[c])
    return out


def int4_quantize(coeffs: np.ndarray):
    """cache.py:417-419: cs = max(colabsmax, 1e-6)/7; q = clamp(round(c/cs), -7, 7)."""
    coeffs = np.asarray(coeffs, dtype=F32)
    col_max = np.maximum(np.abs(coeffs).max(axis=0), F32(1e-6)).astype(F32)
    cs = (col_max / F32(7.0)).astype(F32)
    q = np.clip(np.rint((coeffs / cs).astype(F32)), -7, 7).astype(np.int8)
    return q, cs


def int4_pack(q: np.ndarray) -> np.ndarray:
    """triton_kernels.py:665-676 fallback: ((x+8)&15) | ((x'+8)&15)<<4, pad odd with 0."""
    flat = np.asarray(q).reshape(-1).astype(np.int16)
    if flat.shape[0] & 1:
        flat = np.concatenate([flat, np.zeros(1, np.int16)])
    sh = ((flat + 8) & 0x0F).astype(np.uint8)
    return (sh[0::2] | (sh[1::2] << 4)).astype(np.uint8)


def int4_unpack(packed: np.ndarray, n_total: int, rank: int) -> np.ndarray:
    """attention.py:13-16 / cache.py:94-98: nibble - 8, row-major (n_total, rank)."""
    p = np.asarray(packed, dtype=np.uint8)
    lo = (p & 0x0F).astype(np.int16) - 8
    hi = ((p >> 4) & 0x0F).astype(np.int16) - 8
    return np.stack([lo, hi], axis=1).reshape(-1)[: n_total * rank].reshape(n_total, rank)


def k_code_chain(proj: np.ndarray, alloc):
    """Full integer chain proj -> group codes -> dequant -> int4 -> packed.

    Follows _compress_k's quantize_group (cache.py:395) and _build_gpu_format
    (cache.py:416-420).  Returns dict of every intermediate.
    """
    codes, lo, rng = group_quant(proj, alloc)
    deq = group_dequant(codes, lo, rng, alloc)
    q, cs = int4_quantize(deq)
    return {"codes": codes, "lo": lo, "rng": rng, "deq": deq, "q": q,
            "coeff_scale": cs, "packed": int4_pack(q)}


# --------------------------------------------------------------------------
# Lloyd-Max stream quantizer (streaming.py:11-79, cache.py:193-279)
# --------------------------------------------------------------------------
_A = [-3.969683028665376e+01, 2.209460984245205e+02, -2.759285104469687e+02,
      1.383577518672690e+02, -3.066479806614716e+01, 2.506628277459239e+00]
_B = [-5.447609879822406e+01, 1.615858368580409e+02, -1.556989798598866e+02,
      6.680131188771972e+01, -1.328068155288572e+01]
_C = [-7.784894002430293e-03, -3.223964580411365e-01, -2.400758277161838e+00,
      -2.549732539343734e+00, 4.374664141464968e+00, 2.938163982698783e+00]
_D = [7.784695709041462e-03, 3.224671290700398e-01,
      2.445134137142996e+00, 3.754408661907416e+00]


def acklam_inv_cdf(p):
    """Acklam's rational approximation of the standard normal quantile
    (streaming.py:11-33; published coefficients, P. J. Acklam 2003)."""
    lo, hi = 0.02425, 1 - 0.02425
    if p < lo:
        q = math.sqrt(-2 * math.log(p))
        return (((((_C[0]*q+_C[1])*q+_C[2])*q+_C[3])*q+_C[4])*q+_C[5]) / \
               ((((_D[0]*q+_D[1])*q+_D[2])*q+_D[3])*q+1)
    if p <= hi:
        q = p - 0.5
        r = q * q
        return (((((_A[0]*r+_A[1])*r+_A[2])*r+_A[3])*r+_A[4])*r+_A[5]) * q / \
               (((((_B[0]*r+_B[1])*r+_B[2])*r+_B[3])*r+_B[4])*r+1)
    q = math.sqrt(-2 * math.log(1 - p))
    return -(((((_C[0]*q+_C[1])*q+_C[2])*q+_C[3])*q+_C[4])*q+_C[5]) / \
            ((((_D[0]*q+_D[1])*q+_D[2])*q+_D[3])*q+1)


def lloyd_max_codebook(d, bits, n_iter=100):
    """streaming.py:35-51: Lloyd iterations for N(0, 1/d) in Python double.

    The loop breaks only when the max step < 1e-9 and then keeps the previous
    iterate; for (128, 8) it runs all 100 iterations.  Cast to fp32 at the end.
    """
    n = 1 << bits
    sigma = 1.0 / math.sqrt(d)
    c = [acklam_inv_cdf((i + 0.5) / n) * sigma for i in range(n)]
    phi = lambda z: math.exp(-0.5 * z * z) / math.sqrt(2 * math.pi)
    Phi = lambda z: 0.5 * (1 + math.erf(z / math.sqrt(2)))
    for _ in range(n_iter):
        bounds = [-1e9] + [(c[k - 1] + c[k]) / 2 for k in range(1, n)] + [1e9]
        nc = []
        for k in range(n):
            a, b = bounds[k], bounds[k + 1]
            m = Phi(b / sigma) - Phi(a / sigma)
            nc.append(c[k] if m < 1e-12 else (phi(a / sigma) - phi(b / sigma)) * sigma / m)
        if max(abs(x - y) for x, y in zip(nc, c)) < 1e-9:
            break
        c = nc
    return np.asarray(c, dtype=F32)


def stream_signs(layer_idx: int, hd: int) -> np.ndarray:
    """cache.py:201-204: CPU Generator(42 + layer*7919), randint(0,2)*2-1 as fp32."""
    g = torch.Generator(device="cpu").manual_seed(42 + layer_idx * 7919)
    return ((torch.randint(0, 2, (hd,), generator=g) * 2 - 1).to(torch.float32)).numpy()


def norm_fp32_8lane(t: np.ndarray) -> np.ndarray:
    """torch CPU fp32 last-dim 2-norm order: 8 strided accumulators summed
    left to right, then sqrt (matches torch.norm, checked in the tests)."""
    t = np.asarray(t, dtype=F32)
    d = t.shape[-1]
    sq = (t * t).astype(F32)
    acc = np.zeros(t.shape[:-1] + (8,), F32)
    for i in range(d):
        acc[..., i % 8] = (acc[..., i % 8] + sq[..., i]).astype(F32)
    tot = acc[..., 0].copy()
    for j in range(1, 8):
        tot = (tot + acc[..., j]).astype(F32)
    return np.sqrt(tot).astype(F32)


def mean_fp32_4x8(a: np.ndarray) -> np.ndarray:
    """torch CPU fp32 mean over a contiguous last dim (a multiple of 32): element
    i goes to accumulator (i // 8) % 4, lane i % 8, in increasing i; the four
    accumulators are added in order per lane, then the 8 lanes in order; then one
    division by the length.  (Pinned against torch's mean in the tests.)"""
    a = np.asarray(a, dtype=F32)
    d = a.shape[-1]
    acc = np.zeros(a.shape[:-1] + (4, 8), F32)
    for i in range(d):
        k, j = (i // 8) % 4, i % 8
        acc[..., k, j] = (acc[..., k, j] + a[..., i]).astype(F32)
    v = acc[..., 0, :].copy()
    for k in range(1, 4):
        v = (v + acc[..., k, :]).astype(F32)
    tot = v[..., 0].copy()
    for j in range(1, 8):
        tot = (tot + v[..., j]).astype(F32)
    return (tot / F32(d)).astype(F32)


def quantize_stream_token(x_f16: np.ndarray, signs: np.ndarray, codebook: np.ndarray,
                          qjl: bool = False):
    """cache.py:207-215 (_unit) + streaming.py:59-72 (quantize_per_token).

    x_f16: (..., hd) float16.  Returns (idx uint8 (..., hd), norm float16 (...))
    and, with qjl, also (qsign uint8 (..., hd), qscale float16 (...)): the sign
    of the residual r - cb[idx] and fp16(mean |r - cb[idx]|) (streaming.py:67-70).
    """
    t = np.asarray(x_f16, dtype=np.float16).astype(F32)
    n = np.maximum(norm_fp32_8lane(t), F32(1e-8))
    u = (t / n[..., None]).astype(F32)
    r = hadamard_np((u * np.asarray(signs, F32)).astype(F32))
    cb = np.asarray(codebook, F32)
    idx = np.searchsorted(cb, r, side="left")             # torch.bucketize, right=False
    idx = np.minimum(idx, cb.shape[0] - 1)
    left = np.maximum(idx - 1, 0)
    dl = np.abs((cb[left] - r).astype(F32))
    di = np.abs((cb[idx] - r).astype(F32))
    idx = np.where(dl < di, left, idx).astype(np.uint8)
    if qjl:
        res = (r - cb[idx.astype(np.int64)]).astype(F32)
        qsign = (res >= 0).astype(np.uint8)
        qscale = mean_fp32_4x8(np.abs(res)).astype(np.float16)
        return idx, n.astype(np.float16), qsign, qscale
    return idx, n.astype(np.float16)


def dequantize_stream_token(idx: np.ndarray, norm_f16: np.ndarray, signs, codebook,
                            qsign=None, qscale=None):
    """streaming.py:74-79 + cache.py:275-278: fp16(fp16(H(cb[idx] (+ QJL term))
    * signs) * norm); the QJL term is (2 qsign - 1) * fp32(qscale)."""
    cb = np.asarray(codebook, F32)
    rot = cb[np.asarray(idx).astype(np.int64)]
    if qsign is not None:
        term = ((np.asarray(qsign).astype(F32) * F32(2) - F32(1))
                * np.asarray(qscale, np.float16).astype(F32)[..., None]).astype(F32)
        rot = (rot + term).astype(F32)
    u = (hadamard_np(rot) * np.asarray(signs, F32)).astype(np.float16)
    return (u.astype(F32) * np.asarray(norm_f16, np.float16).astype(F32)[..., None]).astype(np.float16)


# --------------------------------------------------------------------------
# VQ (cache.py:21-61, triton_kernels.py:689-746)
# --------------------------------------------------------------------------
def vq_assign_cdist(x: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    """triton_kernels.py:733-734 (CPU fallback): cdist(x, c).argmin(1)."""
    return torch.cdist(x, c).argmin(dim=1)


def vq_assign_direct(x: np.ndarray, c: np.ndarray) -> np.ndarray:
    """Direct fp32 sum of squared differences in dim order, no FMA; first index
    wins ties (triton_kernels.py:703-725's formula).  Used as the bit-exact
    oracle of the HIP assign kernel; agrees with vq_assign_cdist away from ties.
    """
    x = np.asarray(x, F32)
    c = np.asarray(c, F32)
    n, d = x.shape
    best = np.full(n, np.inf, F32)
    arg = np.zeros(n, np.int64)
    for k in range(c.shape[0]):
        dist = np.zeros(n, F32)
        for j in range(d):
            diff = (x[:, j] - c[k, j]).astype(F32)
            dist = (dist + (diff * diff).astype(F32)).astype(F32)
        better = dist < best
        best = np.where(better, dist, best)
        arg = np.where(better, k, arg)
    return arg


def kmeans(data: torch.Tensor, k: int, n_iter: int = 30, seed: int = 42, assign=None):
    """cache.py:21-39 on the CPU.  Returns (centroids fp32, idx int64) where idx
    is the LAST assignment, made against the centroids before the final update.
    ``assign`` defaults to the reference's CPU fallback (cdist argmin)."""
    assign = assign or vq_assign_cdist
    n, d = data.shape
    g = torch.Generator(device="cpu").manual_seed(seed)
    centroids = data[torch.randperm(n, generator=g)[:k]].clone()
    idx = None
    for it in range(n_iter):
        idx = assign(data, centroids)
        new = torch.zeros_like(centroids)
        counts = torch.zeros(k, dtype=data.dtype)
        new.index_add_(0, idx, data)
        counts.index_add_(0, idx, torch.ones(n, dtype=data.dtype))
        nz = counts > 0
        new[nz] /= counts[nz].unsqueeze(1)
        new[~nz] = centroids[~nz]
        if (new - centroids).abs().max().item() < 1e-4 and it >= 5:
            centroids = new
            break
        centroids = new
    return centroids, idx


def vq_encode(v: torch.Tensor, group_size: int, codebook_size: int, assign=None):
    """cache.py:41-52 (bits=8 packing is the identity, rope.py:164-165).
    ``assign`` is passed to kmeans (default: the CPU fallback's cdist)."""
    bh, seq, hd = v.shape
    ng = hd // group_size
    ch_max = v.abs().amax(dim=1).clamp(min=1e-8)
    flat = (v / ch_max.unsqueeze(1)).reshape(bh * seq, ng, group_size).reshape(-1, group_size)
    centroids, idx = kmeans(flat.float(), codebook_size, n_iter=30, assign=assign)
    return {"centroids": centroids.half(), "idx": idx.to(torch.uint8),
            "ch_maxabs": ch_max.half(), "shape": (bh, seq, hd),
            "group_size": group_size, "flat": flat, "centroids_f32": centroids}


def vq_decode(qd) -> torch.Tensor:
    """cache.py:54-61: centroids[idx] * ch_max (fp32)."""
    bh, seq, hd = qd["shape"]
    gs = qd["group_size"]
    idx = qd["idx"][: bh * seq * (hd // gs)].long()
    cb = qd["centroids"].float()
    ch = qd["ch_maxabs"].float()
    return cb[idx].reshape(bh, seq, hd) * ch.unsqueeze(1)


# --------------------------------------------------------------------------
# Compression (cache.py:338-460) producing the on-device format on the CPU
# --------------------------------------------------------------------------
def compress_layer(k_full: torch.Tensor, v_full: torch.Tensor, layer_idx: int,
                   inv_freq, sink=4, win=64, k_target_cr=20.0, max_rank=192,
                   group_size=4, codebook_size=256, basis=None, assign=None, svd=None):
    """One layer of Cache.compress (cache.py:338-366) + _compress_k (368-396) +
    _compress_v (398-404) + _build_gpu_format (406-454), on the CPU.

    ``basis`` (1024 x rank fp32, columns = components) may be supplied to
    bypass torch.svd_lowrank (its randomized result depends on the device RNG);
    the variances are then the mean squared projections.  ``svd`` = (S, V)
    instead stands for svd_lowrank's result itself (cache.py:376-378): the
    basis is V[:, :rank] and the variances S[:rank]^2 / n, as the reference
    takes them.
    ``assign`` is k-means' nearest-centroid rule (default: the CPU fallback's
    cdist argmin; the reference's GPU kernel sums squared differences directly,
    vq_assign_direct).
    Returns the gc dict with numpy/torch CPU arrays and all integer
    intermediates (codes, q) for parity tests.
    """
    B, nkv, seq, hd = k_full.shape
    start, end = sink, seq - win
    n_comp = end - start
    positions = torch.arange(seq)[start:end]
    torch.manual_seed(42 + layer_idx)
    k_mid = k_full[:, :, start:end, :]
    k = undo_rope(k_mid.float(), positions, inv_freq) if inv_freq is not None else k_mid.float()
    p_dim = nkv * hd
    flat = k.permute(0, 2, 1, 3).reshape(B * n_comp, p_dim)
    n = flat.shape[0]
    mean = flat.mean(dim=0)
    rank = min(max_rank, p_dim, n - 1)
    if svd is not None:
        S, V = (torch.as_tensor(t, dtype=torch.float32) for t in svd)
        basis = V[:, :rank]
        eig = (S[:rank].float() ** 2) / n
    elif basis is None:
        _, S, V = torch.svd_lowrank(flat - mean, q=rank, niter=24)
        basis = V[:, :rank]
        eig = (S[:rank].float() ** 2) / n
    else:
        basis = torch.as_tensor(basis, dtype=torch.float32)[:, :rank]
        eig = ((flat - mean) @ basis).pow(2).mean(dim=0)
    budget = max(64, int(p_dim * 16 / k_target_cr))
    alloc = dp_bit_allocation(eig, budget)
    keep = sum(1 for b in alloc if b > 0)
    if keep & 1:
        keep -= 1
    if keep > 0:
        basis = basis[:, :keep].contiguous()
        alloc = alloc[:keep]
    col_max = basis.abs().max(dim=0).values.clamp(min=1e-6)
    scale = col_max / 127.0
    basis_q = (basis / scale).round().clamp(-127, 127).to(torch.int8)
    if keep == 0:
        # every component dropped: _compress_k leaves basis and alloc whole and
        # projects onto none (cache.py:383-392); _build_gpu_format then stores
        # keep = len(k_alloc) columns of zero coefficients (cache.py:412-420),
        # kept even here as the device format stores ranks
        keep = len(alloc) - (len(alloc) & 1)
        basis_q, scale, alloc = basis_q[:, :keep], scale[:keep], alloc[:keep]
    proj = (flat - mean.float()) @ (basis_q.float() * scale.float())[:, :keep]
    chain = k_code_chain(proj.numpy(), alloc)

    v_mid = v_full[:, :, start:end, :]
    v_flat = v_mid.float().reshape(B * nkv, n_comp, hd)
    qd = vq_encode(hadamard(v_flat), group_size, codebook_size, assign=assign)

    k_scale_h = scale.half()
    gc = {
        "k_coeffs": torch.from_numpy(chain["packed"]),
        "k_coeff_scale": torch.from_numpy(chain["coeff_scale"]).half(),
        "k_coeffs_shape": (B * n_comp, keep),
        "k_basis_q": basis_q,
        "k_basis_scale": k_scale_h,
        "k_basis_f16": (basis_q.to(torch.float16) * k_scale_h.to(torch.float16)).contiguous(),
        "k_mean": mean.half(),
        "k_mean_f16": mean.half(),
        "v_qdata": qd,
        "v_idx_full": qd["idx"].view(B, nkv, n_comp, hd // group_size),
        "v_centroids_f16": qd["centroids"],
        "v_ch_f16": qd["ch_maxabs"].view(B, nkv, hd),
        "sink_k": k_full[:, :, :sink, :].clone(), "sink_v": v_full[:, :, :sink, :].clone(),
        "win_k": k_full[:, :, end:, :].clone(), "win_v": v_full[:, :, end:, :].clone(),
        "n_compress": n_comp, "batch": B, "compress_start": start,
        # intermediates
        "alloc": alloc, "proj": proj, "chain": chain, "basis": basis,
    }
    return gc


# --------------------------------------------------------------------------
# Attention: reference CPU fallback (attention.py:18-121, 270-343)
# --------------------------------------------------------------------------
def _unpack_int4_t(packed, n_total, rank):
    """attention.py:13-16."""
    lo = (packed & 0x0F).to(torch.float16) - 8.0
    hi = ((packed >> 4) & 0x0F).to(torch.float16) - 8.0
    return torch.stack([lo, hi], dim=1).flatten()[: n_total * rank].reshape(n_total, rank)


def compressed_scores(q_rope, gc, pos_q, n_q, nkv, hd, inv_freq):
    """attention.py:18-81, non-Triton branch (68-73).  (B, n_q, 1, n_comp)."""
    B = q_rope.shape[0]
    n_total, rank = gc["k_coeffs_shape"]
    n_comp = gc["n_compress"]
    gqa = n_q // nkv
    hd2 = hd // 2
    freqs = torch.tensor([pos_q]).float().unsqueeze(-1) * inv_freq.float()
    cos_q = torch.cat([freqs, freqs], dim=-1).cos().to(torch.float16).view(1, 1, 1, hd)
    sin_q = torch.cat([freqs, freqs], dim=-1).sin().to(torch.float16).view(1, 1, 1, hd)
    q_n = q_rope * cos_q - rotate_half(q_rope) * sin_q
    a, b = q_n[..., :hd2].contiguous(), q_n[..., hd2:].contiguous()
    k_basis = gc["k_basis_f16"]
    bph = k_basis.view(nkv, hd, rank)
    bc, bd = bph[:, :hd2, :], bph[:, hd2:, :]
    mean = gc["k_mean_f16"].view(nkv, hd)
    mc, md = mean[:, :hd2], mean[:, hd2:]
    kv_idx = torch.arange(n_q) // gqa
    bc, bd, mc, md = bc[kv_idx], bd[kv_idx], mc[kv_idx], md[kv_idx]
    coeff_scale = gc["k_coeff_scale"]
    bc_e, bd_e = bc.unsqueeze(0).unsqueeze(2), bd.unsqueeze(0).unsqueeze(2)
    A_mean = a * mc.unsqueeze(0).unsqueeze(2) + b * md.unsqueeze(0).unsqueeze(2)
    B_mean = b * mc.unsqueeze(0).unsqueeze(2) - a * md.unsqueeze(0).unsqueeze(2)
    A = (a.unsqueeze(-1) * bc_e + b.unsqueeze(-1) * bd_e) * coeff_scale
    Bm = (b.unsqueeze(-1) * bc_e - a.unsqueeze(-1) * bd_e) * coeff_scale
    coefs = _unpack_int4_t(gc["k_coeffs"], n_total, rank).view(B, n_comp, rank)
    U = torch.einsum("bhspr,bcr->bhspc", A, coefs) + A_mean.unsqueeze(-1)
    V = torch.einsum("bhspr,bcr->bhspc", Bm, coefs) + B_mean.unsqueeze(-1)
    pos_t = torch.arange(gc["compress_start"], gc["compress_start"] + n_comp)
    phase = (pos_t - pos_q).float().unsqueeze(-1) * inv_freq.float()
    cos_d = phase.cos().to(torch.float16)
    sin_d = phase.sin().to(torch.float16)
    scores = torch.einsum("bhspc,cp->bhsc", U, cos_d) + torch.einsum("bhspc,cp->bhsc", V, sin_d)
    return scores / math.sqrt(hd)


def v_weighted_sum_compressed(weights_mid, gc, B, nkv, n_comp, hd):
    """attention.py:114-121 (batched einsum fallback) -> hadamard in fp16."""
    gs = 4
    ng = hd // gs
    gqa = weights_mid.shape[1] // nkv
    idx_l = gc["v_idx_full"].reshape(B * nkv, n_comp, ng).long()
    centroids = gc["v_centroids_f16"]
    ch_max = gc["v_ch_f16"].reshape(B * nkv, hd)
    v_rot = centroids.float()[idx_l].view(B * nkv, n_comp, hd) * ch_max.float().unsqueeze(1)
    v_rot = v_rot.view(B, nkv, n_comp, hd).repeat_interleave(gqa, dim=1)
    out_rot = torch.einsum("bhsk,bhkd->bhsd", weights_mid, v_rot)
    return hadamard(out_rot.to(torch.float16)).float()


def stream_dequant(gc, B, nkv, hd):
    """cache.py:243-279: (B, nkv, S, hd) fp16 K and V, or (None, None); with the
    QJL term when the layer holds sign/scale buffers (cache.py:263-273)."""
    s = gc.get("stream_n", 0) // B if gc.get("stream_n", 0) else 0
    if s == 0:
        return None, None
    cb = gc["stream_codebook"]
    signs = gc["signs"]
    qjl = "k_qsign_buf" in gc

    def _q(key):
        return gc[key][:s] if qjl else None

    k = dequantize_stream_token(gc["k_idx_buf"][:s], gc["k_norm_buf"][:s], signs, cb,
                                _q("k_qsign_buf"), _q("k_qscale_buf"))
    v = dequantize_stream_token(gc["v_idx_buf"][:s], gc["v_norm_buf"][:s], signs, cb,
                                _q("v_qsign_buf"), _q("v_qscale_buf"))
    sk = torch.from_numpy(np.ascontiguousarray(np.transpose(k, (1, 2, 0, 3))))
    sv = torch.from_numpy(np.ascontiguousarray(np.transpose(v, (1, 2, 0, 3))))
    return sk, sv


def fused_attention_compressed(q_rope, gc, nkv, pos_q, inv_freq, attn_mask=None):
    """attention.py:270-343 on the CPU (non-Triton branches).  q_rope (B,n_q,1,hd) fp16."""
    B, n_q, _, hd = q_rope.shape
    n_comp = gc["n_compress"]
    gqa = n_q // nkv

    def _static_expanded(key):
        return gc[key].repeat_interleave(gqa, dim=1).float()

    def _score(q, k):
        return torch.einsum("bhsd,bhkd->bhsk", q.float(),
                            k.repeat_interleave(gqa, dim=1).float()) / math.sqrt(hd)

    comp_scores = compressed_scores(q_rope, gc, pos_q, n_q, nkv, hd, inv_freq).float()
    q_fp32 = q_rope.float()
    inv_sqrt_hd = 1.0 / math.sqrt(hd)

    def _score_expanded(k_exp):
        return torch.einsum("bhsd,bhkd->bhsk", q_fp32, k_exp) * inv_sqrt_hd

    stream = stream_dequant(gc, B, nkv, hd)
    if stream[0] is None:
        stream = None
    parts = [_score_expanded(_static_expanded("sink_k")), comp_scores,
             _score_expanded(_static_expanded("win_k"))]
    if "decode_k" in gc:
        parts.append(_score(q_rope, gc["decode_k"]))
    if stream is not None:
        parts.append(_score(q_rope, stream[0]))
    scores = torch.cat(parts, dim=-1)
    if attn_mask is not None:
        scores = scores + attn_mask
    weights = torch.softmax(scores, dim=-1, dtype=torch.float32)
    sink_n = gc["sink_k"].shape[2]
    win_n = gc["win_k"].shape[2]
    w_sink = weights[..., :sink_n]
    w_comp = weights[..., sink_n:sink_n + n_comp]
    w_win = weights[..., sink_n + n_comp:sink_n + n_comp + win_n]
    off = sink_n + n_comp + win_n
    out = v_weighted_sum_compressed(w_comp, gc, B, nkv, n_comp, hd)

    def _add_fp16(w, v):
        return torch.einsum("bhsk,bhkd->bhsd", w, v.repeat_interleave(gqa, dim=1).float())

    out = out + torch.einsum("bhsk,bhkd->bhsd", w_sink, _static_expanded("sink_v"))
    out = out + torch.einsum("bhsk,bhkd->bhsd", w_win, _static_expanded("win_v"))
    if "decode_v" in gc:
        dv = gc["decode_v"]
        out = out + _add_fp16(weights[..., off:off + dv.shape[2]], dv)
        off += dv.shape[2]
    if stream is not None:
        sv = stream[1]
        out = out + _add_fp16(weights[..., off:off + sv.shape[2]], sv)
    return out.to(q_rope.dtype)


def reconstruct_kv(gc, nkv, hd, inv_freq):
    """_ensure_dequant (cache.py:87-124): full fp16 K/V of the compressed segment
    (sink/window/stream concatenation excluded).  Returns (k_mid, v_mid) fp16
    (B, nkv, n_comp, hd)."""
    n_total, rank = gc["k_coeffs_shape"]
    packed = gc["k_coeffs"]
    coeffs = _unpack_int4_t(packed, n_total, rank) * gc["k_coeff_scale"].half()
    basis = gc["k_basis_q"].to(torch.float16) * gc["k_basis_scale"].half()
    recon = coeffs @ basis.T + gc["k_mean"].half()
    B, n_comp = gc["batch"], gc["n_compress"]
    k_layer = recon.view(B, n_comp, nkv, hd)
    if inv_freq is not None:
        pos = torch.arange(gc["compress_start"], gc["compress_start"] + n_comp)
        k_mid = reapply_rope(k_layer.permute(0, 2, 1, 3), pos, inv_freq).half()
    else:
        k_mid = k_layer.permute(0, 2, 1, 3).half()
    qd = gc["v_qdata"]
    v_mid = hadamard(vq_decode(qd)).view(B, nkv, n_comp, hd).half()
    return k_mid, v_mid
