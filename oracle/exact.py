"""fp64 evaluation of decode attention over the dequantized representation.

This is the accuracy yardstick for attention outputs ("the reference
fp32-accumulated result"): the reference fused path's math (attention.py:18-343)
evaluated with every intermediate in float64 instead of the reference's fp16
intermediates.  Stored values enter exactly as the reference holds them:

  compressed K   k_n(t) = sum_r (nib_tr - 8) * cs_r * basis_f16[:, r] + mean_f16
                 (cs = fp16 k_coeff_scale; attention.py:13-16, 35-47, 69-73)
  scores         q_n = undo-RoPE(q_rope, pos_q) with fp32 phase fl(pos_q*theta);
                 s = sum_i (a c + b d) cos(phi) + (b c - a d) sin(phi),
                 phi = fl32(fl32(pos_t - pos_q) * theta_i)   (attention.py:3-6, 27-31, 75-81)
  compressed V   FWHT(cb[idx] * ch)                     (attention.py:83-121)
  fp16 segments  sink / window / decode K,V as stored   (attention.py:280-342)
  stream         H(cb_LM[idx] (+ QJL)) * signs * norm_f16 (streaming.py:74-79, exact)
  softmax        over [sink, comp, win, decode, stream] (+ additive mask)

Pinned by: the relative-delta identity against brute-force
reconstruct -> reapply RoPE -> dot (tests/test_oracle.py), and the
Sylvester-matrix Hadamard.
"""
import math

import numpy as np

F64 = np.float64


def fwht64(x: np.ndarray) -> np.ndarray:
    """Orthonormal Walsh-Hadamard (Sylvester order) in fp64 on the last dim."""
    x = np.asarray(x, F64).copy()
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
    return x / math.sqrt(d)


def unpack_coeffs(packed, n_total, rank):
    p = np.asarray(packed, np.uint8)
    lo = (p & 0x0F).astype(np.int64) - 8
    hi = ((p >> 4) & 0x0F).astype(np.int64) - 8
    return np.stack([lo, hi], axis=1).reshape(-1)[: n_total * rank].reshape(n_total, rank)


def keys_norope(gc, nkv, hd):
    """(B, nkv, n_comp, hd) fp64 no-RoPE compressed keys."""
    n_total, rank = gc["k_coeffs_shape"]
    B, n_comp = gc["batch"], gc["n_compress"]
    coef = unpack_coeffs(_np(gc["k_coeffs"]), n_total, rank).astype(F64)
    cs = _np(gc["k_coeff_scale"]).astype(F64)
    basis = _np(gc["k_basis_f16"]).astype(F64)          # (nkv*hd, rank)
    mean = _np(gc["k_mean_f16"]).astype(F64)
    kn = (coef * cs[None, :]) @ basis.T + mean[None, :]   # (B*n_comp, nkv*hd)
    return kn.reshape(B, n_comp, nkv, hd).transpose(0, 2, 1, 3)


def values_comp(gc, nkv, hd):
    """(B, nkv, n_comp, hd) fp64 compressed values FWHT(cb[idx]*ch)."""
    B, n_comp = gc["batch"], gc["n_compress"]
    cb = _np(gc["v_centroids_f16"]).astype(F64)   # (codebook rows, subvector size)
    idx = _np(gc["v_idx_full"]).astype(np.int64).reshape(B, nkv, n_comp, hd // cb.shape[1])
    ch = _np(gc["v_ch_f16"]).astype(F64).reshape(B, nkv, hd)
    v_rot = cb[idx].reshape(B, nkv, n_comp, hd) * ch[:, :, None, :]
    return fwht64(v_rot)


def stream_kv(gc, B, nkv, hd):
    s = gc.get("stream_n", 0) // B if gc.get("stream_n", 0) else 0
    if s == 0:
        return None, None
    cb = np.asarray(gc["stream_codebook"], F64)
    signs = np.asarray(gc["signs"], F64)

    qjl = "k_qsign_buf" in gc

    def deq(p):
        rot = cb[np.asarray(gc[p + "_idx_buf"][:s]).astype(np.int64)]
        if qjl:   # streaming.py:77-78: + (2 sign - 1) * scale in the rotated domain
            sgn = np.asarray(gc[p + "_qsign_buf"][:s]).astype(F64) * 2 - 1
            rot = rot + sgn * np.asarray(gc[p + "_qscale_buf"][:s], np.float16).astype(F64)[..., None]
        u = fwht64(rot) * signs
        return u * np.asarray(gc[p + "_norm_buf"][:s], np.float16).astype(F64)[..., None]

    k = deq("k")    # (s, B, nkv, hd)
    v = deq("v")
    return k.transpose(1, 2, 0, 3), v.transpose(1, 2, 0, 3)


def _np(t):
    try:
        import torch
        if isinstance(t, torch.Tensor):
            return t.detach().cpu().numpy()
    except ImportError:  # pragma: no cover
        pass
    return np.asarray(t)


def decode_attention(q_rope, gc, nkv, pos_q, inv_freq, attn_mask=None, return_parts=False):
    """fp64 decode attention; q_rope (B, n_q, 1, hd) (any float dtype)."""
    q = _np(q_rope).astype(F64)
    B, n_q, _, hd = q.shape
    hd2 = hd // 2
    gqa = n_q // nkv
    theta32 = _np(inv_freq).astype(np.float32)
    n_comp = gc["n_compress"]
    start = gc["compress_start"]

    # q_n = undo-RoPE(q_rope, pos_q) with the fp32 phase fl(pos_q * theta)
    ph_q = (np.float32(pos_q) * theta32).astype(np.float32).astype(F64)
    cq, sq = np.cos(ph_q), np.sin(ph_q)
    qlo, qhi = q[..., :hd2], q[..., hd2:]
    a = qlo * cq + qhi * sq
    b = qhi * cq - qlo * sq

    kn = keys_norope(gc, nkv, hd)                        # (B, nkv, n, hd)
    delta = (np.arange(start, start + n_comp) - pos_q).astype(np.float32)
    phi = (delta[:, None] * theta32[None, :]).astype(np.float32).astype(F64)   # (n, hd2)
    cos_p, sin_p = np.cos(phi), np.sin(phi)
    s_comp = np.empty((B, n_q, n_comp), F64)
    for g in range(nkv):                                 # one kv head at a time (memory)
        c, d = kn[:, g, :, :hd2], kn[:, g, :, hd2:]      # (B, n, hd2)
        # rotate the key pairs by phi, then dot with q_n of the GQA group
        cr = c * cos_p - d * sin_p
        dr = d * cos_p + c * sin_p
        for h in range(g * gqa, (g + 1) * gqa):
            s_comp[:, h, :] = (np.einsum("bi,bni->bn", a[:, h, 0, :], cr)
                               + np.einsum("bi,bni->bn", b[:, h, 0, :], dr)) / math.sqrt(hd)

    def dot(kseg):
        k = np.repeat(_np(kseg).astype(F64), gqa, axis=1)
        return np.einsum("bhd,bhkd->bhk", q[:, :, 0, :], k) / math.sqrt(hd)

    segs_s = [dot(gc["sink_k"]), s_comp, dot(gc["win_k"])]
    segs_v = [_np(gc["sink_v"]).astype(F64), values_comp(gc, nkv, hd), _np(gc["win_v"]).astype(F64)]
    if "decode_k" in gc:
        segs_s.append(dot(gc["decode_k"]))
        segs_v.append(_np(gc["decode_v"]).astype(F64))
    sk, sv = stream_kv(gc, B, nkv, hd)
    if sk is not None:
        segs_s.append(dot(sk))
        segs_v.append(sv)
    s = np.concatenate(segs_s, axis=-1)
    if attn_mask is not None:
        s = s + _np(attn_mask).astype(F64).reshape(B, -1)[:, None, :]
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    w = p / p.sum(-1, keepdims=True)
    out = np.zeros((B, n_q, hd), F64)
    off = 0
    for v in segs_v:                                     # (B, nkv, n_seg, hd)
        n_seg = v.shape[2]
        ws = w[:, :, off:off + n_seg].reshape(B, nkv, gqa, n_seg)
        out += np.einsum("bgqk,bgkd->bgqd", ws, v).reshape(B, n_q, hd)
        off += n_seg
    out = out[:, :, None, :]
    if return_parts:
        return out, {"scores": s, "weights": w}
    return out
