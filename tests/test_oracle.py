"""Pins the CPU oracle (oracle/) against closed forms, library routines,
brute force and the golden vectors of tests/golden (reference outputs)."""
import itertools
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import exact, ref


# --------------------------------------------------------------------------
# Hadamard: Sylvester closed form, involution, torch/numpy agreement
# --------------------------------------------------------------------------
@pytest.mark.parametrize("d", [2, 4, 8, 16, 32, 64, 128])
def test_hadamard_matches_sylvester(d):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((5, d)).astype(np.float32)
    H = scipy.linalg.hadamard(d).astype(np.float64) / math.sqrt(d)
    want = x.astype(np.float64) @ H.T
    got = ref.hadamard(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6 * math.sqrt(d))
    np.testing.assert_allclose(exact.fwht64(x), want, rtol=0, atol=1e-12)


def test_hadamard_involution_and_np_bitexact():
    x = torch.randn(300, 128)
    y = ref.hadamard(x)
    np.testing.assert_allclose(ref.hadamard(y).numpy(), x.numpy(), atol=5e-6)
    assert np.array_equal(ref.hadamard_np(x.numpy()), y.numpy())


def test_sqrt_divisor_is_correctly_rounded():
    # fp32(double sqrt(d)) equals the correctly rounded fp32 sqrt for the dims used
    for d in (64, 128, 256):
        assert np.float32(math.sqrt(d)) == np.sqrt(np.float32(d))


# --------------------------------------------------------------------------
# RoPE: rotation closed form, undo o reapply = id
# --------------------------------------------------------------------------
def test_rope_rotation_closed_form():
    hd = 128
    inv = ref.default_inv_freq(500000.0, hd)
    pos = torch.arange(0, 50)
    x = torch.randn(1, 2, 50, hd, dtype=torch.float64).float()
    y = ref.reapply_rope(x, pos, inv)
    ph = (pos.float()[:, None] * inv[None, :]).double()
    c, s = ph.cos(), ph.sin()
    x1, x2 = x[..., :64].double(), x[..., 64:].double()
    want = torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)
    np.testing.assert_allclose(y.numpy(), want.numpy(), atol=2e-6)
    back = ref.undo_rope(y, pos, inv)
    np.testing.assert_allclose(back.numpy(), x.numpy(), atol=5e-6)


# --------------------------------------------------------------------------
# DP bit allocation: exhaustive enumeration
# --------------------------------------------------------------------------
@pytest.mark.parametrize("seed", range(6))
def test_dp_allocation_is_optimal(seed):
    rng = np.random.default_rng(seed)
    ng = int(rng.integers(1, 4))
    d = 64 * ng - int(rng.integers(0, 20))
    var = np.sort(rng.exponential(1.0, d))[::-1].astype(np.float32) * 10
    budget = int(rng.integers(64, 64 * 8 * ng))
    alloc = ref.dp_bit_allocation(torch.from_numpy(var.copy()), budget)
    sizes = [min(64, d - 64 * g) for g in range(ng)]
    gv = [float(torch.from_numpy(var[64 * g: 64 * g + sizes[g]].copy()).sum()) for g in range(ng)]
    units = budget // 16 + 1

    def err(bits):
        return sum(gv[g] * 4.0 if b == 0 else gv[g] / (3.0 * (1 << (2 * b))) for g, b in enumerate(bits))

    def cost(bits):
        return sum(0 if b == 0 else (sizes[g] * b + 15) // 16 for g, b in enumerate(bits))

    best = min(err(bits) for bits in itertools.product([0, 2, 4, 6, 8], repeat=ng)
               if cost(bits) <= units)
    got_bits = [alloc[64 * g] for g in range(ng)]
    assert all(alloc[64 * g + i] == got_bits[g] for g in range(ng) for i in range(sizes[g]))
    assert cost(got_bits) <= units
    assert err(got_bits) == pytest.approx(best, rel=1e-12)


# --------------------------------------------------------------------------
# Group quantizer + int4 chain: error bounds, ranges, packing relation
# --------------------------------------------------------------------------
def test_group_quant_error_bound():
    rng = np.random.default_rng(0)
    proj = (rng.standard_normal((777, 10)) * rng.uniform(0.1, 5, 10)).astype(np.float32)
    alloc = [8, 8, 6, 6, 4, 4, 2, 2, 0, 0]
    codes, lo, rng_ = ref.group_quant(proj, alloc)
    deq = ref.group_dequant(codes, lo, rng_, alloc)
    for c, b in enumerate(alloc):
        if b == 0:
            assert np.all(deq[:, c] == 0)
            continue
        L = (1 << b) - 1
        assert codes[:, c].max() <= L
        assert lo[c] == proj[:, c].min()
        assert codes[np.argmin(proj[:, c]), c] == 0 and codes[np.argmax(proj[:, c]), c] == L
        step = rng_[c] / L
        assert np.max(np.abs(deq[:, c] - proj[:, c])) <= step / 2 * (1 + 1e-4) + 1e-6


def test_int4_chain_matches_reference_golden(golden):
    """The whole K code chain against the reference's own quantize_group ->
    dequantize_group -> int4 -> int4_pack (tests/golden/int4_chain.npz): every
    intermediate bit for bit, on columns of all widths, including thousands of
    values on exact .5 boundaries in both rounding steps."""
    g = golden("int4_chain.npz")
    proj, alloc = g["proj"], [int(b) for b in g["alloc"]]
    ch = ref.k_code_chain(proj, alloc)
    for key, want in (("lo", g["lo"]), ("rng", g["rng"]), ("deq", g["deq"]), ("q", g["q"]),
                      ("coeff_scale", g["coeff_scale"]), ("packed", g["packed"])):
        assert ch[key].dtype == want.dtype or key in ("q",), key
        assert np.array_equal(ch[key], want), key
    # the fixture does exercise both tie rules: values on j + 0.5 exactly
    F = np.float32
    ties = 0
    for c, b in enumerate(alloc):
        if b:
            v = np.clip(((proj[:, c] - g["lo"][c]) / g["rng"][c]).astype(F), 0, 1)
            v = (v * F((1 << b) - 1)).astype(F)
            ties += int(np.sum(v - np.floor(v) == 0.5))
    r = (g["deq"] / g["coeff_scale"]).astype(F)
    assert ties > 1000 and int(np.sum(r - np.floor(r) == 0.5)) > 1000


def test_int4_chain_pack_relation_and_roundtrip():
    rng = np.random.default_rng(1)
    y = (rng.standard_normal((301, 12)) * rng.uniform(0.1, 3, 12)).astype(np.float32)
    q, cs = ref.int4_quantize(y)
    assert q.min() >= -7 and q.max() <= 7
    for c in range(y.shape[1]):
        assert np.abs(q[:, c]).max() == 7
        ok = np.abs(y[:, c] / cs[c]) <= 7
        assert np.all(np.abs(q[ok, c] * cs[c] - y[ok, c]) <= cs[c] / 2 * (1 + 1e-5))
    packed = ref.int4_pack(q)
    flat = (q.astype(np.int16) + 8).astype(np.uint8).reshape(-1)   # kernel_test.py:140-143
    if flat.size % 2:
        flat = np.concatenate([flat, np.zeros(1, np.uint8)])
    assert np.array_equal(packed, flat[0::2] | (flat[1::2] << 4))
    assert np.array_equal(ref.int4_unpack(packed, *q.shape), q)


# --------------------------------------------------------------------------
# Lloyd-Max codebook and the stream quantizer
# --------------------------------------------------------------------------
def test_lloyd_max_matches_reference_golden(golden):
    g = golden("lloyd_max.npz")
    cb = ref.lloyd_max_codebook(128, 8)
    assert cb.dtype == np.float32 and np.array_equal(cb, g["codebook"])


def test_lloyd_max_is_near_fixed_point():
    cb = ref.lloyd_max_codebook(128, 8).astype(np.float64)
    assert np.all(np.diff(cb) > 0)
    np.testing.assert_allclose(cb, -cb[::-1], atol=1e-7)          # symmetric
    # centroid condition E[X | cell] for N(0, 1/128) holds to ~1e-3 relative
    from scipy.stats import norm
    s = 1 / math.sqrt(128)
    b = np.concatenate([[-np.inf], (cb[1:] + cb[:-1]) / 2, [np.inf]]) / s
    m = norm.cdf(b[1:]) - norm.cdf(b[:-1])
    cond = (norm.pdf(b[:-1]) - norm.pdf(b[1:])) * s / m
    assert np.max(np.abs(cond - cb)[16:-16]) < 2e-3 * s


def test_norm_order_matches_torch():
    x = (torch.randn(20000, 128) * 4).half().float()
    assert np.array_equal(ref.norm_fp32_8lane(x.numpy()), x.norm(dim=-1).numpy())


def test_stream_quant_is_nearest_code():
    cb = ref.lloyd_max_codebook(128, 8)
    signs = ref.stream_signs(3, 128)
    x = (torch.randn(2000, 128) * 2).half().numpy()
    idx, nrm = ref.quantize_stream_token(x, signs, cb)
    t = x.astype(np.float64)
    n = np.maximum(np.sqrt((t * t).sum(-1)), 1e-8)
    import scipy.linalg as sl
    H = sl.hadamard(128) / math.sqrt(128)
    r = ((t / n[:, None]) * signs) @ H.T
    d = np.abs(r[..., None] - cb.astype(np.float64)[None, None, :])
    best = d.argmin(-1)
    srt = np.sort(d, axis=-1)
    clear = (srt[..., 1] - srt[..., 0]) > 1e-6
    assert np.array_equal(idx[clear], best[clear])
    np.testing.assert_allclose(nrm.astype(np.float64), n, rtol=1e-3)
    # dequantized tokens reproduce the inputs (tails beyond the last level clip)
    y = ref.dequantize_stream_token(idx, nrm, signs, cb).astype(np.float64)
    cos = (y * t).sum(-1) / (np.linalg.norm(y, axis=-1) * n)
    assert cos.mean() > 0.9999 and cos.min() > 0.99


@pytest.mark.parametrize("d", [64, 128, 256])
def test_mean_order_matches_torch(d):
    """The QJL scale is torch's CPU fp32 mean of |residual| (streaming.py:70)."""
    g = torch.Generator().manual_seed(d)
    x = torch.rand(20000, d, generator=g) * torch.exp(torch.randn(20000, 1, generator=g) * 3)
    x[:50] = torch.rand(50, d, generator=g) * 1e-3 + torch.arange(d) * 1e3   # wide spread
    assert np.array_equal(ref.mean_fp32_4x8(x.numpy()), x.mean(-1).numpy())


# Max (1960), Table 1: optimum output levels of the N(0, 1) quantizer (4 digits).
# The 1- and 2-bit iterations converge (break before 100 steps) to these.
_MAX_LEVELS = {1: [0.7979], 2: [0.4528, 1.510]}


@pytest.mark.parametrize("bits", [1, 2])
def test_lloyd_max_converged_widths_match_max_table(bits):
    cb = ref.lloyd_max_codebook(128, bits).astype(np.float64) * math.sqrt(128)
    half = np.array(_MAX_LEVELS[bits])
    np.testing.assert_allclose(cb, np.concatenate([-half[::-1], half]), atol=6e-4)
    if bits == 1:
        assert abs(cb[1] - math.sqrt(2 / math.pi)) < 1e-6      # E|X| closed form


@pytest.mark.parametrize("bits", [3, 4, 5, 6, 7])
def test_lloyd_max_widths_match_reference_golden(golden, bits):
    """Widths whose iteration stops at the 100-step cap: the reference's own output."""
    assert np.array_equal(ref.lloyd_max_codebook(128, bits), golden("lloyd_max_bits.npz")[f"cb{bits}"])


def _rotated64(x, signs):
    import scipy.linalg as sl
    t = x.astype(np.float64)
    n = np.maximum(np.sqrt((t * t).sum(-1)), 1e-8)
    H = sl.hadamard(x.shape[-1]) / math.sqrt(x.shape[-1])
    return ((t / n[:, None]) * signs) @ H.T, n


@pytest.mark.parametrize("bits", [8, 4, 2])
def test_stream_qjl_oracle(bits):
    """QJL fields (streaming.py:67-70, 77-78) against an fp64 restatement, and the
    exact per-token error identity ||r - cb - s m||^2 = ||r - cb||^2 - d m^2 for
    m = mean |r - cb| that makes the 1-bit term a strict improvement."""
    cb = ref.lloyd_max_codebook(128, bits)
    signs = ref.stream_signs(4, 128)
    x = (torch.randn(1500, 128, generator=torch.Generator().manual_seed(bits)) * 2).half().numpy()
    idx, nrm = ref.quantize_stream_token(x, signs, cb)
    idx2, nrm2, qs, qsc = ref.quantize_stream_token(x, signs, cb, qjl=True)
    assert np.array_equal(idx, idx2) and np.array_equal(nrm, nrm2)
    assert qs.dtype == np.uint8 and qsc.dtype == np.float16 and qsc.shape == nrm.shape
    r, n = _rotated64(x, signs)
    res = r - cb.astype(np.float64)[idx.astype(np.int64)]
    clear = np.abs(res) > 1e-6
    assert np.array_equal(qs[clear], (res >= 0)[clear])
    m = np.abs(res).mean(-1)
    np.testing.assert_allclose(qsc.astype(np.float64), m, rtol=1.2e-3)
    # the oracle's dequantization adds +-scale: output-domain error drops by ~d m^2 n^2
    y0 = ref.dequantize_stream_token(idx, nrm, signs, cb).astype(np.float64)
    y1 = ref.dequantize_stream_token(idx, nrm, signs, cb, qs, qsc).astype(np.float64)
    t = x.astype(np.float64)
    e0 = ((y0 - t) ** 2).sum(-1)
    e1 = ((y1 - t) ** 2).sum(-1)
    pred = e0 - 128 * (qsc.astype(np.float64) * n) ** 2
    fp16_noise = 128 * (np.abs(t).max(-1) * 2.0 ** -10) ** 2
    assert np.all(np.abs(e1 - pred) <= 0.02 * e0 + 4 * fp16_noise)
    assert e1.mean() < e0.mean() * (0.9 if bits <= 4 else 1.0)


# --------------------------------------------------------------------------
# VQ assignment and k-means
# --------------------------------------------------------------------------
def test_vq_assign_direct_matches_cdist_and_fp64():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(20000, 4, generator=g)
    c = torch.randn(256, 4, generator=g)
    direct = ref.vq_assign_direct(x.numpy(), c.numpy())
    cd = ref.vq_assign_cdist(x, c).numpy()
    d64 = ((x.double()[:, None, :] - c.double()[None]) ** 2).sum(-1).argmin(1).numpy()
    assert np.array_equal(direct, cd)
    assert np.array_equal(direct, d64)


def test_c_vq_assign_direct_equals_numpy():
    """oracle/cref.c restates ref.vq_assign_direct: same index on every row,
    including exact ties (duplicate centroids, midpoints), zero and NaN rows."""
    from oracle import cref
    if cref.load() is None:
        cref.build()
    rs = np.random.default_rng(3)
    c = rs.standard_normal((256, 4)).astype(np.float32)
    c[17] = c[200]
    c[31] = 0.0
    x = rs.standard_normal((30000, 4)).astype(np.float32)
    x[:64] = (c[rs.integers(0, 256, 64)] + c[rs.integers(0, 256, 64)]) / 2
    x[64:80] = c[200]
    x[80:90] = 0.0
    x[90:95] = np.nan
    assert np.array_equal(cref.vq_assign_direct(x, c), ref.vq_assign_direct(x, c))


def test_kmeans_matches_reference_golden(golden):
    g = golden("kmeans.npz")
    cent, idx = ref.kmeans(torch.from_numpy(g["data"]), int(g["k"]), int(g["n_iter"]), int(g["seed"]))
    assert np.array_equal(cent.numpy(), g["centroids"])
    assert np.array_equal(idx.numpy(), g["idx"])


def test_kmeans_direct_assign_equals_cdist_assign(golden):
    g = golden("kmeans.npz")
    data = torch.from_numpy(g["data"])
    direct = lambda x, c: torch.from_numpy(ref.vq_assign_direct(x.numpy(), c.numpy()))
    c1, i1 = ref.kmeans(data, 16, 30, 42, assign=direct)
    assert np.array_equal(c1.numpy(), g["centroids"]) and np.array_equal(i1.numpy(), g["idx"])


# --------------------------------------------------------------------------
# Attention: relative-delta identity and the reference's fused path
# --------------------------------------------------------------------------
def _gc_from_fixture(f):
    rank, n_comp, start = int(f["rank"]), int(f["n_comp"]), int(f["start"])
    nkv = f["sink_k"].shape[1]
    basis_q = torch.from_numpy(f["k_basis_q"])
    bs = torch.from_numpy(f["k_basis_scale"])
    idx = torch.from_numpy(f["v_idx"])
    gc = {
        "k_coeffs": torch.from_numpy(f["k_coeffs"]), "k_coeffs_shape": (n_comp, rank),
        "k_coeff_scale": torch.from_numpy(f["k_coeff_scale"]),
        "k_basis_q": basis_q, "k_basis_scale": bs,
        "k_basis_f16": (basis_q.to(torch.float16) * bs.to(torch.float16)).contiguous(),
        "k_mean": torch.from_numpy(f["k_mean"]), "k_mean_f16": torch.from_numpy(f["k_mean"]),
        "v_qdata": {"centroids": torch.from_numpy(f["centroids"]), "idx": idx,
                    "ch_maxabs": torch.from_numpy(f["ch"]), "shape": (nkv, n_comp, 128),
                    "group_size": 4},
        "v_idx_full": idx.view(1, nkv, n_comp, 32),
        "v_centroids_f16": torch.from_numpy(f["centroids"]),
        "v_ch_f16": torch.from_numpy(f["ch"]).view(1, nkv, 128),
        "sink_k": torch.from_numpy(f["sink_k"]), "sink_v": torch.from_numpy(f["sink_v"]),
        "win_k": torch.from_numpy(f["win_k"]), "win_v": torch.from_numpy(f["win_v"]),
        "n_compress": n_comp, "batch": 1, "compress_start": start,
        "signs": f["signs"], "stream_codebook": ref.lloyd_max_codebook(128, 8),
        "stream_n": f["s_kidx"].shape[0],
        "k_idx_buf": f["s_kidx"], "v_idx_buf": f["s_vidx"],
        "k_norm_buf": f["s_knorm"], "v_norm_buf": f["s_vnorm"],
    }
    return gc, nkv


def test_reference_fused_path_matches_golden(golden):
    f = golden("fused_attn.npz")
    gc, nkv = _gc_from_fixture(f)
    out = ref.fused_attention_compressed(torch.from_numpy(f["q_rope"]), gc, nkv, int(f["pos_q"]),
                                         torch.from_numpy(f["inv_freq"]))
    assert np.array_equal(out.numpy(), f["out"])


def test_exact_oracle_close_to_reference_fused_path(golden):
    f = golden("fused_attn.npz")
    gc, nkv = _gc_from_fixture(f)
    out = exact.decode_attention(f["q_rope"], gc, nkv, int(f["pos_q"]), f["inv_freq"])
    g = f["out"].astype(np.float64)
    assert np.max(np.abs(out - g)) < 5e-3          # the reference's fp16 intermediates
    cos = (out * g).sum() / (np.linalg.norm(out) * np.linalg.norm(g))
    assert cos > 0.9999


def test_relative_delta_identity_against_reapplied_rope(golden):
    """exact.decode_attention's compressed scores equal q_rope . RoPE(k_n, pos_t)
    computed by brute force (reconstruct, reapply RoPE, dot)."""
    f = golden("fused_attn.npz")
    gc, nkv = _gc_from_fixture(f)
    q = f["q_rope"].astype(np.float64)
    pos_q = int(f["pos_q"])
    inv = f["inv_freq"]
    _, parts = exact.decode_attention(q, gc, nkv, pos_q, inv, return_parts=True)
    kn = exact.keys_norope(gc, nkv, 128)                      # (1, nkv, n, 128)
    n = gc["n_compress"]
    pos = np.arange(gc["compress_start"], gc["compress_start"] + n)
    ph = (pos[:, None] * inv[None, :].astype(np.float64))
    c, s = np.cos(ph), np.sin(ph)
    k1, k2 = kn[..., :64], kn[..., 64:]
    krope = np.concatenate([k1 * c - k2 * s, k2 * c + k1 * s], -1)
    krope = np.repeat(krope, 4, axis=1)
    qph = pos_q * inv.astype(np.float64)
    brute = np.einsum("bhd,bhkd->bhk", q[:, :, 0], krope) / math.sqrt(128)
    got = parts["scores"][..., 4:4 + n]
    np.testing.assert_allclose(got, brute, atol=1e-4)
    # a wrong sign of the sin term would break the identity
    bad = np.concatenate([k1 * c + k2 * s, k2 * c - k1 * s], -1)
    bad = np.einsum("bhd,bhkd->bhk", q[:, :, 0], np.repeat(bad, 4, axis=1)) / math.sqrt(128)
    assert np.max(np.abs(bad - got)) > 1e-2
    del qph


def test_batch_rows_slice_matches_full_oracle():
    """tests.helpers.batch_rows: the oracle on a subset of batch rows (in any
    order) equals those rows of the oracle on the whole layer, fp16 segments
    and decode tokens included; a slice that swapped per-row data would not."""
    from tests.helpers import batch_rows, random_layer
    gc, inv = random_layer(B=4, n_comp=300, n_dec=3, seed=5)
    q = torch.randn(4, 32, 1, 128, generator=torch.Generator().manual_seed(4)).half()
    pos_q = 4 + 300 + 64 + 3 - 1
    full = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
    part = exact.decode_attention(q[[3, 1]].numpy(), batch_rows(gc, [3, 1]), 8, pos_q, inv.numpy())
    np.testing.assert_array_equal(part, full[[3, 1]])
    swapped = exact.decode_attention(q[[3, 1]].numpy(), batch_rows(gc, [1, 3]), 8, pos_q, inv.numpy())
    assert np.max(np.abs(swapped - full[[3, 1]])) > 1e-2


# --------------------------------------------------------------------------
# Composites: one layer of Cache.compress and _ensure_dequant (reference
# outputs of tests/golden/compress.npz and ensure_dequant.npz)
# --------------------------------------------------------------------------
def _compress_golden(golden):
    g = golden("compress.npz")
    gc = ref.compress_layer(torch.from_numpy(g["k_full"]), torch.from_numpy(g["v_full"]), 0,
                            torch.from_numpy(g["inv_freq"]), sink=int(g["sink"]), win=int(g["win"]),
                            k_target_cr=float(g["k_target_cr"]), max_rank=int(g["max_rank"]),
                            svd=(g["svd_S"], g["svd_V"]))
    return g, gc


def test_compress_layer_matches_reference_golden(golden):
    """oracle.ref.compress_layer reproduces the reference's _compress_k +
    _compress_v + _build_gpu_format bit for bit (svd_lowrank stubbed to the
    same fixed (S, V) on both sides): int8 basis and scales, mean, the DP
    allocation, the group codes' (lo, rng), the dequantized coefficients, the
    int4 codes and their packing, the V codebook, indices and channel scales."""
    g, gc = _compress_golden(golden)
    assert gc["alloc"] == list(g["alloc"])
    assert np.array_equal(gc["k_basis_q"].numpy(), g["k_basis_q"])
    assert np.array_equal(gc["k_basis_scale"].numpy(), g["k_scale"])
    assert np.array_equal(gc["k_mean"].numpy(), g["k_mean"])
    assert np.array_equal(gc["k_basis_f16"].numpy(), g["k_basis_f16"])
    ch = gc["chain"]
    assert np.array_equal(ch["lo"], g["lo"]) and np.array_equal(ch["rng"], g["rng"])
    assert np.array_equal(ch["deq"], g["deq"])
    assert np.array_equal(ch["q"], g["q"])
    assert np.array_equal(ch["coeff_scale"], g["coeff_scale"])
    assert np.array_equal(gc["k_coeffs"].numpy(), g["k_coeffs"])
    assert np.array_equal(gc["v_centroids_f16"].numpy(), g["centroids"])
    assert np.array_equal(gc["v_qdata"]["idx"].numpy(), g["v_packed"])
    assert np.array_equal(gc["v_qdata"]["ch_maxabs"].numpy(), g["ch_maxabs"])
    # the reference's on-device V index view keeps batch row 0 (cache.py:426-427);
    # the batch-major layout's row 0 is that view
    assert np.array_equal(gc["v_idx_full"][0].numpy(), g["v_indices_row0"])


def test_compress_golden_is_sensitive_to_layout():
    """A flatten order with heads and tokens swapped, or no centring, changes
    the reference's codes: the golden pins the stitching, not only the leaves."""
    import os
    from tests.conftest import GOLDEN
    g = np.load(os.path.join(GOLDEN, "compress.npz"))
    k = torch.from_numpy(g["k_full"])
    swapped = k.view(2, 2, 200, 128).permute(0, 2, 1, 3).reshape(2, 2, 200, 128)  # heads <-> tokens mixed
    gc = ref.compress_layer(swapped.contiguous(), torch.from_numpy(g["v_full"]), 0,
                            torch.from_numpy(g["inv_freq"]), k_target_cr=float(g["k_target_cr"]),
                            max_rank=int(g["max_rank"]), svd=(g["svd_S"], g["svd_V"]))
    assert not np.array_equal(gc["k_coeffs"].numpy(), g["k_coeffs"])
    assert not np.array_equal(gc["k_mean"].numpy(), g["k_mean"])


def test_compress_with_every_component_dropped_decodes_to_the_mean():
    """A 64-dim K (one kv head of 64 dims): the budget max(64, 64*16/20) = 64
    bits is 5 units, below the cheapest option of a 64-component group (2 bits
    = 8 units), so the DP drops every component.  _compress_k then keeps basis
    and allocation whole and _build_gpu_format stores them with zero
    coefficients (cache.py:383-392, 412-420): every int4 code is 0 (nibble 8),
    each coefficient scale is max(0, 1e-6) / 7, and the rebuilt keys are the
    mean exactly."""
    g = torch.Generator().manual_seed(3)
    k = torch.randn(1, 1, 300, 64, generator=g).half()
    v = torch.randn(1, 1, 300, 64, generator=g).half()
    inv = ref.default_inv_freq(10000.0, 64)
    gc = ref.compress_layer(k, v, 0, inv, k_target_cr=20.0, max_rank=192)
    n = 300 - 4 - 64
    assert gc["k_coeffs_shape"] == (n, 64)
    assert gc["alloc"] == [0] * 64
    assert np.all(gc["k_coeffs"].numpy() == 0x88)
    assert np.all(gc["k_coeff_scale"].numpy() == np.float16(np.float32(1e-6) / np.float32(7)))
    kn = exact.keys_norope(gc, 1, 64)
    assert np.array_equal(kn[0, 0], np.broadcast_to(gc["k_mean_f16"].numpy().astype(np.float64), (n, 64)))


def _ensure_dequant_gc(f):
    B, rank, n_comp, start = int(f["batch"]), int(f["rank"]), int(f["n_comp"]), int(f["start"])
    nkv = f["sink_k"].shape[1]
    return {
        "k_coeffs": torch.from_numpy(f["k_coeffs"]), "k_coeffs_shape": (B * n_comp, rank),
        "k_coeff_scale": torch.from_numpy(f["k_coeff_scale"]),
        "k_basis_q": torch.from_numpy(f["k_basis_q"]),
        "k_basis_scale": torch.from_numpy(f["k_basis_scale"]),
        "k_mean": torch.from_numpy(f["k_mean"]),
        "v_qdata": {"centroids": torch.from_numpy(f["centroids"]), "idx": torch.from_numpy(f["v_idx"]),
                    "ch_maxabs": torch.from_numpy(f["ch"]), "shape": (B * nkv, n_comp, 128),
                    "group_size": 4},
        "n_compress": n_comp, "batch": B, "compress_start": start,
    }, nkv


def test_vq_decode_matches_reference_golden(golden):
    f = golden("ensure_dequant.npz")
    gc, _ = _ensure_dequant_gc(f)
    assert np.array_equal(ref.vq_decode(gc["v_qdata"]).numpy(), f["vq_decoded"])


def test_reconstruct_kv_matches_reference_golden(golden):
    """oracle.ref.reconstruct_kv is the compressed segment of the reference's
    _ensure_dequant output (batch 2: the view(B, n, nkv, hd).permute order),
    bit for bit; the stream and decode tokens of the same golden are the
    oracle's stream dequantization and the stored fp16 rows."""
    f = golden("ensure_dequant.npz")
    gc, nkv = _ensure_dequant_gc(f)
    k_mid, v_mid = ref.reconstruct_kv(gc, nkv, 128, torch.from_numpy(f["inv_freq"]))
    sink, n = f["sink_k"].shape[2], int(f["n_comp"])
    keys, values = f["keys"], f["values"]
    assert np.array_equal(k_mid.numpy(), keys[:, :, sink:sink + n])
    assert np.array_equal(v_mid.numpy(), values[:, :, sink:sink + n])
    win = f["win_k"].shape[2]
    assert np.array_equal(keys[:, :, :sink], f["sink_k"])
    assert np.array_equal(keys[:, :, sink + n:sink + n + win], f["win_k"])
    s = f["s_kidx"].shape[0]
    cb = ref.lloyd_max_codebook(128, 8)
    sk = ref.dequantize_stream_token(f["s_kidx"], f["s_knorm"], f["signs"], cb)
    sv = ref.dequantize_stream_token(f["s_vidx"], f["s_vnorm"], f["signs"], cb)
    off = sink + n + win
    assert np.array_equal(keys[:, :, off:off + s], np.transpose(sk, (1, 2, 0, 3)))
    assert np.array_equal(values[:, :, off:off + s], np.transpose(sv, (1, 2, 0, 3)))
    assert np.array_equal(keys[:, :, off + s:], f["decode_k"])
    assert np.array_equal(values[:, :, off + s:], f["decode_v"])
