"""The product compression (shard_amd.cache.compress_layer, HIP kernels) against
the oracle's restatement of the reference's _compress_k / _compress_v /
_build_gpu_format (oracle.ref.compress_layer, cache.py:338-460) on one
Llama-3.1-8B-shaped layer: 2048 tokens of the seeded synthetic K/V, one PCA basis
supplied to both (the reference's svd_lowrank is randomized).

What must agree:
  * V: channel scales, k-means centroids (fp16) and VQ indices bit for bit;
    the oracle's k-means uses the reference GPU kernel's nearest-centroid rule
    (direct fp32 sum of squared differences, first index on ties), restated in
    oracle/cref.c.
  * K: the int4 chain bit for bit given the product's own projection, and the
    packed codes against the oracle's fp32 projection at a measured agreement
    rate (the product projects with fp16 MFMA operands and an fp32 sum, the
    reference in fp32, so a code can flip where the value sits on a rounding
    boundary).
"""
import numpy as np
import pytest
import torch

from oracle import cref, ref

pytestmark = pytest.mark.gpu

# Share of int4 codes equal to the fp32-projection oracle's at this config:
# 0.99955 measured on MI355X; asserted with margin.
K_CODE_AGREEMENT_FLOOR = 0.999


@pytest.fixture(scope="module")
def config1(cuda):
    from shard_amd import bench_data
    from shard_amd.cache import Cache, compress_layer, pca_basis
    k, v = bench_data.make_kv(2048)
    inv = bench_data.inv_freq()
    cache = Cache(head_dim=128, num_layers=1, n_kv_heads=8, device="cuda", rope_inv_freq=inv)
    # a realistic basis: the product's own PCA of this layer, handed to both sides
    sink, win = cache._sink_tokens, cache._residual_window
    k_mid = ref.undo_rope(k[:, :, sink:2048 - win, :].float(), torch.arange(sink, 2048 - win), inv)
    flat = k_mid.permute(0, 2, 1, 3).reshape(-1, 1024)
    basis, _ = pca_basis((flat - flat.mean(0)).to(cuda), 192)
    basis = basis.cpu()
    dbg = {}
    print("[compress config1] product compress_layer", flush=True)
    got = compress_layer(cache, k.to(cuda), v.to(cuda), 0, basis=basis.to(cuda), debug=dbg)
    torch.cuda.synchronize()
    print("[compress config1] oracle compress_layer", flush=True)
    want = ref.compress_layer(k, v, 0, inv, basis=basis, assign=cref.vq_assign_direct_t)
    return got, want, dbg


def test_compress_v_bitexact(config1):
    got, want, _ = config1
    assert torch.equal(got["v_ch_f16"].cpu().view(-1, 128).view(torch.int16),
                       want["v_qdata"]["ch_maxabs"].view(-1, 128).view(torch.int16))
    assert torch.equal(got["v_centroids_f16"].cpu().view(torch.int16),
                       want["v_centroids_f16"].view(torch.int16))
    gi = got["v_indices"].cpu().reshape(-1)
    wi = want["v_idx_full"].reshape(-1)
    assert torch.equal(gi, wi), f"{int((gi != wi).sum())} of {gi.numel()} VQ indices differ"


def test_compress_k_chain_bitexact_given_projection(config1):
    got, want, dbg = config1
    assert dbg["alloc"] == list(want["alloc"])
    chain = ref.k_code_chain(dbg["proj"].cpu().numpy(), dbg["alloc"])
    assert np.array_equal(got["k_coeffs"].cpu().numpy(), chain["packed"])
    assert np.array_equal(got["k_coeff_scale"].cpu().numpy(),
                          chain["coeff_scale"].astype(np.float16))
    assert torch.equal(got["k_basis_q"].cpu(), want["k_basis_q"])
    assert torch.equal(got["k_basis_f16"].cpu().view(torch.int16),
                       want["k_basis_f16"].view(torch.int16))


def test_compress_k_codes_agree_with_fp32_projection(config1):
    got, want, dbg = config1
    n, keep = got["k_coeffs_shape"]
    gq = ref.int4_unpack(got["k_coeffs"].cpu().numpy(), n, keep)
    wq = ref.int4_unpack(want["k_coeffs"].numpy(), n, keep)
    agree = float(np.mean(gq == wq))
    # where they differ, the cause is the first rounding step: the group codes
    # (2-8 bit levels of each column) differ by one level at most; one level of
    # a 2-bit column moves the int4 code by several steps
    g_codes = ref.k_code_chain(dbg["proj"].cpu().numpy(), dbg["alloc"])["codes"].astype(np.int32)
    w_codes = want["chain"]["codes"].astype(np.int32)
    code_step = int(np.abs(g_codes - w_codes).max())
    proj_err = float((dbg["proj"].cpu() - want["proj"]).abs().max())
    mean_ulps = np.abs(got["k_mean_f16"].cpu().view(torch.int16).numpy().astype(np.int32)
                       - want["k_mean_f16"].view(torch.int16).numpy().astype(np.int32)).max()
    print(f"[compress config1] int4 code agreement {agree:.6f}, group codes "
          f"{float(np.mean(g_codes == w_codes)):.6f} (max level step {code_step}), "
          f"max |proj - proj_fp32| {proj_err:.3e}, k_mean max ulp diff {mean_ulps}", flush=True)
    assert agree >= K_CODE_AGREEMENT_FLOOR
    assert code_step <= 1
    assert mean_ulps <= 1
