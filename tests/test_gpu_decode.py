"""GPU parity of the fused decode-attention kernel.

Bar (from the north star): max-abs-err <= 2e-3 and cosine >= 0.9999 against the
fp64 evaluation of the reference's math over the same stored representation
(oracle/exact.py).  Inputs are built on the CPU (seeded) and uploaded, so the
kernel and the oracle see identical bits."""
import numpy as np
import pytest
import torch

from oracle import exact, ref
from tests.helpers import batch_rows, compare, random_layer, to_device

pytestmark = pytest.mark.gpu

TOL_ABS = 2e-3
TOL_COS = 0.9999


def _run(cuda, gc, inv, q, pos_q, mask=None, n_splits=0, nkv=8, kernel=0, hd=128):
    from shard_amd import ops
    d = to_device(gc, cuda, inv, nkv=nkv, hd=hd)
    B = gc["batch"]
    stream_n = gc.get("stream_n", 0) // B
    dec = (d["decode_k"], d["decode_v"]) if "decode_k" in d else None
    m = None if mask is None else torch.from_numpy(mask).to(cuda)
    call = ops.make_decode_args(q.to(cuda).reshape(B, -1, hd), d, pos_q, None, mask=m,
                                n_splits=n_splits, stream_n=stream_n, decode_kv=dec)
    call.args.kernel = kernel
    out = ops.decode_attn(call)
    torch.cuda.synchronize()
    return out.cpu().float().numpy().reshape(B, -1, 1, hd)


CASES = [
    # (B, nkv, rank, n_comp, sink, win, n_stream, n_dec)
    (1, 8, 192, 1980, 4, 64, 0, 0),      # config-1 shape (T = 2048)
    (1, 8, 192, 8124, 4, 64, 0, 0),      # config-2 shape (T = 8192)
    (1, 8, 192, 1980, 4, 64, 37, 0),     # with an 8-bit stream
    (1, 8, 128, 517, 4, 64, 0, 5),       # fp16 decode tokens, rank 128, ragged tile
    (2, 8, 192, 300, 4, 64, 3, 0),       # batch 2
    (1, 2, 64, 33, 2, 3, 1, 0),          # tiny, 2 kv heads
    (1, 8, 96, 1, 4, 64, 0, 0),          # a single compressed token
    (4, 8, 192, 1100, 4, 64, 2, 0),      # batch 4
    (8, 8, 192, 400, 4, 64, 2, 0),       # batch 8 (the merge's 2-slice grid)
    (16, 8, 128, 300, 4, 16, 1, 0),      # batch 16
    (1, 8, 192, 700, 4, 64, 3000, 0),    # 3,068 extra tokens: spread over many splits
    (2, 4, 160, 900, 4, 64, 700, 9),     # long stream and decode tokens together
    (1, 8, 192, 600, 0, 0, 0, 0),        # no sink, window or stream: compressed tokens alone
    # row-split launches of 512 workgroups in two classes with every split of a
    # (batch row, kv head) group on one XCD and its merge there too
    (2, 4, 192, 4200, 4, 64, 0, 0),      # 8 groups, 64 splits each
    (2, 8, 192, 2100, 4, 64, 2, 0),      # 16 groups, 32 splits each
    (1, 16, 128, 2100, 4, 64, 0, 0),     # 16 kv heads, 32 splits each
]

# split kernels: 0 = automatic, 1 = row-split, 2 = token-tiled
KERNELS = [0, 1, 2]


def _kernels_for(n_x):
    # the earlier split kernels take at most 2048 extra tokens
    return [k for k in KERNELS if k != 1 or n_x <= 2048]


@pytest.mark.parametrize("case", CASES, ids=[str(c) for c in CASES])
def test_decode_matches_exact_oracle(cuda, case):
    B, nkv, rank, n_comp, sink, win, n_stream, n_dec = case
    gc, inv = random_layer(B=B, nkv=nkv, rank=rank, n_comp=n_comp, sink=sink, win=win,
                           n_stream=n_stream, n_dec=n_dec, seed=n_comp + rank)
    g = torch.Generator().manual_seed(1)
    q = torch.randn(B, 4 * nkv, 1, 128, generator=g).half()
    pos_q = sink + n_comp + win + n_dec + n_stream - 1
    want = exact.decode_attention(q.numpy(), gc, nkv, pos_q, inv.numpy())
    for kernel in _kernels_for(sink + win + n_stream + n_dec):
        got = _run(cuda, gc, inv, q, pos_q, nkv=nkv, kernel=kernel)
        err, cos = compare(got, want)
        print(f"case={case} kernel={kernel} max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS, (kernel, err, cos)


GQA_CASES = [
    # (B, nkv, query heads per kv head, rank, n_comp, n_stream)
    (1, 8, 1, 192, 1500, 10),   # multi-head attention (no grouping)
    (2, 4, 2, 128, 900, 40),
    (1, 4, 8, 192, 2000, 70),   # 8 query heads per kv head: two workgroups of 4 per head
    (3, 2, 8, 64, 333, 5),
    (1, 2, 16, 128, 700, 3),    # 16 query heads per kv head
    (1, 8, 3, 192, 3000, 20),   # Llama-3.2-3B's 24 query heads over 8 kv heads: groups of 3
    (2, 4, 6, 128, 800, 9),     # two groups of 3 per kv head
    (1, 4, 5, 160, 640, 2),     # 5 per kv head: five single-head workgroups
    (2, 2, 12, 192, 500, 4),    # three groups of 4
]


@pytest.mark.parametrize("case", GQA_CASES, ids=[str(c) for c in GQA_CASES])
def test_decode_other_gqa_groups(cuda, case):
    """Query-head groups of 1, 2, 3, 5, 6, 8, 12 and 16 on the token-tiled
    kernel (the reference's fused path takes any n_q / n_kv,
    attention.py:18-81)."""
    B, nkv, gqa, rank, n_comp, n_stream = case
    gc, inv = random_layer(B=B, nkv=nkv, rank=rank, n_comp=n_comp, n_stream=n_stream,
                           seed=7 * gqa + n_comp)
    q = torch.randn(B, gqa * nkv, 1, 128, generator=torch.Generator().manual_seed(6)).half()
    pos_q = 4 + n_comp + 64 + n_stream - 1
    want = exact.decode_attention(q.numpy(), gc, nkv, pos_q, inv.numpy())
    got = _run(cuda, gc, inv, q, pos_q, nkv=nkv, kernel=0)
    err, cos = compare(got, want)
    print(f"gqa case={case} max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= TOL_ABS and cos >= TOL_COS


HD64_CASES = [
    # (B, nkv, query heads per kv head, rank, n_comp, sink, win, n_stream, n_dec)
    (1, 8, 4, 192, 2000, 4, 64, 10, 0),    # 32 query heads over 8 kv heads of 64 dims
    (2, 4, 2, 128, 900, 4, 64, 40, 5),     # groups of 2: a workgroup holds both heads of a pair
    (1, 2, 1, 64, 333, 2, 3, 3, 0),        # no grouping: 2 query heads per pair
    (3, 2, 8, 100, 517, 4, 16, 1, 2),      # rank 100 (padded to 128), ragged tile
    (1, 4, 16, 192, 700, 4, 64, 2100, 0),  # 32 query heads per pair, 2,168 extra tokens
    (16, 8, 4, 128, 300, 4, 16, 1, 0),     # batch 16
    (1, 2, 6, 96, 1, 4, 64, 0, 0),         # a single compressed token, groups of 6 (12 per pair)
    (1, 4, 3, 128, 1500, 4, 64, 30, 0),    # 3 per kv head: groups of 3 over a pair's 6
    (2, 2, 5, 64, 400, 4, 32, 7, 3),       # 5 per kv head: groups of 2 over a pair's 10
]


@pytest.mark.parametrize("case", HD64_CASES, ids=[str(c) for c in HD64_CASES])
def test_decode_head_dim_64_matches_exact_oracle(cuda, case):
    """head_dim-64 layers (Llama-3.2-1B and TinyLlama shapes): the library runs
    kv heads 2j and 2j+1 as one 128-dim head on the token-tiled kernel (the
    reference's fused path takes any head_dim, attention.py:18-121); every
    kernel request, explicit split counts, same bar as head_dim 128."""
    B, nkv, gqa, rank, n_comp, sink, win, n_stream, n_dec = case
    gc, inv = random_layer(B=B, nkv=nkv, hd=64, rank=rank, n_comp=n_comp, sink=sink, win=win,
                           n_stream=n_stream, n_dec=n_dec, seed=3 * n_comp + gqa)
    q = torch.randn(B, gqa * nkv, 1, 64, generator=torch.Generator().manual_seed(9)).half()
    pos_q = sink + n_comp + win + n_dec + n_stream - 1
    want = exact.decode_attention(q.numpy(), gc, nkv, pos_q, inv.numpy())
    for kernel, ns in ((0, 0), (1, 0), (2, 0), (2, 1), (2, 7), (0, 300)):
        got = _run(cuda, gc, inv, q, pos_q, nkv=nkv, kernel=kernel, n_splits=ns, hd=64)
        err, cos = compare(got, want)
        print(f"hd64 case={case} kernel={kernel} n_splits={ns} max_abs={err:.3e} cos={cos:.7f}",
              flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS, (kernel, ns, err, cos)


def test_decode_head_dim_64_mask_and_device_position(cuda):
    """head_dim 64 with an additive mask over every segment, and the position
    read from device memory giving the host position's bits."""
    gc, inv = random_layer(B=2, nkv=4, hd=64, rank=128, n_comp=1200, n_stream=9, n_dec=3, seed=17)
    q = torch.randn(2, 16, 1, 64, generator=torch.Generator().manual_seed(2)).half()
    T = 4 + 1200 + 64 + 3 + 9
    mask = np.zeros((2, T), np.float32)
    rng = np.random.default_rng(1)
    mask[0, rng.choice(T, 60, replace=False)] = -65504.0
    mask[1, rng.choice(T, 60, replace=False)] = 0.75
    want = exact.decode_attention(q.numpy(), gc, 4, T - 1, inv.numpy(), attn_mask=mask)
    got = _run(cuda, gc, inv, q, T - 1, mask=mask, nkv=4, hd=64)
    err, cos = compare(got, want)
    print(f"hd64 mask max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= TOL_ABS and cos >= TOL_COS
    host = _run(cuda, gc, inv, q, T - 1, nkv=4, hd=64)
    dev = _run(cuda, gc, inv, q, torch.tensor([T - 1], dtype=torch.int64, device=cuda), nkv=4, hd=64)
    assert np.array_equal(host, dev)


def test_decode_split_counts_with_long_extras(cuda):
    """Explicit split counts from 1 to more splits than tiles: splits that hold
    only extra tiles, only compressed tiles, both, or nothing to do."""
    gc, inv = random_layer(n_comp=260, n_stream=300, n_dec=0, seed=21)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(8)).half()
    pos_q = 4 + 260 + 64 + 300 - 1
    want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
    for kernel in KERNELS:
        for ns in (1, 2, 3, 7, 13, 40, 500):
            got = _run(cuda, gc, inv, q, pos_q, n_splits=ns, kernel=kernel)
            err, cos = compare(got, want)
            print(f"kernel={kernel} n_splits={ns} max_abs={err:.3e} cos={cos:.7f}", flush=True)
            assert err <= TOL_ABS and cos >= TOL_COS, (kernel, ns, err, cos)


def test_decode_is_deterministic(cuda):
    """Repeated calls give the same bits with every split kernel: the tile to
    wave map and every merge order are fixed, nothing depends on wave timing.
    One split (188 tiles) takes the token-tiled kernel's unequal wave shares."""
    from shard_amd import ops
    gc, inv = random_layer(B=2, n_comp=6000, n_stream=37, seed=5)
    d = to_device(gc, cuda, inv)
    q = torch.randn(2, 32, 128, generator=torch.Generator().manual_seed(6)).half().to(cuda)
    for ns in (0, 1):
        call = ops.make_decode_args(q, d, 4 + 6000 + 64 + 37 - 1, None, stream_n=37, n_splits=ns)
        for kernel in KERNELS:
            call.args.kernel = kernel
            first = ops.decode_attn(call).clone()
            for rep in range(4):
                again = ops.decode_attn(call)
                torch.cuda.synchronize()
                assert torch.equal(again.view(torch.int16), first.view(torch.int16)), (ns, kernel, rep)


@pytest.mark.parametrize("kernel", KERNELS)
@pytest.mark.parametrize("bits,qjl", [(4, True), (2, False), (8, True)])
def test_decode_with_qjl_and_narrow_stream(cuda, bits, qjl, kernel):
    """Stream tokens quantized with 2/4-bit codes and the QJL residual
    (cache.py:234-240, 263-273): the oracle adds (2 sign - 1) * scale in the
    rotated domain before the inverse Hadamard."""
    gc, inv = random_layer(B=2, n_comp=400, n_stream=23, seed=bits, stream_bits=bits, qjl=qjl)
    q = torch.randn(2, 32, 1, 128, generator=torch.Generator().manual_seed(4)).half()
    pos_q = 4 + 400 + 64 + 23 - 1
    want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
    got = _run(cuda, gc, inv, q, pos_q, kernel=kernel)
    err, cos = compare(got, want)
    print(f"bits={bits} qjl={qjl} max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= TOL_ABS and cos >= TOL_COS


def test_large_rebuild_constant_decodes_fused(cuda):
    """Coefficient scales x 2000 (the rebuild constant C near 5e6, beyond what
    16 fp16 parts hold; q scaled down alike so the scores keep their range): the
    bf16 parts of the constant k-step carry it, both split kernels decode the
    layer within the bar, and a non-finite constant leaves the layer unfused
    with the reason given."""
    from shard_amd import attention, ops
    gc, inv = random_layer(B=1, rank=192, n_comp=1200, n_stream=3, seed=31)
    gc["k_coeff_scale"] = (gc["k_coeff_scale"].float() * 2000).half()
    d = to_device(gc, cuda, inv)
    cmax = ops.decode_constant_max(d["k_basis_pad"], d["k_coeff_scale_pad"], d["k_mean_f16"])
    assert cmax > 16 * 65504 and d["decode_prep"] is not None
    q = (torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(4)) / 2000).half()
    pos_q = 4 + 1200 + 64 + 3 - 1
    want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
    for kernel in KERNELS:
        got = _run(cuda, gc, inv, q, pos_q, kernel=kernel)
        err, cos = compare(got, want)
        print(f"[C={cmax:.3g}] kernel={kernel} max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS, (kernel, err, cos)
    bad = dict(gc)
    bad["k_coeff_scale"] = gc["k_coeff_scale"].clone()
    bad["k_coeff_scale"][3] = float("inf")
    d2 = to_device(bad, cuda, inv)
    assert d2["decode_prep"] is None and "rebuild constant" in d2["decode_refusal"]
    assert not attention.fused_supported(d2, 32)


@pytest.mark.parametrize("rank", [224, 256])
def test_decode_ranks_above_192(cuda, rank):
    """Ranks 224 and 256 (a Cache with a larger max_rank_k): the token-tiled
    kernel takes them (a forced row-split request routes there too), batch 2
    with stream and decode tokens, the same bar."""
    gc, inv = random_layer(B=2, rank=rank, n_comp=1500, n_stream=6, n_dec=3, seed=rank,
                           basis_amp=0.02)
    q = torch.randn(2, 32, 1, 128, generator=torch.Generator().manual_seed(3)).half()
    pos_q = 4 + 1500 + 64 + 3 + 6 - 1
    want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
    for kernel in KERNELS:
        got = _run(cuda, gc, inv, q, pos_q, kernel=kernel)
        err, cos = compare(got, want)
        print(f"rank={rank} kernel={kernel} max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS, (kernel, err, cos)


@pytest.mark.parametrize("kernel", KERNELS)
def test_decode_rank_padding_and_splits(cuda, kernel):
    """rank 100 (padded to 128 on the device) and several explicit split counts."""
    gc, inv = random_layer(rank=100, n_comp=1000, seed=5)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(2)).half()
    pos_q = 4 + 1000 + 64 - 1
    want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
    for ns in (8, 16, 64, 200):
        got = _run(cuda, gc, inv, q, pos_q, n_splits=ns, kernel=kernel)
        err, cos = compare(got, want)
        assert err <= TOL_ABS and cos >= TOL_COS, (ns, err, cos)


@pytest.mark.parametrize("kernel", KERNELS)
def test_decode_additive_mask(cuda, kernel):
    gc, inv = random_layer(n_comp=700, n_stream=4, seed=8)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(3)).half()
    T = 4 + 700 + 64 + 4
    mask = np.zeros((1, T), np.float32)
    rng = np.random.default_rng(0)
    mask[0, rng.choice(T, 50, replace=False)] = -65504.0   # HF fp16 masked entries
    mask[0, rng.choice(T, 50, replace=False)] = 0.5
    want = exact.decode_attention(q.numpy(), gc, 8, T - 1, inv.numpy(), attn_mask=mask)
    got = _run(cuda, gc, inv, q, T - 1, mask=mask, kernel=kernel)
    err, cos = compare(got, want)
    assert err <= TOL_ABS and cos >= TOL_COS


@pytest.mark.parametrize("kernel", KERNELS)
def test_decode_softmax_max_moves_late(cuda, kernel):
    """Scores that keep rising along the context (an additive ramp, then steps of
    +5.4 and +30 in natural-log units): the token-tiled kernel's reference max
    then moves in later tiles (rescaling the sums it holds) and, between moves,
    numerators come within 2^0.2 of their 2^8 bound."""
    gc, inv = random_layer(n_comp=4000, n_stream=4, seed=11)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(5)).half()
    T = 4 + 4000 + 64 + 4
    mask = np.zeros((1, T), np.float32)
    mask[0, 4:4004] = np.linspace(0.0, 60.0, 4000, dtype=np.float32)
    mask[0, 2500:2600] += 5.4      # log2 7.8 above its neighbours: no move, large numerators
    mask[0, 3300:3310] += 30.0     # forces a move inside the compressed span
    want = exact.decode_attention(q.numpy(), gc, 8, T - 1, inv.numpy(), attn_mask=mask)
    got = _run(cuda, gc, inv, q, T - 1, mask=mask, kernel=kernel)
    err, cos = compare(got, want)
    print(f"[max moves late] kernel={kernel} max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= TOL_ABS and cos >= TOL_COS


@pytest.mark.parametrize("kernel", KERNELS)
def test_decode_vs_reference_golden(cuda, golden, kernel):
    """The reference's own CPU output on its stub cache (fp16 intermediates)."""
    from tests.test_oracle import _gc_from_fixture
    f = golden("fused_attn.npz")
    gc, nkv = _gc_from_fixture(f)
    gc["v_idx_full"] = gc["v_idx_full"].reshape(1, nkv, gc["n_compress"], 32)
    inv = torch.from_numpy(f["inv_freq"])
    got = _run(cuda, gc, inv, torch.from_numpy(f["q_rope"]), int(f["pos_q"]), nkv=nkv, kernel=kernel)
    want64 = exact.decode_attention(f["q_rope"], gc, nkv, int(f["pos_q"]), f["inv_freq"])
    err, cos = compare(got, want64)
    assert err <= TOL_ABS and cos >= TOL_COS
    err_ref, cos_ref = compare(got, f["out"])
    print(f"vs reference fp16 path: max_abs={err_ref:.3e} cos={cos_ref:.7f}")
    assert err_ref <= 5e-3 and cos_ref >= 0.9999


@pytest.mark.parametrize("kernel", KERNELS)
def test_decode_compressed_real_synthetic(cuda, kernel):
    """Config-1 synthetic K/V compressed by the CPU oracle (PCA + DP bits + int4 +
    k-means VQ), then decoded on the GPU."""
    from shard_amd import bench_data
    k, v = bench_data.make_kv(2048, seed=0)
    inv = bench_data.inv_freq()
    basis = bench_data.random_orthonormal_basis(rank=192, seed=0)
    gc = ref.compress_layer(k, v, 0, inv, basis=basis)
    q = bench_data.make_q(seed=0)
    want = exact.decode_attention(q.numpy(), gc, 8, 2048, inv.numpy())
    got = _run(cuda, gc, inv, q, 2048, kernel=kernel)
    err, cos = compare(got, want)
    print(f"synthetic T=2048: max_abs={err:.3e} cos={cos:.7f}")
    assert err <= TOL_ABS and cos >= TOL_COS


# The bench's 32K context at batch 1, and batch 16 with more than 64 tiles per
# split, where the token-tiled kernel gives the two waves of a SIMD unequal
# shares (batch 16 x 16K itself: test_decode_config5_layer_full_size).
LARGE = [(1, 32700, 0), (1, 32700, 512), (16, 4200, 8)]


_large_cases = {}


def _large_case(shape):
    """Layer, query and fp64 oracle output of a LARGE shape (the oracle takes
    10-15 s, so it runs once per shape for the three kernel choices)."""
    if shape not in _large_cases:
        B, n_comp, n_stream = shape
        gc, inv = random_layer(B=B, n_comp=n_comp, n_stream=n_stream, seed=11)
        g = torch.Generator().manual_seed(2)
        q = torch.randn(B, 32, 1, 128, generator=g).half()
        pos_q = 4 + n_comp + 64 + n_stream - 1
        want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
        _large_cases.clear()
        _large_cases[shape] = (gc, inv, q, pos_q, want)
    return _large_cases[shape]


@pytest.mark.parametrize("shape", LARGE, ids=[f"B{b}xn{n}+s{s}" for b, n, s in LARGE])
def test_decode_large_contexts(cuda, shape):
    """32K context, also with a 512-token 8-bit stream (the extra tokens spread
    over several splits)."""
    B, n_comp, n_stream = shape
    gc, inv, q, pos_q, want = _large_case(shape)
    for kernel in KERNELS:
        got = _run(cuda, gc, inv, q, pos_q, kernel=kernel)
        err, cos = compare(got, want)
        print(f"B={B} n_comp={n_comp} stream={n_stream} kernel={kernel} max_abs={err:.3e} cos={cos:.7f}",
              flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS, (kernel, err, cos)


def test_decode_config5_layer_full_size(cuda):
    """The end-to-end workload's layer at full size: batch 16 x 16,316 compressed
    tokens (16,384 with the 4 sink and 64 window tokens).  Every kernel against
    the fp64 oracle on batch rows 0 and 15 (the oracle over all 16 rows takes
    minutes), and the 16 rows of the row-split and token-tiled kernels against
    each other (two independent split schemes)."""
    B, n_comp = 16, 16316
    gc, inv = random_layer(B=B, n_comp=n_comp, seed=13)
    q = torch.randn(B, 32, 1, 128, generator=torch.Generator().manual_seed(4)).half()
    pos_q = 4 + n_comp + 64 - 1
    rows = [0, 15]
    want = exact.decode_attention(q[rows].numpy(), batch_rows(gc, rows), 8, pos_q, inv.numpy())
    outs = {}
    for kernel in KERNELS:
        got = _run(cuda, gc, inv, q, pos_q, kernel=kernel)
        err, cos = compare(got[rows], want)
        print(f"B=16 n_comp={n_comp} kernel={kernel} rows {rows}: max_abs={err:.3e} cos={cos:.7f}",
              flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS, (kernel, err, cos)
        outs[kernel] = got
    err, cos = compare(outs[1], outs[2])
    print(f"row-split vs token-tiled, all rows: max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= TOL_ABS and cos >= TOL_COS, (err, cos)


@pytest.mark.parametrize("rank,nkv,hd", [(160, 8, 128), (320, 8, 128), (512, 4, 128), (320, 8, 64)])
def test_kv_reconstruct(cuda, rank, nkv, hd):
    """Unfused fp16 reconstruction (_ensure_dequant): V bit-exact, K within fp16
    rounding.  Ranks above 256 (a Cache with a larger max_rank_k: the fused call
    does not take them, these layers decode through this path) up to the LDS
    staging limit, 512 at head_dim 128."""
    from shard_amd import ops
    gc, inv = random_layer(B=2, nkv=nkv, hd=hd, rank=rank, n_comp=300, seed=12)
    d = to_device(gc, cuda, inv, nkv=nkv, hd=hd)
    assert (d["decode_prep"] is None) == (rank > 256)
    k_got, v_got = ops.kv_reconstruct(d, 2)
    k_want, v_want = ref.reconstruct_kv(gc, nkv, hd, inv)
    assert np.array_equal(v_got.cpu().numpy().view(np.uint16), v_want.numpy().view(np.uint16))
    # the fp16 rounding of the rebuilt key depends on the fp32 accumulation order,
    # so a key may differ by an ulp of its pre-RoPE value (|k| < 2: ulp <= 2^-10)
    kg, kw = k_got.cpu().float(), k_want.float()
    diff = (kg - kw).abs()
    assert float(diff.max()) <= 2 * 2.0 ** -10
    assert float((diff > 0).float().mean()) < 0.02


@pytest.mark.parametrize("group,n_cent", [(2, 256), (8, 256), (1, 16), (4, 64)])
def test_kv_reconstruct_vq_shapes(cuda, group, n_cent):
    """V subvectors of 1, 2 or 8 values and codebooks below 256 rows (a Cache
    built with another v_vq_group_size or v_vq_codebook_size): the unfused
    reconstruction's V bit-exact with the oracle's vq_decode + hadamard; the
    fused call takes only 4-value subvectors (a smaller codebook padded to 256
    rows)."""
    from shard_amd import ops
    gc, inv = random_layer(B=2, nkv=4, hd=128, rank=64, n_comp=200, seed=21,
                           v_group=group, v_codebook=n_cent)
    d = to_device(gc, cuda, inv, nkv=4, hd=128)
    assert (d["decode_prep"] is None) == (group != 4)
    _, v_got = ops.kv_reconstruct(d, 2)
    _, v_want = ref.reconstruct_kv(gc, 4, 128, inv)
    assert np.array_equal(v_got.cpu().numpy().view(np.uint16), v_want.numpy().view(np.uint16))


def test_decode_small_codebook_fused(cuda):
    """A 64-row codebook of 4-value subvectors decodes on the fused kernels
    (padded to 256 rows that no index names) within the fp64 oracle's
    tolerance, on both split kernels."""
    gc, inv = random_layer(B=1, n_comp=900, seed=22, v_codebook=64)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(23)).half()
    pos_q = 4 + 900 + 64
    want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
    for kernel in KERNELS:
        got = _run(cuda, gc, inv, q, pos_q, kernel=kernel)
        err, cos = compare(got, want)
        print(f"kernel {kernel}: max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS


@pytest.mark.parametrize("kernel", KERNELS)
def test_decode_device_position_matches_host_position(cuda, kernel):
    """pos_q read by the kernel from a device int64 (the patched forward passes
    cache_position[-1:] instead of the reference's .item(), attention.py:383)
    gives the same bits as the host integer, also with a position that is not
    the last cached token."""
    gc, inv = random_layer(B=2, n_comp=700, n_stream=4, seed=11)
    q = torch.randn(2, 32, 1, 128, generator=torch.Generator().manual_seed(5)).half()
    for pos_q in (4 + 700 + 64 + 4 - 1, 5000):
        host = _run(cuda, gc, inv, q, pos_q, kernel=kernel)
        dev = _run(cuda, gc, inv, q, torch.tensor([pos_q - 3, pos_q], dtype=torch.int64, device=cuda),
                   kernel=kernel)
        print(f"pos_q={pos_q} max diff={np.abs(host - dev).max():.3e}", flush=True)
        assert np.array_equal(host, dev)
        want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
        err, cos = compare(dev, want)
        assert err <= TOL_ABS and cos >= TOL_COS


def test_fused_attention_grows_a_small_workspace(cuda):
    """The patched forward's call runs on the device's shared workspace and asks
    for the size only when the library reports it too small (before it
    launches anything): a too-small buffer is replaced and the call retried,
    with the same bits as a call on a workspace of the queried size."""
    from shard_amd import attention, ops
    gc, inv = random_layer(B=2, n_comp=3000, n_stream=5, seed=17)
    d = to_device(gc, cuda, inv)
    q = torch.randn(2, 32, 1, 128, generator=torch.Generator().manual_seed(9)).half().to(cuda)
    pos_q = 4 + 3000 + 64 + 5 - 1

    class _CacheRef:
        _rope_inv_freq = d["inv_freq_dev"]
        _n_splits = 0

    class _Layer:
        _gpu_compressed = d
        _cache_ref = _CacheRef()

    key = (cuda.type, cuda.index)
    saved = attention._workspaces.get(key)
    try:
        attention._workspaces[key] = torch.zeros(16, dtype=torch.uint8, device=cuda)
        got = attention.fused_attention_compressed(q, _Layer(), pos_q, d["inv_freq_dev"]).clone()
        call = d["_decode_call"]
        assert attention._workspaces[key].numel() >= call.workspace_bytes() > 16
        want = ops.decode_attn(ops.make_decode_args(q.reshape(2, 32, 128), d, pos_q, None, stream_n=5))
        torch.cuda.synchronize()
        assert torch.equal(got.reshape(2, 32, 128).view(torch.int16), want.view(torch.int16))
    finally:
        if saved is None:
            attention._workspaces.pop(key, None)
        else:
            attention._workspaces[key] = saved


def test_decode_one_split_past_the_phase_tables(cuda):
    """n_splits = 1 over 40,000 compressed tokens (1,250 tiles): the token-tiled
    kernel's phase tables cover 1,024 tiles per split, so its plan splits the
    range in two; the row-split kernel advances its phases per tile and takes
    the whole range in one split."""
    n_comp = 40000
    gc, inv = random_layer(B=1, n_comp=n_comp, n_stream=3, seed=41)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(14)).half()
    pos_q = 4 + n_comp + 64 + 3 - 1
    want = exact.decode_attention(q.numpy(), gc, 8, pos_q, inv.numpy())
    for kernel in KERNELS:
        got = _run(cuda, gc, inv, q, pos_q, n_splits=1, kernel=kernel)
        err, cos = compare(got, want)
        print(f"one split over {n_comp} tokens, kernel={kernel}: max_abs={err:.3e} cos={cos:.7f}",
              flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS, (kernel, err, cos)


@pytest.mark.parametrize("case", [(1, 8, 1, 192, 2500), (1, 4, 8, 128, 2300), (2, 2, 2, 192, 2200)],
                         ids=["gqa1", "gqa8", "gqa2_b2"])
def test_decode_long_split_other_groups(cuda, case):
    """One split of 70+ tiles (the token-tiled kernel's 3:2 wave shares) with
    1, 2 and 8 query heads per kv head."""
    B, nkv, gqa, rank, n_comp = case
    gc, inv = random_layer(B=B, nkv=nkv, rank=rank, n_comp=n_comp, n_stream=7, seed=31 + gqa)
    q = torch.randn(B, gqa * nkv, 1, 128, generator=torch.Generator().manual_seed(12)).half()
    pos_q = 4 + n_comp + 64 + 7 - 1
    want = exact.decode_attention(q.numpy(), gc, nkv, pos_q, inv.numpy())
    got = _run(cuda, gc, inv, q, pos_q, nkv=nkv, n_splits=1, kernel=2)
    err, cos = compare(got, want)
    print(f"long split {case}: max_abs={err:.3e} cos={cos:.7f}", flush=True)
    assert err <= TOL_ABS and cos >= TOL_COS


@pytest.mark.parametrize("kernel", KERNELS)
def test_decode_stream_count_from_device(cuda, kernel):
    """shard_decode_args.n_stream_dev: a call planned for 40 stream rows that
    reads a smaller count (and a larger one, clamped) from the device attends
    over exactly that many rows: against the fp64 oracle of the layer holding
    only those rows, and one call block reused with new counts (as a captured
    graph replays it)."""
    from shard_amd import ops
    B, n_comp, n_plan = 2, 700, 40
    gc, inv = random_layer(B=B, n_comp=n_comp, n_stream=n_plan, seed=21)
    d = to_device(gc, cuda, inv)
    q = torch.randn(B, 32, 1, 128, generator=torch.Generator().manual_seed(6)).half()
    cnt = torch.zeros(1, dtype=torch.int32, device=cuda)
    pos = torch.zeros(1, dtype=torch.int64, device=cuda)
    call = ops.make_decode_args(q.to(cuda).reshape(B, 32, 128), d, pos, None, stream_n=n_plan,
                                stream_n_dev=cnt)
    call.args.kernel = kernel
    ws = ops.decode_workspace(call)
    for n_now in (25, 0, 1, 40, 57):
        s = min(n_now, n_plan)
        part = dict(gc, stream_n=s * B)
        pos_q = 4 + n_comp + 64 + s - 1
        want = exact.decode_attention(q.numpy(), part, 8, pos_q, inv.numpy())
        cnt.fill_(n_now)
        pos.fill_(pos_q)
        got = ops.decode_attn(call, ws).cpu().float().numpy().reshape(B, 32, 1, 128)
        err, cos = compare(got, want)
        print(f"kernel={kernel} count={n_now}: max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= TOL_ABS and cos >= TOL_COS, (n_now, err, cos)


def test_decode_stream_count_from_device_rejects_mask(cuda):
    """A device stream count with an attention mask is refused (the mask row
    would have to follow the count) before anything is launched."""
    from shard_amd import ops
    from shard_amd._lib import ShardHipError
    gc, inv = random_layer(B=1, n_comp=100, n_stream=8, seed=22)
    d = to_device(gc, cuda, inv)
    q = torch.randn(1, 32, 128).half().to(cuda)
    mask = torch.zeros(1, 4 + 100 + 64 + 8, device=cuda)
    cnt = torch.full((1,), 8, dtype=torch.int32, device=cuda)
    call = ops.make_decode_args(q, d, 4 + 100 + 64 + 7, None, mask=mask, stream_n=8,
                                stream_n_dev=cnt)
    with pytest.raises(ShardHipError) as exc:
        ops.decode_attn(call)
    assert exc.value.code == -1  # SHARD_ERR_ARG


def test_fused_attention_across_the_kernel_switch(cuda):
    """One layer's argument block refreshed across the automatic kernel switch:
    with 257 extra tokens (4 sink + 64 window + 189 stream) the call takes the
    token-tiled kernel, with 256 the row-split one, whose plan needs a larger
    workspace.  The patched forward's shared workspace, sized by the first
    call, grows for the second; both match the fp64 oracle."""
    from shard_amd import attention
    n_comp, n_st = 1500, 189
    gc, inv = random_layer(B=1, n_comp=n_comp, n_stream=n_st, seed=23)
    d = to_device(gc, cuda, inv)
    q = torch.randn(1, 32, 1, 128, generator=torch.Generator().manual_seed(4)).half()

    class _CacheRef:
        _rope_inv_freq = d["inv_freq_dev"]
        _n_splits = 0

    class _Layer:
        _gpu_compressed = d
        _cache_ref = _CacheRef()

    key = (cuda.type, cuda.index)
    saved = attention._workspaces.get(key)
    try:
        attention._workspaces[key] = torch.zeros(16, dtype=torch.uint8, device=cuda)
        sizes = []
        for s in (189, 188):
            d["stream_n"] = s
            pos_q = 4 + n_comp + 64 + s - 1
            print(f"[kernel switch] extra tokens {68 + s}", flush=True)
            got = attention.fused_attention_compressed(q.to(cuda), _Layer(), pos_q, d["inv_freq_dev"])
            torch.cuda.synchronize()
            sizes.append(d["_decode_call"].workspace_bytes())
            assert attention._workspaces[key].numel() >= sizes[-1]
            g_s = dict(gc)
            g_s["stream_n"] = s
            for name in ("k_idx_buf", "v_idx_buf", "k_norm_buf", "v_norm_buf"):
                g_s[name] = gc[name][:s]
            want = exact.decode_attention(q.numpy(), g_s, 8, pos_q, inv.numpy())
            err, cos = compare(got.cpu().float().numpy().reshape(want.shape), want)
            print(f"[kernel switch] extras {68 + s}: workspace {sizes[-1]} B max_abs={err:.3e} cos={cos:.7f}",
                  flush=True)
            assert err <= TOL_ABS and cos >= TOL_COS
        assert sizes[1] > sizes[0], sizes  # the row-split plan has more partial rows
    finally:
        if saved is None:
            attention._workspaces.pop(key, None)
        else:
            attention._workspaces[key] = saved
