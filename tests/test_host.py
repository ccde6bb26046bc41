"""Host logic of shard_amd on the CPU: tables, HF Cache glue, the Llama patch
and its fallbacks (forced from the host, no kernel launched)."""
import os

import numpy as np
import pytest
import torch

from oracle import ref


def test_dp_allocation_matches_oracle():
    from shard_amd import host
    rng = np.random.default_rng(0)
    for trial in range(20):
        d = int(rng.integers(2, 400))
        var = np.sort(rng.exponential(1.0, d))[::-1].astype(np.float32) * rng.uniform(0.1, 100)
        budget = int(rng.integers(16, 4096))
        assert host.dp_bit_allocation(torch.from_numpy(var.copy()), budget) == \
            ref.dp_bit_allocation(torch.from_numpy(var.copy()), budget)


def test_lloyd_max_and_signs(golden):
    from shard_amd import host
    assert np.array_equal(host.lloyd_max_codebook(128, 8).numpy(), golden("lloyd_max.npz")["codebook"])
    for layer in (0, 1, 31):
        assert np.array_equal(host.stream_signs(layer, 128).numpy(), ref.stream_signs(layer, 128))


def test_cache_constructs_and_prefill_glue():
    import shard
    from shard_amd import Cache
    assert shard.Cache is Cache
    c = Cache(num_layers=2)
    assert len(c.layers) == 2 and c.get_seq_length() == 0
    k = torch.randn(1, 8, 100, 128).half()
    v = torch.randn(1, 8, 100, 128).half()
    kk, vv = c.update(k, v, 0)
    assert kk is k and vv is v
    assert c.get_seq_length(0) == 100
    assert c.layers[0].get_mask_sizes(1) == (101, 0)
    assert c.layers[0].get_max_length() == -1
    assert c.memory_bytes() == 2 * k.numel() * 2
    assert c.fp16_equivalent_bytes() == 100 * 8 * 128 * 4 * 2


def test_accounting_counts_one_batch_row_like_the_reference():
    """fp16_equivalent_bytes / compress_ratio count one batch row, as
    cache.py:518-532 does; the *_all_rows variants count the whole batch."""
    from shard_amd import Cache
    c = Cache(num_layers=2)
    k = torch.randn(3, 8, 50, 128).half()
    c.update(k, k.clone(), 0)
    c.update(k.clone(), k.clone(), 1)
    one_row = 50 * 8 * 128 * 4 * 2
    assert c.fp16_equivalent_bytes() == one_row
    assert c.fp16_equivalent_bytes_all_rows() == 3 * one_row
    assert c.memory_bytes() == 4 * k.numel() * 2
    assert c.compress_ratio() == one_row / c.memory_bytes()


def test_compress_on_cpu_fails_loudly():
    from shard_amd import Cache, ops
    c = Cache(num_layers=1)
    c.update(torch.randn(1, 8, 200, 128).half(), torch.randn(1, 8, 200, 128).half(), 0)
    with pytest.raises(ops.ShardHipUnavailable):
        c.update(torch.randn(1, 8, 1, 128).half(), torch.randn(1, 8, 1, 128).half(), 0)


def test_compress_refuses_non_fp16_models():
    """The compressed format is fp16 (the reference's documented model dtype):
    a bfloat16 prefill raises a clear TypeError at the compressing step."""
    from shard_amd import Cache
    c = Cache(num_layers=1)
    c.update(torch.randn(1, 8, 200, 128).bfloat16(), torch.randn(1, 8, 200, 128).bfloat16(), 0)
    with pytest.raises(TypeError, match="fp16"):
        c.update(torch.randn(1, 8, 1, 128).bfloat16(), torch.randn(1, 8, 1, 128).bfloat16(), 0)


def test_short_prompt_skips_compression():
    from shard_amd import Cache
    c = Cache(num_layers=1)
    c.update(torch.randn(1, 8, 60, 128), torch.randn(1, 8, 60, 128), 0)
    k, v = c.update(torch.randn(1, 8, 1, 128), torch.randn(1, 8, 1, 128), 0)
    assert k.shape[2] == 61 and c.layers[0]._gpu_compressed is None


def _tiny_llama():
    from transformers import LlamaConfig, LlamaForCausalLM
    # the fused decode kernel's shapes: head_dim 128, 4 query heads per kv head
    cfg = LlamaConfig(vocab_size=64, hidden_size=512, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=1, head_dim=128,
                      max_position_embeddings=256, rope_theta=500000.0)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).eval()


def test_llama_patch_falls_back_on_uncompressed_layers():
    """Patched forward == original forward when no layer is compressed
    (attention.py:359-368 routing), with both a DynamicCache and a shard Cache."""
    from transformers import DynamicCache
    from shard_amd import Cache, enable_llama_fused_attention
    from shard_amd.host import get_rope_inv_freq
    model = _tiny_llama()
    ids = torch.randint(0, 64, (1, 20))
    with torch.no_grad():
        base = model(ids, past_key_values=DynamicCache(), use_cache=True).logits
    assert enable_llama_fused_attention(model) is True
    assert enable_llama_fused_attention(model) is True   # idempotent
    with torch.no_grad():
        patched = model(ids, past_key_values=DynamicCache(), use_cache=True).logits
        c = Cache.from_model(model)
        sh = model(ids, past_key_values=c, use_cache=True).logits
    assert torch.equal(base, patched)
    assert torch.allclose(base, sh)
    assert torch.equal(get_rope_inv_freq(model), model.model.rotary_emb.inv_freq.float())
    assert c.get_seq_length() == 20


def test_full_fused_error_is_counted_then_default_path_runs(monkeypatch):
    """A failing opt-in full-fused call is counted and the default path runs
    (attention.py:386-403); forced from the host with stub layers."""
    from shard_amd import attention
    calls = []

    def boom(*a, **k):
        raise RuntimeError("forced")

    def ok(q, layer, pos_q, inv, mask):
        calls.append(pos_q)
        return torch.zeros_like(q)

    monkeypatch.setattr(attention, "fused_attention_compressed_full", boom)
    monkeypatch.setattr(attention, "fused_attention_compressed", ok)
    from shard_amd import Cache, enable_llama_fused_attention
    model = _tiny_llama()
    enable_llama_fused_attention(model)
    c = Cache.from_model(model)
    c._full_fused = True
    for l in c.layers:  # stub format of a shape the fused kernel takes
        l._gpu_compressed = {"head_dim": 128, "n_kv": 1, "rank_pad": 32, "decode_prep": object()}
        l._prefilled = True
        l._seq_len = 10
    c._compressed = True
    c._streaming = False

    def upd(self, k, v, *a, **kw):
        self._seq_len += 1
        return k, v
    monkeypatch.setattr(type(c.layers[0]), "update", upd)
    ids = torch.randint(0, 64, (1, 1))
    with torch.no_grad():
        model(ids, past_key_values=c, use_cache=True)
    assert c._full_fused_attempts == 2 and c._full_fused_errors == 2
    assert "forced" in c._last_full_fused_error
    assert calls == [10, 10]


def test_unsupported_shapes_take_the_original_forward(monkeypatch):
    """A model outside the decode kernel's shapes (head_dim 16) decodes through
    the original forward on compressed layers, without calling the fused path,
    and every such layer-step is counted with its shape."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from shard_amd import attention, Cache, enable_llama_fused_attention
    called = []
    monkeypatch.setattr(attention, "fused_attention_compressed",
                        lambda *a, **k: called.append(1) or None)
    cfg = LlamaConfig(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                      max_position_embeddings=256, rope_theta=500000.0)
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    enable_llama_fused_attention(model)
    c = Cache.from_model(model)
    for l in c.layers:  # what finalize_format leaves for a head_dim the kernel lacks
        l._gpu_compressed = {"head_dim": 16, "n_kv": 2, "rank_pad": 32, "decode_prep": None}
        l._prefilled = True
        l._seq_len = 10
    c._compressed = True
    seen = []

    def upd(self, k, v, *a, **kw):  # the original forward's cache update
        seen.append(self.layer_idx)
        self._seq_len += 1
        return k, v
    monkeypatch.setattr(type(c.layers[0]), "update", upd)
    with torch.no_grad():
        model(torch.randint(0, 64, (1, 1)), past_key_values=c, use_cache=True)
    assert called == [] and seen == [0, 1]
    assert c._fused_fallbacks == 2 and "head_dim=16" in c._last_fused_fallback


def test_decode_supported_shapes():
    """The host mirror of shard_decode_supported agrees with the library's own
    answer (no GPU needed) on every combination it distinguishes."""
    import ctypes
    from shard_amd import _lib, ops
    lib = _lib.load()
    for hd in (64, 128, 256):
        for n_kv in (1, 2, 8):
            for g in (1, 2, 3, 4, 6, 8, 16, 64, 68):
                for rank in (32, 96, 100, 192, 224, 256, 288):
                    a = _lib.DecodeArgs()
                    a.batch, a.n_q_heads, a.n_kv_heads, a.head_dim = 1, g * n_kv, n_kv, hd
                    a.rank, a.n_comp = rank, 100
                    want = bool(lib.shard_decode_supported(ctypes.byref(a)))
                    assert ops.decode_supported(hd, g * n_kv, n_kv, rank) == want, (hd, n_kv, g, rank)


def test_decode_constant_formula():
    """decode_constant_max equals a direct float64 evaluation of the decode
    kernels' constant k-step, 16 mean - 16512 sum_even A' - 1152 sum_odd A'
    with A' = fp16(basis * cs); and 16 greedy bf16 parts (each the bf16
    rounding of what remains, as shard_decode_prepare splits it) hold C far
    beyond fp16's 16 x 65504 to below fp32 resolution."""
    from shard_amd import ops
    g = torch.Generator().manual_seed(0)
    basis = (torch.randn(256, 64, generator=g) * 0.1).half()
    cs = (torch.rand(64, generator=g) * 3).half()
    mean = torch.randn(256, generator=g).half()
    want = 0.0
    for row in range(256):
        c = 16.0 * float(mean[row])
        for r in range(64):
            a = float(np.float16(np.float32(basis[row, r]) * np.float32(cs[r])))
            c -= (16512.0 if r % 2 == 0 else 1152.0) * a
        want = max(want, abs(c))
    assert abs(ops.decode_constant_max(basis, cs, mean) - want) <= 1e-9 * want
    for c in (12345.678, -654321.5, 3.1e6, -7.77e8):
        rest = c
        for _ in range(16):
            h = float(torch.tensor(np.float32(rest)).to(torch.bfloat16).float())
            rest -= h
        assert abs(rest) <= abs(c) * 2.0 ** -40, (c, rest)


def test_decode_graph_refuses_other_caches():
    """DecodeGraph takes a compressed, streaming shard Cache only (checked before
    anything touches the GPU)."""
    import torch
    from shard_amd import Cache
    from shard_amd.graph import DecodeGraph
    ids = torch.zeros(1, 1, dtype=torch.long)
    with pytest.raises(TypeError):
        DecodeGraph(None, object(), ids, 4)
    with pytest.raises(ValueError):
        DecodeGraph(None, Cache(num_layers=1, device="cpu"), ids, 4)


@pytest.mark.parametrize("n", [1, 2, 3, 10, 256, 257, 1000, 123457, 5_000_000])
@pytest.mark.parametrize("seed", [0, 7, 42])
def test_kmeans_init_rows_equal_torch_randperm(n, seed):
    """The k-means init rows (the first 256 entries of the reference's CPU
    torch.randperm, cache.py:25) computed without the full permutation equal
    torch.randperm's own."""
    import torch
    from shard_amd import ops
    want = torch.randperm(n, generator=torch.Generator().manual_seed(seed))[:256]
    assert torch.equal(ops._randperm_head(n, 256, seed), want)


def test_bench_roofline_picks_the_binding_roof():
    """bench.roofline: above the fp16 MFMA ridge (312.5 flop/B) the MFMA peak
    binds and `achieved` is TFLOP/s; below it HBM binds and `achieved` is GB/s;
    the other roof is reported beside it.  The 8K decode call's algorithmic
    figures (about 1,000 flop/B) are MFMA-bound."""
    import bench
    r = bench.roofline(bench.algorithmic_flops(8124, 192), bench.algorithmic_bytes(8124, 192), 17.5)
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["peak"] == 2500.0
    assert abs(r["achieved"] - 3_360_866_304 / 17.5e-6 / 1e12) < 0.01
    assert abs(r["frac"] - r["achieved"] / 2500.0) < 1e-4
    assert r["hbm"]["unit"] == "GB/s" and abs(r["hbm"]["achieved"] - 3_358_080 / 17.5e-6 / 1e9) < 0.1
    assert r["ridge_flop_per_byte"] == 312.5 and 990 < r["intensity_flop_per_byte"] < 1010
    low = bench.roofline(1e9, 1e8, 100.0)  # 10 flop/B: HBM-bound
    assert low["bound"] == "hbm" and low["unit"] == "GB/s" and low["achieved"] == 1000.0
    assert low["mfma"]["unit"] == "TFLOP/s"


def test_decode_graph_refuses_a_masked_cache_and_reorder_under_a_graph():
    """A decode graph replays without an attention mask: it refuses a cache
    whose last eager decode step attended with a padding mask.  While a graph
    is open, reorder_cache (which replaces tensors the graph captured) raises."""
    import torch
    from shard_amd.cache import Cache
    from shard_amd.graph import DecodeGraph
    cache = Cache(head_dim=128, num_layers=2, n_kv_heads=8, device="cpu")
    cache._compressed, cache._streaming = True, True
    cache._last_attn_mask = torch.tensor([[0.0, float("-inf"), 0.0]])
    with pytest.raises(ValueError, match="padding mask"):
        DecodeGraph(None, cache, torch.zeros(1, 1, dtype=torch.long), 3)
    cache._last_attn_mask = torch.zeros(1, 3)
    with pytest.raises(ValueError, match="on the GPU"):
        DecodeGraph(None, cache, torch.zeros(1, 1, dtype=torch.long), 3)
    cache._graph = object()
    with pytest.raises(RuntimeError, match="decode graph"):
        cache.reorder_cache(torch.tensor([0]))


def test_boolean_attention_masks_become_additive():
    """transformers' sdpa masks are boolean (True = attend): the decode path
    takes them as the additive mask they stand for (0 / fp32 min), so padding
    keys are masked rather than shifted by 1.0; float masks pass as added."""
    from shard_amd.ops import additive_mask
    b = torch.tensor([[[[True, False, True]]]])
    m = additive_mask(b)
    assert m.dtype == torch.float32 and m.shape == b.shape
    assert m.reshape(-1).tolist() == [0.0, torch.finfo(torch.float32).min, 0.0]
    f = torch.tensor([[0.0, -1e9, 0.0]], dtype=torch.float16)
    assert additive_mask(f).dtype == torch.float32
    f32 = torch.tensor([[0.0, float("-inf")]])
    assert additive_mask(f32) is f32


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 exits with a message (one GPU is built and
    measured); nothing is launched."""
    import json
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode != 0
    assert "one GPU" in json.loads(out.stdout.strip().splitlines()[-1])["error"]


def test_cache_refuses_vq_shapes_it_cannot_decode():
    """V subvectors of 1, 2, 4 or 8 values and 1..256 centroids are taken;
    other values are refused when the Cache is built, not after a layer's
    compression."""
    from shard_amd import Cache
    for gs in (1, 2, 4, 8):
        Cache(num_layers=1, v_vq_group_size=gs, device="cpu")
    Cache(num_layers=1, v_vq_codebook_size=1, device="cpu")
    for kw in ({"v_vq_group_size": 3}, {"v_vq_group_size": 16}, {"v_vq_codebook_size": 300},
               {"v_vq_codebook_size": 0}, {"head_dim": 100, "v_vq_group_size": 8}):
        with pytest.raises(ValueError):
            Cache(num_layers=1, device="cpu", **kw)


def test_reference_import_paths_resolve():
    """The import paths the reference's scripts use (example.py:9,
    benchmarks/benchmark.py:43-45) resolve to this build's objects."""
    import shard
    import shard_amd
    from shard.attention import enable_llama_fused_attention, fused_attention_compressed
    from shard.cache import Cache
    from shard.rope import get_rope_inv_freq
    assert shard.Cache is Cache is shard_amd.Cache
    assert enable_llama_fused_attention is shard_amd.enable_llama_fused_attention
    assert fused_attention_compressed is shard_amd.fused_attention_compressed
    from shard_amd.host import get_rope_inv_freq as mine
    assert get_rope_inv_freq is mine
