"""The shard Cache driven by a real (random-init) Llama on the GPU:

* transformers' generate() with the Cache, as the reference's example.py
  drives it, against a hand-written greedy loop;

* batch 16 (the end-to-end decode batch, shorter prompt): the fused
  decode call the patched forward makes, checked against the fp64 oracle over
  the layer's own compressed representation (attention.py:300-343,
  cache.py:156-181);
* beam reordering of a compressed cache (cache.py:287-292): the dequantized
  rows are selected as the reference does, and later decode steps read the
  reordered compressed rows;
* a head_dim-64 model with an even kv head count (kv heads paired) and
  Llama-3.2-3B's 3 query heads per kv head: every decode step is fused and
  checked against the oracle; head_dim 64 with one kv head: decode runs the
  original forward on rebuilt K/V, every such layer-step counted;
* other Cache options: 64 centroids, no sink tokens, longer sinks and
  windows (fused, oracle-checked); subvectors of 8 values (unfused, equal to
  the unpatched forward).
"""
import pytest
import torch

from oracle import exact
from tests.helpers import compare

pytestmark = pytest.mark.gpu

VOCAB = 512


def _llama(dev, n_q=32, n_kv=8, hd=128, hidden=1024):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=VOCAB, hidden_size=hidden, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=n_q, num_key_value_heads=n_kv,
                      head_dim=hd, max_position_embeddings=4096, rope_theta=500000.0)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(dev, torch.float16).eval()


def _oracle_format(gc):
    """The oracle's view (CPU) of a device-format compressed layer, stream rows
    up to the current length."""
    B = gc["batch"]
    o = {k: gc[k].detach().cpu() for k in ("k_coeffs", "k_coeff_scale", "k_basis_f16", "k_mean_f16",
                                           "v_centroids_f16", "v_ch_f16", "sink_k", "sink_v",
                                           "win_k", "win_v")}
    o.update({"k_coeffs_shape": gc["k_coeffs_shape"], "n_compress": gc["n_compress"], "batch": B,
              "compress_start": gc["compress_start"], "v_idx_full": gc["v_indices"].cpu()})
    s = gc.get("stream_n", 0) // B
    if s:
        o.update({"stream_n": gc["stream_n"], "signs": gc["signs"].cpu().numpy(),
                  "stream_codebook": gc["stream_codebook"].cpu().numpy()})
        for k in ("k_idx_buf", "v_idx_buf", "k_norm_buf", "v_norm_buf"):
            o[k] = gc[k][:s].cpu().numpy()
    if "decode_k" in gc:
        o["decode_k"], o["decode_v"] = gc["decode_k"].cpu(), gc["decode_v"].cpu()
    return o


def test_batch16_cache_decode_matches_oracle(cuda, monkeypatch):
    from shard_amd import Cache, attention, enable_llama_fused_attention
    model = _llama(cuda)
    assert enable_llama_fused_attention(model)
    seen = []
    inner = attention.fused_attention_compressed

    def record(q, layer, pos_q, inv, mask=None):
        out = inner(q, layer, pos_q, inv, mask)
        if layer.layer_idx == 1:
            p = int(pos_q.reshape(-1)[-1].item()) if torch.is_tensor(pos_q) else int(pos_q)
            seen.append((q.detach().cpu(), p, out.detach().cpu(),
                         _oracle_format(layer._gpu_compressed), inv.cpu()))
        return out
    monkeypatch.setattr(attention, "fused_attention_compressed", record)
    g = torch.Generator().manual_seed(3)
    B, T = 16, 600
    ids = torch.randint(0, VOCAB, (B, T), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (B, 3), generator=g).to(cuda)
    cache = Cache.from_model(model)
    cache._streaming = True
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        for s in range(steps.shape[1]):
            model(steps[:, s:s + 1], past_key_values=cache, use_cache=True)
    assert len(seen) == 3 and cache.layers[1]._gpu_compressed["batch"] == B
    for i, (q, pos_q, out, gc, inv) in enumerate(seen):
        assert pos_q == T + i and gc["stream_n"] == B * (i + 1)
        want = exact.decode_attention(q.float().numpy().reshape(B, 32, 1, 128), gc, 8, pos_q,
                                      inv.numpy())
        err, cos = compare(out.float().numpy().reshape(want.shape), want)
        print(f"[batch16 cache] step {i} pos_q={pos_q} max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= 2e-3 and cos >= 0.9999


@pytest.mark.parametrize("B", [1, 2])
def test_generate_with_the_cache(cuda, B):
    """transformers' generate() with the Cache as past_key_values, as the
    reference's example.py and benchmark drive it (greedy, an all-ones
    attention mask): compression at the first decode step, fused decode after
    it, the same tokens as a hand-written greedy loop over a fresh Cache, and
    the accounting methods afterwards."""
    from shard_amd import Cache, enable_llama_fused_attention
    model = _llama(cuda)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(12)
    ids = torch.randint(0, VOCAB, (B, 300), generator=g).to(cuda)
    n_new = 6
    cache = Cache.from_model(model)
    cache._streaming = True
    with torch.no_grad():
        out = model.generate(input_ids=ids, attention_mask=torch.ones_like(ids), max_new_tokens=n_new,
                             do_sample=False, past_key_values=cache, pad_token_id=0)
    assert out.shape == (B, 300 + n_new)
    assert cache.layers[0]._gpu_compressed is not None
    assert getattr(cache, "_fused_fallbacks", 0) == 0
    # the same greedy steps by hand
    ref_cache = Cache.from_model(model)
    ref_cache._streaming = True
    toks = []
    with torch.no_grad():
        logits = model(ids, past_key_values=ref_cache, use_cache=True).logits[:, -1]
        for _ in range(n_new):
            nxt = logits.argmax(-1, keepdim=True)
            toks.append(nxt)
            logits = model(nxt, past_key_values=ref_cache, use_cache=True).logits[:, -1]
    assert torch.equal(out[:, 300:], torch.cat(toks, 1))
    # the reference's ratios count one batch row of fp16 (cache.py:511-539);
    # over all rows the compressed cache is the smaller one at any batch
    assert cache.memory_bytes() > 0 and cache.clean_compress_ratio_all_rows() > 1
    if B == 1:
        assert cache.compress_ratio() > 1
        assert cache.fp16_equivalent_bytes() > cache.memory_bytes()


def test_left_padded_batch_decodes_fused(cuda, monkeypatch):
    """generate() on a left-padded batch (rows of 300 and 260 prompt tokens):
    the fused calls receive the padding mask, and each one matches the fp64
    oracle with the same additive mask over the layer's own representation
    (sink, compressed, window and stream keys in position order, as
    attention.py:300-343 concatenates them)."""
    from shard_amd import Cache, attention, enable_llama_fused_attention
    model = _llama(cuda)
    assert enable_llama_fused_attention(model)
    seen, mask_bool = [], []
    inner = attention.fused_attention_compressed

    def record(q, layer, pos_q, inv, mask=None):
        out = inner(q, layer, pos_q, inv, mask)
        if layer.layer_idx == 1:
            p = int(pos_q.reshape(-1)[-1].item()) if torch.is_tensor(pos_q) else int(pos_q)
            seen.append((q.detach().cpu(), p, out.detach().cpu(), _oracle_format(layer._gpu_compressed),
                         inv.cpu(), None if mask is None else mask.detach().float().cpu()))
            mask_bool.append(mask is not None and mask.dtype == torch.bool)
        return out
    monkeypatch.setattr(attention, "fused_attention_compressed", record)
    g = torch.Generator().manual_seed(13)
    T, pad = 300, 40
    ids = torch.randint(1, VOCAB, (2, T), generator=g)
    ids[1, :pad] = 0
    am = torch.ones_like(ids)
    am[1, :pad] = 0
    cache = Cache.from_model(model)
    cache._streaming = True
    with torch.no_grad():
        model.generate(input_ids=ids.to(cuda), attention_mask=am.to(cuda), max_new_tokens=4,
                       do_sample=False, past_key_values=cache, pad_token_id=0)
    assert getattr(cache, "_fused_fallbacks", 0) == 0 and len(seen) == 3
    for i, (q, pos_q, out, ogc, inv, mask) in enumerate(seen):
        assert mask is not None
        n_keys = (ogc["sink_k"].shape[2] + ogc["n_compress"] + ogc["win_k"].shape[2]
                  + ogc.get("stream_n", 0) // 2)
        # transformers' sdpa attention masks are boolean (True = attend)
        m = torch.zeros(mask.shape).masked_fill_(mask == 0, torch.finfo(torch.float32).min) \
            if mask_bool[i] else mask
        m = m.reshape(2, -1)[:, -n_keys:]
        assert bool((m[1, :pad] < -1e30).all()) and bool((m[0] == 0).all())
        want = exact.decode_attention(q.float().numpy().reshape(2, 32, 1, 128), ogc, 8, pos_q,
                                      inv.numpy(), attn_mask=m.numpy())
        err, cos = compare(out.float().numpy().reshape(want.shape), want)
        print(f"[left-padded] step {i} max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= 2e-3 and cos >= 0.9999


def test_beam_search_decodes_fused(cuda, monkeypatch):
    """generate(num_beams=2) with the Cache: transformers reorders the cache
    between steps (Cache.reorder_cache -> CacheLayer.reorder_cache,
    cache.py:287-292), and every fused call after a reorder matches the fp64
    oracle over the reordered representation, with no fallback."""
    from shard_amd import Cache, attention, enable_llama_fused_attention
    from shard_amd import cache as cache_mod
    model = _llama(cuda)
    assert enable_llama_fused_attention(model)
    seen, reorders = [], []
    inner = attention.fused_attention_compressed

    def record(q, layer, pos_q, inv, mask=None):
        out = inner(q, layer, pos_q, inv, mask)
        if layer.layer_idx == 1:
            p = int(pos_q.reshape(-1)[-1].item()) if torch.is_tensor(pos_q) else int(pos_q)
            seen.append((q.detach().cpu(), p, out.detach().cpu(), _oracle_format(layer._gpu_compressed),
                         inv.cpu()))
        return out
    inner_reorder = cache_mod.CacheLayer.reorder_cache

    def record_reorder(self, beam_idx):
        if self.layer_idx == 1:
            reorders.append(beam_idx.detach().cpu().clone())
        return inner_reorder(self, beam_idx)
    monkeypatch.setattr(attention, "fused_attention_compressed", record)
    monkeypatch.setattr(cache_mod.CacheLayer, "reorder_cache", record_reorder)
    g = torch.Generator().manual_seed(21)
    ids = torch.randint(1, VOCAB, (1, 300), generator=g).to(cuda)
    cache = Cache.from_model(model)
    cache._streaming = True
    with torch.no_grad():
        out = model.generate(input_ids=ids, attention_mask=torch.ones_like(ids), max_new_tokens=5,
                             num_beams=2, do_sample=False, past_key_values=cache, pad_token_id=0)
    assert out.shape[0] == 1 and out.shape[1] > 300
    assert getattr(cache, "_fused_fallbacks", 0) == 0
    assert len(seen) >= 2 and len(reorders) >= 1
    for i, (q, pos_q, o, ogc, inv) in enumerate(seen):
        B = q.shape[0]
        want = exact.decode_attention(q.float().numpy().reshape(B, 32, 1, 128), ogc, 8, pos_q,
                                      inv.numpy())
        err, cos = compare(o.float().numpy().reshape(want.shape), want)
        print(f"[beam] step {i} B={B} max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= 2e-3 and cos >= 0.9999


def test_reorder_cache_selects_compressed_rows(cuda):
    from shard_amd import Cache, attention, enable_llama_fused_attention
    model = _llama(cuda)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(4)
    B = 4
    ids = torch.randint(0, VOCAB, (B, 400), generator=g).to(cuda)
    tok = torch.randint(0, VOCAB, (B, 1), generator=g).to(cuda)
    caches = []
    for _ in range(2):
        c = Cache.from_model(model)
        c._streaming = True
        with torch.no_grad():
            model(ids, past_key_values=c, use_cache=True)
            model(tok, past_key_values=c, use_cache=True)   # compress + one stream token
        caches.append(c)
    base, beam = caches
    order = torch.tensor([2, 0, 3, 1])
    layer = beam.layers[1]
    want_keys = base.layers[1].keys.index_select(0, order.to(cuda))
    want_values = base.layers[1].values.index_select(0, order.to(cuda))
    beam.reorder_cache(order)   # the HF Cache entry point: every layer
    # the reference's semantics for the dequantized rows (rebuilt lazily from
    # the selected compressed rows: no full rebuild inside the reorder)
    assert layer._keys is None and layer._needs_decompress
    assert torch.equal(layer.keys, want_keys) and torch.equal(layer.values, want_values)
    # the next fused step reads the reordered compressed rows: row b of the
    # reordered cache equals row order[b] of the original, bit for bit
    q = torch.randn(B, 32, 1, 128, generator=g).half().to(cuda)
    inv = base._rope_inv_freq
    pos = 400 + 1
    with torch.no_grad():
        a = attention.fused_attention_compressed(q[order.to(cuda)], layer, pos, inv)
        b = attention.fused_attention_compressed(q, base.layers[1], pos, inv)
    assert torch.equal(a.view(torch.int16), b[order.to(cuda)].view(torch.int16))
    # and the rebuilt K/V of the reordered layer are the original rows, reordered
    layer._needs_decompress = True
    assert torch.equal(layer.keys, base.layers[1].keys.index_select(0, order.to(cuda)))


@pytest.mark.parametrize("n_q,n_kv,hd", [(8, 2, 64), (24, 8, 128)],
                         ids=["hd64-gqa4", "llama32-3b-gqa3"])
def test_other_shapes_decode_fused(cuda, monkeypatch, n_q, n_kv, hd):
    """A head_dim-64 model (8 query heads over 2 kv heads: kv heads paired into
    128-dim heads) and Llama-3.2-3B's grouping (24 query heads over 8 kv heads,
    groups of 3), streaming: every decode step of every compressed layer takes
    the fused kernel, none falls back, and the fused call matches the fp64
    oracle over the layer's own representation."""
    from shard_amd import Cache, attention, enable_llama_fused_attention
    model = _llama(cuda, n_q=n_q, n_kv=n_kv, hd=hd, hidden=n_q * hd)
    assert enable_llama_fused_attention(model)
    seen = []
    inner = attention.fused_attention_compressed

    def record(q, layer, pos_q, inv, mask=None):
        out = inner(q, layer, pos_q, inv, mask)
        if layer.layer_idx == 1:
            p = int(pos_q.reshape(-1)[-1].item()) if torch.is_tensor(pos_q) else int(pos_q)
            seen.append((q.detach().cpu(), p, out.detach().cpu(),
                         _oracle_format(layer._gpu_compressed), inv.cpu()))
        return out
    monkeypatch.setattr(attention, "fused_attention_compressed", record)
    g = torch.Generator().manual_seed(5)
    B, T = 2, 300
    ids = torch.randint(0, VOCAB, (B, T), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (B, 3), generator=g).to(cuda)
    cache = Cache.from_model(model)
    cache._streaming = True
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        for s in range(steps.shape[1]):
            model(steps[:, s:s + 1], past_key_values=cache, use_cache=True)
    gc = cache.layers[0]._gpu_compressed
    assert gc is not None and gc["head_dim"] == hd and gc["decode_prep"] is not None
    assert getattr(cache, "_fused_fallbacks", 0) == 0
    assert len(seen) == 3
    for i, (q, pos_q, out, ogc, inv) in enumerate(seen):
        assert pos_q == T + i and ogc["stream_n"] == B * (i + 1)
        want = exact.decode_attention(q.float().numpy().reshape(B, n_q, 1, hd), ogc, n_kv, pos_q,
                                      inv.numpy())
        err, cos = compare(out.float().numpy().reshape(want.shape), want)
        print(f"[{n_q}q/{n_kv}kv hd{hd} cache] step {i} pos_q={pos_q} max_abs={err:.3e} "
              f"cos={cos:.7f}", flush=True)
        assert err <= 2e-3 and cos >= 0.9999


@pytest.mark.parametrize("n_q,n_kv,hd", [(32, 8, 128), (8, 2, 64)], ids=["hd128", "hd64-2kv"])
def test_shortest_compressible_prompt_decodes_fused(cuda, monkeypatch, n_q, n_kv, hd):
    """The shortest prompt Cache.compress takes (sink + window + 5 tokens,
    cache.py:343-344): 5 compressed tokens, so the PCA keeps at most 4
    components (rank padded to 32) and, at head_dim 64 with 2 kv heads, k-means
    has 160 subvectors for 256 centroids (cache.py:25 then draws only 160: the
    codebook has 160 rows, padded for the kernel).  Decode stays fused and
    matches the fp64 oracle."""
    from shard_amd import Cache, attention, enable_llama_fused_attention
    model = _llama(cuda, n_q=n_q, n_kv=n_kv, hd=hd, hidden=n_q * hd)
    assert enable_llama_fused_attention(model)
    seen = []
    inner = attention.fused_attention_compressed

    def record(q, layer, pos_q, inv, mask=None):
        out = inner(q, layer, pos_q, inv, mask)
        if layer.layer_idx == 1:
            p = int(pos_q.reshape(-1)[-1].item()) if torch.is_tensor(pos_q) else int(pos_q)
            seen.append((q.detach().cpu(), p, out.detach().cpu(),
                         _oracle_format(layer._gpu_compressed), inv.cpu()))
        return out
    monkeypatch.setattr(attention, "fused_attention_compressed", record)
    g = torch.Generator().manual_seed(8)
    T = 4 + 64 + 5
    ids = torch.randint(0, VOCAB, (1, T), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (1, 3), generator=g).to(cuda)
    cache = Cache.from_model(model)
    cache._streaming = True
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        for s in range(steps.shape[1]):
            model(steps[:, s:s + 1], past_key_values=cache, use_cache=True)
    gc = cache.layers[1]._gpu_compressed
    assert gc is not None and gc["n_compress"] == 5 and gc["k_coeffs_shape"][1] <= 4
    n_sub = 5 * n_kv * hd // 4
    assert gc["v_centroids_f16"].shape[0] == min(256, n_sub)
    assert getattr(cache, "_fused_fallbacks", 0) == 0 and len(seen) == 3
    for i, (q, pos_q, out, ogc, inv) in enumerate(seen):
        want = exact.decode_attention(q.float().numpy().reshape(1, n_q, 1, hd), ogc, n_kv, pos_q,
                                      inv.numpy())
        err, cos = compare(out.float().numpy().reshape(want.shape), want)
        print(f"[shortest prompt {n_q}q/{n_kv}kv hd{hd}] step {i} max_abs={err:.3e} cos={cos:.7f}",
              flush=True)
        assert err <= 2e-3 and cos >= 0.9999


@pytest.mark.parametrize("opts", [{"v_vq_codebook_size": 64},
                                  {"sink_tokens": 0, "residual_window": 16},
                                  {"sink_tokens": 8, "residual_window": 128}],
                         ids=["codebook64", "no-sink-window16", "sink8-window128"])
def test_cache_options_decode_fused(cuda, monkeypatch, opts):
    """Cache options other than the defaults: a 64-centroid codebook (k-means
    trains 64, the fused kernel takes the layer with its codebook padded to
    256 rows no index names), no sink tokens with a 16-token window, 8 sink
    tokens with a 128-token window: no step falls back, and every fused call
    matches the fp64 oracle over the layer's own representation."""
    from shard_amd import Cache, attention, enable_llama_fused_attention
    model = _llama(cuda)
    assert enable_llama_fused_attention(model)
    seen = []
    inner = attention.fused_attention_compressed

    def record(q, layer, pos_q, inv, mask=None):
        out = inner(q, layer, pos_q, inv, mask)
        if layer.layer_idx == 1:
            p = int(pos_q.reshape(-1)[-1].item()) if torch.is_tensor(pos_q) else int(pos_q)
            seen.append((q.detach().cpu(), p, out.detach().cpu(),
                         _oracle_format(layer._gpu_compressed), inv.cpu()))
        return out
    monkeypatch.setattr(attention, "fused_attention_compressed", record)
    g = torch.Generator().manual_seed(8)
    B, T = 1, 400
    ids = torch.randint(0, VOCAB, (B, T), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (B, 2), generator=g).to(cuda)
    cache = Cache.from_model(model, **opts)
    cache._streaming = True
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        for s in range(steps.shape[1]):
            model(steps[:, s:s + 1], past_key_values=cache, use_cache=True)
    gc = cache.layers[1]._gpu_compressed
    n_cent = opts.get("v_vq_codebook_size", 256)
    assert tuple(gc["v_centroids_f16"].shape) == (n_cent, 4) and gc["decode_prep"] is not None
    assert int(gc["v_indices"].max()) < n_cent
    assert gc["sink_k"].shape[2] == opts.get("sink_tokens", 4)
    assert gc["win_k"].shape[2] == opts.get("residual_window", 64)
    assert getattr(cache, "_fused_fallbacks", 0) == 0 and len(seen) == 2
    n_q, n_kv, hd = 32, 8, 128
    for i, (q, pos_q, out, ogc, inv) in enumerate(seen):
        want = exact.decode_attention(q.float().numpy().reshape(B, n_q, 1, hd), ogc, n_kv, pos_q,
                                      inv.numpy())
        err, cos = compare(out.float().numpy().reshape(want.shape), want)
        print(f"[{opts}] step {i} max_abs={err:.3e} cos={cos:.7f}", flush=True)
        assert err <= 2e-3 and cos >= 0.9999


def test_vq_group_8_falls_back(cuda):
    """Cache(v_vq_group_size=8): V subvectors of 8 values (k-means over 8-dim
    rows), which the fused value stage does not take: every decode step of a
    compressed layer runs the original forward over kv_reconstruct's K/V
    (counted, with the reason), with the unpatched forward's logits."""
    from transformers.models.llama.modeling_llama import LlamaAttention
    from shard_amd import Cache, enable_llama_fused_attention
    model = _llama(cuda)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, VOCAB, (1, 400), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (1, 2), generator=g).to(cuda)

    def run():
        c = Cache.from_model(model, v_vq_group_size=8)
        c._streaming = True
        out = []
        with torch.no_grad():
            model(ids, past_key_values=c, use_cache=True)
            for s in range(steps.shape[1]):
                out.append(model(steps[:, s:s + 1], past_key_values=c, use_cache=True).logits.float())
        return torch.cat(out, 1), c

    got, cache = run()
    gc = cache.layers[0]._gpu_compressed
    assert gc is not None and tuple(gc["v_centroids_f16"].shape) == (256, 8)
    assert gc["decode_prep"] is None and "subvectors of 8" in gc["decode_refusal"]
    assert cache._fused_fallbacks == 2 * steps.shape[1] - 1
    patched = LlamaAttention.forward
    try:
        LlamaAttention.forward = patched.__wrapped__
        want, _ = run()
    finally:
        LlamaAttention.forward = patched
    assert torch.isfinite(got).all()
    assert torch.equal(got, want)


def test_head_dim_64_odd_kv_heads_fall_back(cuda):
    """A shape the fused kernel does not take (head_dim 64 with one kv head:
    no pair): Cache.compress builds the format without the fused operands,
    decode steps run the original forward over kv_reconstruct's K/V, and each
    layer-step is counted."""
    from transformers.models.llama.modeling_llama import LlamaAttention
    from shard_amd import Cache, enable_llama_fused_attention
    model = _llama(cuda, n_q=8, n_kv=1, hd=64, hidden=512)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, VOCAB, (1, 300), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (1, 2), generator=g).to(cuda)

    def run():
        c = Cache.from_model(model)
        c._streaming = True
        out = []
        with torch.no_grad():
            model(ids, past_key_values=c, use_cache=True)
            for s in range(steps.shape[1]):
                out.append(model(steps[:, s:s + 1], past_key_values=c, use_cache=True).logits.float())
        return torch.cat(out, 1), c

    got, cache = run()
    gc = cache.layers[0]._gpu_compressed
    assert gc is not None and gc["head_dim"] == 64 and gc["decode_prep"] is None
    # a 64-dim K: the bit budget drops every component, which the format keeps
    # with zero coefficients (the reference's keep = len(k_alloc))
    assert gc["k_alloc"] == [0] * 64 and gc["k_coeffs_shape"][1] == 64
    # layer 0 of the first decode step is not compressed yet when the forward
    # routes it (its own cache update compresses every layer), so it is not a
    # fallback; every later layer-step is
    assert cache._fused_fallbacks == 2 * steps.shape[1] - 1
    assert "head_dim=64" in cache._last_fused_fallback and "n_kv=1" in cache._last_fused_fallback
    patched = LlamaAttention.forward
    try:
        LlamaAttention.forward = patched.__wrapped__
        want, _ = run()
    finally:
        LlamaAttention.forward = patched
    assert torch.isfinite(got).all()
    assert torch.equal(got, want)


def test_rank_above_256_falls_back(cuda):
    """A Cache with max_rank_k = 320 and a budget that keeps every component
    (k_target_cr = 4; 4 kv heads of 128 dims): compression keeps 320
    components (the fp32 projection in two launches), the fused call (ranks up
    to 256) does not take the layer, and decode steps run the original forward over
    kv_reconstruct's K/V, counted, with the unpatched forward's logits."""
    from transformers.models.llama.modeling_llama import LlamaAttention
    from shard_amd import Cache, enable_llama_fused_attention
    model = _llama(cuda, n_q=16, n_kv=4, hd=128, hidden=2048)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, VOCAB, (1, 600), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (1, 2), generator=g).to(cuda)

    def run():
        c = Cache.from_model(model, k_target_cr=4.0, max_rank_k=320)
        c._streaming = True
        out = []
        with torch.no_grad():
            model(ids, past_key_values=c, use_cache=True)
            for s in range(steps.shape[1]):
                out.append(model(steps[:, s:s + 1], past_key_values=c, use_cache=True).logits.float())
        return torch.cat(out, 1), c

    got, cache = run()
    gc = cache.layers[0]._gpu_compressed
    assert gc is not None and gc["rank"] == 320 and gc["decode_prep"] is None
    assert cache._fused_fallbacks == 2 * steps.shape[1] - 1
    assert "rank=320" in cache._last_fused_fallback
    patched = LlamaAttention.forward
    try:
        LlamaAttention.forward = patched.__wrapped__
        want, _ = run()
    finally:
        LlamaAttention.forward = patched
    assert torch.isfinite(got).all()
    assert torch.equal(got, want)
