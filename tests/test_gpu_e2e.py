"""End to end on the GPU: a random-init Llama (head_dim 128, GQA 4) with the
shard Cache, decode steps through the patched LlamaAttention.forward (fused HIP
kernel) against the same model and cache type on the original forward, where
the cache hands back dequantized K/V (shard_kv_reconstruct) to the model's own
attention.  Both read the same compressed representation, so their logits agree
to fp16-level tolerance; this also checks the routing of the patched forward
(attention.py:345-414) and the first-decode compression trigger
(cache.py:150-151) as HF drives them."""
import pytest
import torch

pytestmark = pytest.mark.gpu

VOCAB = 512


def _model(dev):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=VOCAB, hidden_size=1024, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=8, num_key_value_heads=2,
                      head_dim=128, max_position_embeddings=4096, rope_theta=500000.0)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(dev, torch.float16).eval()


def _run(model, ids, steps, streaming, bits=8, qjl=False, lazy=True):
    from shard import Cache
    cache = Cache.from_model(model)
    cache._streaming = streaming
    cache._stream_bits = bits
    cache._stream_qjl = qjl
    cache._lazy_per_layer = lazy
    logits = []
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        for s in range(steps.shape[1]):
            out = model(steps[:, s:s + 1], past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1].float())
    return torch.stack(logits, 1), cache


@pytest.mark.parametrize("streaming,bits,qjl", [(True, 8, False), (False, 8, False),
                                                (True, 4, True)])
def test_llama_fused_decode_matches_unfused(cuda, streaming, bits, qjl):
    from transformers.models.llama.modeling_llama import LlamaAttention
    from shard import enable_llama_fused_attention
    model = _model(cuda)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, VOCAB, (1, 600), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (1, 5), generator=g).to(cuda)   # teacher-forced decode tokens
    assert enable_llama_fused_attention(model)
    patched = LlamaAttention.forward
    try:
        LlamaAttention.forward = patched.__wrapped__
        ref, cache_ref = _run(model, ids, steps, streaming, bits, qjl)
    finally:
        LlamaAttention.forward = patched
    got, cache = _run(model, ids, steps, streaming, bits, qjl)
    print(f"[e2e streaming={streaming} bits={bits} qjl={qjl}] logits scale {ref.abs().max().item():.3f}")
    for layer in cache.layers:                       # fused path: nothing was dequantized
        assert layer._gpu_compressed is not None and layer._keys is None
    # original path: dequantized K/V (lazy eviction keeps them for the last layer only)
    assert cache_ref.layers[-1]._keys is not None
    if streaming:
        from shard_amd import ops
        gc = cache.layers[0]._gpu_compressed
        s = steps.shape[1]
        assert gc["stream_n"] == s and gc["stream_codebook"].numel() == 1 << bits
        assert ("k_qsign_buf" in gc) == qjl
        # the fp16 rows the decode kernel reads are the reference dequantization
        # (cache.py:243-279) of the stored codes, QJL term included
        for p in ("k", "v"):
            extra = (gc[p + "_qsign_buf"][:s], gc[p + "_qscale_buf"][:s]) if qjl else ()
            y = ops.stream_dequant(gc[p + "_idx_buf"][:s], gc[p + "_norm_buf"][:s], gc["signs"],
                                   gc["stream_codebook"], *extra)
            assert torch.equal(y.view(torch.int16), gc[p + "_deq_buf"][:s].view(torch.int16))
    err = (got - ref).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
    scale = ref.abs().max().item()
    print(f"[e2e streaming={streaming} bits={bits} qjl={qjl}] max|diff| {err:.3e} (scale {scale:.3f}) cos {cos:.6f}")
    assert err <= 2e-2 * max(scale, 1.0)
    assert cos >= 0.9999


@pytest.mark.parametrize("streaming", [True, False])
def test_multi_token_extend_after_compression(cuda, streaming):
    """q_len > 1 after compression (the perplexity-style extend of the
    reference's benchmark.py:478-482): the chunk is appended to the stream (or
    the fp16 decode tokens) and the model's own attention runs over the
    reconstructed K/V with a causal mask (cache.py:149-191).  Its logits agree
    with the same tokens fed one at a time through the fused kernel."""
    from shard import Cache, enable_llama_fused_attention
    model = _model(cuda)
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, VOCAB, (1, 500), generator=g).to(cuda)
    chunk = torch.randint(0, VOCAB, (1, 8), generator=g).to(cuda)
    assert enable_llama_fused_attention(model)
    step, _ = _run(model, ids, chunk, streaming)
    cache = Cache.from_model(model)
    cache._streaming = streaming
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        out = model(chunk, past_key_values=cache, use_cache=True).logits.float()
    assert cache._compressed and cache.get_seq_length() == 508
    gc = cache.layers[0]._gpu_compressed
    assert gc["stream_n"] == 8 if streaming else gc["decode_k"].shape[2] == 8
    err = (out - step).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(out.flatten(), step.flatten(), dim=0).item()
    scale = step.abs().max().item()
    print(f"[extend streaming={streaming}] max|diff| {err:.3e} (scale {scale:.3f}) cos {cos:.6f}")
    assert err <= 2e-2 * max(scale, 1.0)
    assert cos >= 0.9999


def test_lazy_per_layer_off_keeps_every_layers_kv(cuda):
    """_lazy_per_layer (cache.py:74-85): on the original forward the cache hands
    back dequantized K/V; with the knob on only the last layer read keeps them,
    with it off every layer does.  The logits are the same bits either way."""
    from transformers.models.llama.modeling_llama import LlamaAttention
    model = _model(cuda)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, VOCAB, (1, 500), generator=g).to(cuda)
    steps = torch.randint(0, VOCAB, (1, 3), generator=g).to(cuda)
    fwd = LlamaAttention.forward
    try:
        LlamaAttention.forward = getattr(fwd, "__wrapped__", fwd)  # the original forward
        lazy, c_lazy = _run(model, ids, steps, True, lazy=True)
        keep, c_keep = _run(model, ids, steps, True, lazy=False)
    finally:
        LlamaAttention.forward = fwd
    assert torch.equal(lazy, keep)
    assert all(l._keys is not None for l in c_keep.layers)
    assert [l._keys is not None for l in c_lazy.layers] == [False] * (len(c_lazy.layers) - 1) + [True]
