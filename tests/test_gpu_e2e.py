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


def _run(model, ids, steps, streaming):
    from shard import Cache
    cache = Cache.from_model(model)
    cache._streaming = streaming
    logits = []
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        for s in range(steps.shape[1]):
            out = model(steps[:, s:s + 1], past_key_values=cache, use_cache=True)
            logits.append(out.logits[:, -1].float())
    return torch.stack(logits, 1), cache


@pytest.mark.parametrize("streaming", [True, False])
def test_llama_fused_decode_matches_unfused(cuda, streaming):
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
        ref, cache_ref = _run(model, ids, steps, streaming)
    finally:
        LlamaAttention.forward = patched
    got, cache = _run(model, ids, steps, streaming)
    print(f"[e2e streaming={streaming}] logits scale {ref.abs().max().item():.3f}")
    for layer in cache.layers:                       # fused path: nothing was dequantized
        assert layer._gpu_compressed is not None and layer._keys is None
    # original path: dequantized K/V (lazy eviction keeps them for the last layer only)
    assert cache_ref.layers[-1]._keys is not None
    if streaming:
        assert cache.layers[0]._gpu_compressed["stream_n"] == steps.shape[1]
    err = (got - ref).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten(), ref.flatten(), dim=0).item()
    scale = ref.abs().max().item()
    print(f"[e2e streaming={streaming}] max|diff| {err:.3e} (scale {scale:.3f}) cos {cos:.6f}")
    assert err <= 2e-2 * max(scale, 1.0)
    assert cos >= 0.9999
