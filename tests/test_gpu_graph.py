"""A decode step captured in a HIP graph (shard_amd.graph.DecodeGraph) against
eager decode steps of the same random-init Llama on an identical cache state.
The graph's attention calls read the stream count and the position from
device counters and plan for the reserved stream rows, so their split plan
differs from the eager calls': the logits agree to fp32 summation order, and
layer 0's stream codes (its K/V do not depend on attention) are bit-identical,
which also shows that every replay appended its token to the next row."""
import pytest
import torch

pytestmark = pytest.mark.gpu

VOCAB = 512


def _model(dev, n_q=8, n_kv=2, hd=128):
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=VOCAB, hidden_size=n_q * hd, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=n_q, num_key_value_heads=n_kv,
                      head_dim=hd, max_position_embeddings=4096, rope_theta=500000.0)
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).to(dev, torch.float16).eval()


def _prefilled(model, ids, first, qjl):
    """Prefill, then one eager decode step (it compresses the layers and
    starts the stream)."""
    from shard import Cache
    cache = Cache.from_model(model)
    cache._streaming = True
    cache._stream_qjl = qjl
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
        model(first, past_key_values=cache, use_cache=True)
    return cache


def _compare(got, want, what):
    err = (got - want).abs().max().item()
    cos = torch.nn.functional.cosine_similarity(got.flatten(), want.flatten(), dim=0).item()
    scale = want.abs().max().item()
    print(f"{what}: max|diff| {err:.3e} (scale {scale:.3f}) cos {cos:.7f}", flush=True)
    assert err <= 1e-2 * max(scale, 1.0) and cos >= 0.9999, (what, err, cos)


@pytest.mark.parametrize("B,qjl,kernel,shape", [(1, False, 0, (8, 2, 128)), (3, False, 0, (8, 2, 128)),
                                                (2, True, 0, (8, 2, 128)), (2, False, 2, (8, 2, 128)),
                                                (2, False, 0, (8, 2, 64)), (2, False, 0, (12, 4, 128))],
                         ids=["b1", "b3", "b2-qjl", "b2-tok", "b2-hd64", "b2-gqa3"])
def test_decode_graph_matches_eager_steps(cuda, B, qjl, kernel, shape):
    """Also a head_dim-64 model (kv heads paired) and 3 query heads per kv head."""
    from shard import enable_llama_fused_attention
    from shard_amd.graph import DecodeGraph
    model = _model(cuda, *shape)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(B)
    ids = torch.randint(0, VOCAB, (B, 300), generator=g).to(cuda)
    first = torch.randint(0, VOCAB, (B, 1), generator=g).to(cuda)
    feed = torch.randint(0, VOCAB, (B, 12), generator=g).to(cuda)  # teacher-forced tokens
    cache_e = _prefilled(model, ids, first, qjl)
    cache_g = _prefilled(model, ids, first, qjl)
    cache_e._decode_kernel = cache_g._decode_kernel = kernel  # 2: the token-tiled kernel
    steps = feed.shape[1]

    want = []
    with torch.no_grad():
        for s in range(steps):
            want.append(model(feed[:, s:s + 1], past_key_values=cache_e, use_cache=True).logits[:, -1].float())
    dg = DecodeGraph(model, cache_g, feed[:, :1], max_steps=steps)
    got = []
    for s in range(steps):
        tok = dg.step(feed[:, s:s + 1])
        got.append(dg.logits.float().clone())
        assert torch.equal(tok, got[-1].argmax(-1))
    for s in range(steps):
        _compare(got[s], want[s], f"[graph B={B} qjl={qjl} kernel={kernel}] step {s}")
    with pytest.raises(RuntimeError):
        dg.step()

    # the host counters followed the replays; layer 0's stream rows are the eager ones
    for le, lg in zip(cache_e.layers, cache_g.layers):
        assert lg._gpu_compressed["stream_n"] == le._gpu_compressed["stream_n"] == (steps + 1) * B
        assert lg._seq_len == le._seq_len
    ge, gg = cache_e.layers[0]._gpu_compressed, cache_g.layers[0]._gpu_compressed
    n = steps + 1
    names = ["k_idx_buf", "v_idx_buf", "k_norm_buf", "v_norm_buf", "k_deq_buf", "v_deq_buf"]
    if qjl:
        names += ["k_qsign_buf", "v_qsign_buf", "k_qscale_buf", "v_qscale_buf"]
    for name in names:
        assert torch.equal(gg[name][:n].view(torch.uint8), ge[name][:n].view(torch.uint8)), name

    # back to eager steps on the graph's cache
    dg.close()
    nxt = torch.randint(0, VOCAB, (B, 1), generator=g).to(cuda)
    with torch.no_grad():
        a = model(nxt, past_key_values=cache_e, use_cache=True).logits[:, -1].float()
        b = model(nxt, past_key_values=cache_g, use_cache=True).logits[:, -1].float()
    _compare(b, a, f"[graph B={B} qjl={qjl} kernel={kernel}] eager step after close")


def test_decode_graph_greedy_feeds_its_own_tokens(cuda):
    """Without supplied tokens each replay decodes the previous step's argmax:
    the same tokens as eager greedy steps from the same state."""
    from shard import enable_llama_fused_attention
    from shard_amd.graph import DecodeGraph
    model = _model(cuda)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, VOCAB, (2, 300), generator=g).to(cuda)
    first = torch.randint(0, VOCAB, (2, 1), generator=g).to(cuda)
    cache_e = _prefilled(model, ids, first, False)
    cache_g = _prefilled(model, ids, first, False)
    start = torch.randint(0, VOCAB, (2, 1), generator=g).to(cuda)
    steps = 8
    dg = DecodeGraph(model, cache_g, start, max_steps=steps)
    got = [dg.step() for _ in range(steps)]
    cur, want, agree = start, [], 0
    with torch.no_grad():
        for s in range(steps):
            logits = model(cur, past_key_values=cache_e, use_cache=True).logits[:, -1]
            nxt = logits.argmax(-1)
            want.append(nxt)
            if not torch.equal(nxt, got[s]):
                # a near-tie may flip under the graph's other summation order;
                # then the two runs decode different tokens from here on
                top2 = logits.float().topk(2, dim=-1).values
                assert (top2[:, 0] - top2[:, 1]).min().item() < 5e-2, s
                break
            agree += 1
            cur = nxt.view(-1, 1)
    print(f"[graph greedy] {agree} of {steps} steps agree", flush=True)
    assert agree >= 1
    dg.close()


def test_decode_graph_keeps_its_workspace_when_another_call_grows_it(cuda):
    """The captured attention calls write their partial rows into the device's
    shared decode workspace.  An eager call elsewhere that needs a larger one
    replaces the shared buffer; the graph still holds the one it captured, so
    that memory is not handed out again and later replays match eager steps."""
    from shard import enable_llama_fused_attention
    from shard_amd import attention
    from shard_amd.graph import DecodeGraph
    model = _model(cuda)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(21)
    ids = torch.randint(0, VOCAB, (1, 300), generator=g).to(cuda)
    first = torch.randint(0, VOCAB, (1, 1), generator=g).to(cuda)
    feed = torch.randint(0, VOCAB, (1, 6), generator=g).to(cuda)
    cache_e = _prefilled(model, ids, first, False)
    cache_g = _prefilled(model, ids, first, False)
    want = []
    with torch.no_grad():
        for s in range(feed.shape[1]):
            want.append(model(feed[:, s:s + 1], past_key_values=cache_e, use_cache=True).logits[:, -1].float())
    dg = DecodeGraph(model, cache_g, feed[:, :1], max_steps=feed.shape[1])
    key = (cuda.type, cuda.index if cuda.index is not None else torch.cuda.current_device())
    for s in range(feed.shape[1]):
        if s == 3:  # captured at step 1, replayed at step 2
            old = attention._workspaces[key]
            old_ptr, old_n = old.data_ptr(), old.numel()
            del old
            attention._workspace(cuda, 4 * old_n)      # another call grows the shared buffer
            assert attention._workspaces[key].data_ptr() != old_ptr
            junk = torch.full((old_n,), 0x7F, dtype=torch.uint8, device=cuda)
            assert junk.data_ptr() != old_ptr, "the captured workspace was freed and reused"
        dg.step(feed[:, s:s + 1])
        _compare(dg.logits.float(), want[s], f"[graph workspace] step {s}")
    dg.close()


def test_decode_graph_refuses_reorder_while_open(cuda):
    from shard import enable_llama_fused_attention
    from shard_amd.graph import DecodeGraph
    model = _model(cuda)
    assert enable_llama_fused_attention(model)
    g = torch.Generator().manual_seed(22)
    ids = torch.randint(0, VOCAB, (2, 300), generator=g).to(cuda)
    first = torch.randint(0, VOCAB, (2, 1), generator=g).to(cuda)
    cache = _prefilled(model, ids, first, False)
    dg = DecodeGraph(model, cache, first, max_steps=3)
    with pytest.raises(RuntimeError):
        cache.reorder_cache(torch.tensor([1, 0], device=cuda))
    dg.close()
    cache.reorder_cache(torch.tensor([1, 0], device=cuda))
