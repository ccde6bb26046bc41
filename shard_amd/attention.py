"""Fused compressed-KV decode attention and the Llama integration.

fused_attention_compressed (attention.py:270-343 of the reference) computes
softmax(q.K^T/sqrt(d)).V over [sink, compressed, window, decode, stream]
without materializing the compressed K or V: one HIP split kernel rebuilds
no-RoPE keys on chip from int4 PCA coefficients, scores them with the
relative-delta RoPE identity

    pair_i(D) = (a_i c_i + b_i d_i) cos(theta_i D) + (b_i c_i - a_i d_i) sin(theta_i D)

(q_n = [a, b] = undo-RoPE(q, pos_q), k_n = [c, d], D = pos_t - pos_q), and
accumulates the VQ values in Hadamard-rotated space, together with the fp16
segments and the 8-bit stream in one online softmax; each split applies ch and
one inverse Hadamard to its partial row, and a merge kernel combines the rows.
"""
import torch

from . import ops
from ._lib import ShardHipError

_workspaces = {}


def _workspace(device, nbytes):
    key = (device.type, device.index)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def fused_attention_compressed(q_rope, layer, pos_q, inv_freq, attn_mask=None):
    """q_rope (B, n_q, 1, hd) post-RoPE; returns (B, n_q, 1, hd) in q's dtype,
    or None when the layer is not compressed (attention.py:270-274).  pos_q is
    an int or a device int64 tensor whose last element is the position."""
    gc = getattr(layer, "_gpu_compressed", None)
    if gc is None:
        return None
    B, n_q, s, hd = q_rope.shape
    if s != 1:
        return None
    if not fused_supported(gc, n_q):
        return None
    q = q_rope.reshape(B, n_q, hd)
    if q.dtype != torch.float16:
        q = q.to(torch.float16)
    if not q.is_contiguous():
        q = q.contiguous()
    c = layer._cache_ref
    inv = gc["inv_freq_dev"]
    if inv_freq is not None and inv_freq is not getattr(c, "_rope_inv_freq", None):
        inv = inv_freq.to(q.device, torch.float32).contiguous()
    stream_n = gc.get("stream_n", 0) // B if gc.get("stream_n", 0) else 0
    dec = (gc["decode_k"], gc["decode_v"]) if "decode_k" in gc else None
    mask = None
    if attn_mask is not None:
        # the reference adds the mask to the scores (attention.py:314); a
        # boolean mask (transformers' sdpa masks: True = attend) is taken as
        # the additive mask it stands for, not as 1.0 / 0.0 added to scores
        mask = ops.additive_mask(attn_mask).reshape(B, -1)[
            :, -(gc["sink_k"].shape[2] + gc["n_compress"] + gc["win_k"].shape[2] + stream_n +
                 (dec[0].shape[2] if dec else 0)):]
    n_splits = getattr(c, "_n_splits", 0)
    stream_n_dev = None
    graph = getattr(c, "_graph", None)
    if graph is None:
        c._last_attn_mask = mask  # checked once when a decode graph opens
    if graph is not None:
        # a captured decode step: the stream count and the position come from
        # the graph's device counters, the plan covers the reserved rows.  The
        # graph runs the model without an attention mask (rows of equal
        # length), so the causal mask transformers builds for the one query
        # token keeps every key: the call takes none.
        mask = None
        stream_n, stream_n_dev, pos_q = graph.cap, graph.rows[1:2], graph.pos
    call = gc.get("_decode_call")
    if call is None or call.args.batch != B or call.args.n_q_heads != n_q:
        call = ops.make_decode_args(q, gc, pos_q, inv, mask=mask, n_splits=n_splits,
                                    stream_n=stream_n, decode_kv=dec, stream_n_dev=stream_n_dev)
        gc["_decode_call"] = call  # the layer's argument block, refreshed per step
    else:
        call.refresh(q, gc, pos_q, inv, mask, n_splits, None, stream_n, dec, stream_n_dev)
    call.args.kernel = int(getattr(c, "_decode_kernel", 0))
    # the device's shared workspace; the size query runs only when the library
    # reports it too small (before launching anything)
    try:
        out = ops.decode_attn(call, _workspace(q.device, 0), allocate=False)
    except ShardHipError as exc:
        if exc.code != ops.ERR_WORKSPACE:
            raise
        out = ops.decode_attn(call, _workspace(q.device, call.workspace_bytes()), allocate=False)
    call.step = []  # drop this step's tensors (the output is returned)
    return out.view(B, n_q, 1, hd).to(q_rope.dtype)


def fused_supported(gc, n_q: int) -> bool:
    """Whether the fused kernel takes this compressed layer with n_q query heads."""
    return (gc.get("decode_prep") is not None
            and ops.decode_supported(gc.get("head_dim", 0), n_q, gc.get("n_kv", 0),
                                     gc.get("rank_pad", 0)))


def fused_attention_compressed_full(q_rope, layer, pos_q, inv_freq, attn_mask=None):
    """The reference's opt-in single-pass variant (attention.py:183-267).  The HIP
    kernel is already single-pass over every segment, so both entry points run it."""
    return fused_attention_compressed(q_rope, layer, pos_q, inv_freq, attn_mask)


def enable_llama_fused_attention(model=None):
    """Patch LlamaAttention.forward process-wide so decode steps (q_len == 1) on a
    compressed shard Cache layer go through the fused HIP kernel; everything else
    calls the original forward (attention.py:345-414).  Returns False when the
    transformers Llama module is unavailable."""
    from .cache import Cache
    try:
        from transformers.models.llama.modeling_llama import LlamaAttention, apply_rotary_pos_emb
    except ImportError:
        return False
    if getattr(LlamaAttention.forward, "_shard_amd_patched", False):
        return True
    original = LlamaAttention.forward

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                past_key_values=None, cache_position=None, **kwargs):
        is_shard = isinstance(past_key_values, Cache)
        layer = past_key_values.layers[self.layer_idx] if is_shard else None
        gc = getattr(layer, "_gpu_compressed", None) if layer is not None else None
        fuse = (gc is not None and hidden_states.shape[1] == 1
                and past_key_values._rope_inv_freq is not None)
        if fuse and not fused_supported(gc, self.config.num_attention_heads):
            # a shape the fused kernel does not take (head_dim other than 128 or
            # 64, an odd kv head count at 64, query groups it cannot split,
            # rank above 192): the original forward runs on the rebuilt fp16
            # K/V (layer.keys / values); counted
            past_key_values._fused_fallbacks = getattr(past_key_values, "_fused_fallbacks", 0) + 1
            past_key_values._last_fused_fallback = (
                f"head_dim={gc.get('head_dim')} n_q={self.config.num_attention_heads} "
                f"n_kv={gc.get('n_kv')} rank={gc.get('rank_pad')}"
                + (f" ({gc['decode_refusal']})" if gc.get("decode_refusal") else ""))
            fuse = False
        if not fuse:
            if cache_position is not None:
                kwargs["cache_position"] = cache_position
            return original(self, hidden_states, position_embeddings, attention_mask,
                            past_key_values, **kwargs)
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        k = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        if (past_key_values._streaming and not getattr(past_key_values, "offloading", False)
                and cos.shape[0] in (1, q.shape[0])
                and all(t.dtype == torch.float16 for t in (q, k, v, cos, sin))):
            # apply_rotary_pos_emb + update(k, v) of a streaming layer in one
            # launch, with the same fp16 arithmetic (attention.py:376-381)
            q = layer.fused_rope_append(q, k, v, cos, sin).unsqueeze(2)
        else:
            q, k = apply_rotary_pos_emb(q, k, cos, sin)
            past_key_values._fused_decode_update = True
            try:
                past_key_values.update(k, v, self.layer_idx,
                                       {"sin": sin, "cos": cos, "cache_position": cache_position})
            finally:
                past_key_values._fused_decode_update = False
        # the reference reads cache_position[-1].item() (attention.py:383); a
        # device int64 position goes to the kernel as a pointer instead, so the
        # step needs no host read-back
        if cache_position is None:
            pos_q = past_key_values.get_seq_length() - 1
        elif cache_position.is_cuda and cache_position.dtype == torch.int64:
            pos_q = cache_position.reshape(-1)[-1:]
        else:
            pos_q = int(cache_position.reshape(-1)[-1].item())
        out = None
        if getattr(past_key_values, "_full_fused", False):
            past_key_values._full_fused_attempts = getattr(past_key_values, "_full_fused_attempts", 0) + 1
            try:
                out = fused_attention_compressed_full(q, layer, pos_q, past_key_values._rope_inv_freq,
                                                      attention_mask)
                if out is not None:
                    past_key_values._full_fused_hits = getattr(past_key_values, "_full_fused_hits", 0) + 1
            except Exception as exc:  # counted, then the default fused path runs
                past_key_values._full_fused_errors = getattr(past_key_values, "_full_fused_errors", 0) + 1
                past_key_values._last_full_fused_error = repr(exc)
                out = None
        if out is None:
            out = fused_attention_compressed(q, layer, pos_q, past_key_values._rope_inv_freq,
                                             attention_mask)
        if out is None:
            if cache_position is not None:
                kwargs["cache_position"] = cache_position
            return original(self, hidden_states, position_embeddings, attention_mask,
                            past_key_values, **kwargs)
        out = out.transpose(1, 2).contiguous().view(*input_shape, -1)
        return self.o_proj(out), None

    forward._shard_amd_patched = True
    forward.__wrapped__ = original
    LlamaAttention.forward = forward
    return True
