"""Greedy decode steps of a Llama model over a shard Cache, captured once in a
HIP graph and replayed per token.

The reference decodes through `generate()`, one Python-driven step per token
(attention.py:345-414 patched into every layer).  A captured step replays the
whole model's launches without the host: the embedding, every layer's
projections, the fused RoPE + stream append (`shard_rope_stream_append_dev`),
the fused decode attention (`shard_decode_attn` with `n_stream_dev`), the MLPs,
the LM head and the argmax that feeds the next step.  What changes between
steps lives in device memory: the stream row the token goes to, the number of
stream rows attention reads, the position and the input ids.  The host keeps
the cache's own counters (stream length, sequence length) in step with the
replays, so the cache can go back to eager steps afterwards.

Requirements: a compressed, streaming cache whose every layer takes the fused
kernel, rows of equal length (no attention mask: refused when the cache's last
eager decode step was masked) and transformers' Llama attention patched by
`enable_llama_fused_attention`.  While the graph is open the cache's device
tensors must keep their addresses: `reorder_cache` raises, and eager appends
go through the graph's rows.  The graph keeps the shared decode workspace it
captured alive.  The work plan of every captured call (its kernel choice and
split balance) covers the stream rows of all `max_steps` steps from step 0.
"""
import torch

from .attention import _workspaces, fused_supported


class DecodeGraph:
    """Runs up to `max_steps` decode steps: the first one eagerly (it sizes
    the workspaces), the second one captured and replayed, every later one
    replayed.  `next_ids` (B, 1) int64 on the device are the tokens of the
    first step; each step returns the (B,) greedy tokens it produced, which
    are also the next step's input unless `step(ids)` supplies other ones."""

    def __init__(self, model, cache, next_ids, max_steps):
        from .cache import Cache
        if not isinstance(cache, Cache):
            raise TypeError("DecodeGraph needs a shard Cache")
        if not (cache._compressed and cache._streaming):
            raise ValueError("DecodeGraph needs a compressed cache in streaming mode")
        if getattr(cache, "_graph", None) is not None:
            raise ValueError("the cache already runs a decode graph")
        mask = getattr(cache, "_last_attn_mask", None)
        if mask is not None and bool((mask != 0).any()):
            # the replays attend without a mask; eager steps that were masked
            # (a left-padded batch) would attend to pad tokens under the graph
            raise ValueError("the cache's last decode step attended with a padding mask; "
                             "a decode graph needs rows of equal length")
        if next_ids.dim() != 2 or next_ids.shape[1] != 1 or not next_ids.is_cuda:
            raise ValueError("next_ids must be (B, 1) on the GPU")
        if max_steps < 1:
            raise ValueError("max_steps must be positive")
        B = next_ids.shape[0]
        n_q = model.config.num_attention_heads
        layers = cache.layers
        stream_rows = set()
        for layer in layers:
            gc = getattr(layer, "_gpu_compressed", None)
            if gc is None or not fused_supported(gc, n_q):
                raise ValueError(f"layer {layer.layer_idx} does not take the fused decode kernel")
            if gc.get("stream_n", 0) % B:
                raise ValueError("stream rows do not match the batch")
            stream_rows.add(gc.get("stream_n", 0) // B)
        if len(stream_rows) != 1 or len({layer._seq_len for layer in layers}) != 1:
            raise ValueError("every layer must hold the same tokens")
        s0 = stream_rows.pop()
        dev = next_ids.device
        self.model, self.cache, self.B = model, cache, B
        self.max_steps, self.steps = max_steps, 0
        # stream rows the steps can fill: the plan of every captured attention
        # call covers them, the appends past them write nothing
        self.cap = s0 + max_steps
        for layer in layers:
            gc = layer._gpu_compressed
            D, G = gc["head_dim"], gc["n_kv"]
            layer._stream_rows(B, G, D, dev, min_cap=self.cap)
        # rows = [stream rows before the step (the append's row), after it]
        self.rows = torch.tensor([s0, s0 + 1], dtype=torch.int32, device=dev)
        self.pos_ids = torch.full((1, 1), layers[0]._seq_len, dtype=torch.int64, device=dev)
        self.pos = self.pos_ids.view(-1)
        self.ids = next_ids.clone()
        self.graph = None
        self.next = None
        self.logits = None
        self._pinned = None
        cache._graph = self

    def _body(self):
        out = self.model(input_ids=self.ids, position_ids=self.pos_ids,
                         past_key_values=self.cache, use_cache=True)
        logits = out.logits[:, -1]
        nxt = logits.argmax(-1)
        self.ids.copy_(nxt.view(-1, 1))
        self.rows.add_(1)
        self.pos.add_(1)
        return logits, nxt

    def _advance_host(self):
        """The cache's host counters after one replayed step (what the eager
        step's fused_rope_append does)."""
        for layer in self.cache.layers:
            gc = layer._gpu_compressed
            gc["stream_n"] = gc.get("stream_n", 0) + self.B
            layer._seq_len += 1
            layer._needs_decompress = True

    @torch.no_grad()
    def step(self, ids=None):
        """One decode step; ids (B, 1) int64 overrides the input tokens."""
        if self.cache._graph is not self:
            raise RuntimeError("this decode graph is closed")
        if self.steps >= self.max_steps:
            raise RuntimeError(f"the decode graph holds {self.max_steps} steps")
        if ids is not None:
            self.ids.copy_(ids.view(-1, 1))
        if self.steps == 0:
            self.logits, self.next = self._body()
        elif self.graph is None:
            # capture: the Python side runs once (and moves the host counters
            # one step on), the launches run at the replay below
            torch.cuda.synchronize()
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph):
                self.logits, self.next = self._body()
            # the captured attention calls hold the address of the device's
            # shared decode workspace; a later eager call that needs a larger
            # one replaces it in the dict, so the graph keeps this one alive
            self._pinned = dict(_workspaces)
            self.graph.replay()
        else:
            self._advance_host()
            self.graph.replay()
        self.steps += 1
        return self.next.clone()

    def close(self):
        """Back to eager decode steps on the cache."""
        if self.cache._graph is self:
            self.cache._graph = None
        self.graph = None
        self._pinned = None
