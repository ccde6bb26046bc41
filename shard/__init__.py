"""Drop-in import name of the reference package: ``from shard import Cache, ...``
resolves to the MI355X implementation in shard_amd, and so do the submodule
paths the reference's own scripts import (``shard.cache``, ``shard.attention``,
``shard.rope``; benchmarks/benchmark.py:43-45)."""
from shard_amd import Cache, enable_llama_fused_attention, fused_attention_compressed

__all__ = ["Cache", "enable_llama_fused_attention", "fused_attention_compressed"]
