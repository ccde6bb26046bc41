"""``shard.attention`` of the reference (src/shard/attention.py): the patch of
transformers' Llama attention and the fused calls, from shard_amd."""
from shard_amd.attention import (enable_llama_fused_attention, fused_attention_compressed,
                                 fused_attention_compressed_full)

__all__ = ["enable_llama_fused_attention", "fused_attention_compressed",
           "fused_attention_compressed_full"]
