"""shard_amd — MI355X-native compressed-KV attention path of Shard.

Public API (same names as the reference package ``shard``):
    Cache, enable_llama_fused_attention, fused_attention_compressed
The kernels live in libshard_hip.so (built in-tree by shard_amd.build).
"""
from .cache import Cache, CacheLayer
from .attention import enable_llama_fused_attention, fused_attention_compressed

__all__ = ["Cache", "CacheLayer", "enable_llama_fused_attention", "fused_attention_compressed"]
__version__ = "0.1.0"
