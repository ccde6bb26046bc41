"""``shard.cache`` of the reference (src/shard/cache.py): the Cache and its
layer type, from shard_amd."""
from shard_amd.cache import Cache, CacheLayer

__all__ = ["Cache", "CacheLayer"]
