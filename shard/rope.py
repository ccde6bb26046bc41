"""``shard.rope`` of the reference (src/shard/rope.py): the RoPE frequency
lookup the reference's benchmark imports (rope.py:32-47), from shard_amd."""
from shard_amd.host import get_rope_inv_freq

__all__ = ["get_rope_inv_freq"]
