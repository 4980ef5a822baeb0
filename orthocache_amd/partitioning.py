"""Single-device form of the reference's partitioned entry point
(src/orthocache/partitioning.py:38-44).

The reference wraps compact_and_attend in jax custom_partitioning so that a
head-sharded call runs one compact_and_attend per shard.  On one GPU the
call is compact_and_attend itself.
"""

from __future__ import annotations

from .compaction import compact_and_attend


def orthocache_attention_partitioned(q, keys, values, block_mask, block_size: int = 512):
    """Attention output of compact_and_attend (metadata dropped, as in the reference)."""
    out, _ = compact_and_attend(q, keys, values, block_mask, block_size=block_size)
    return out
