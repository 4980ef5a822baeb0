"""Head-sharded form of the reference's partitioned entry point
(src/orthocache/partitioning.py:20-50).

The reference wraps compact_and_attend in jax custom_partitioning with the
sharding rule 'q h d, k h d, k h d, b h -> q h d': the head axis is
sharded, and each shard runs compact_and_attend on its own heads and its
own slice of the block mask.  A shard therefore compacts over the union of
ITS heads' masks, not of all heads', so the output depends on the shard
count.  `num_shards` states that count; each shard's call runs here in
turn on the one device, as each device would run it, and the outputs are
joined along the head axis (the reference's output sharding).  With one
shard this is compact_and_attend itself.
"""

from __future__ import annotations

import torch

from .compaction import compact_and_attend


def orthocache_attention_partitioned(q, keys, values, block_mask, block_size: int = 512, num_shards: int = 1):
    """Attention output of compact_and_attend per head shard (metadata dropped,
    as in the reference).

    q (Sq, Hq, D), keys/values (S, Hkv, D), block_mask (num_blocks, Hkv).  Hq
    and Hkv must both split evenly into `num_shards` contiguous groups (an
    uneven split of a sharded axis is an error in the reference's sharding
    rule); with Hq = g * Hkv, shard s holds query heads [s*Hq/N, (s+1)*Hq/N),
    which are exactly the query heads of its kv heads.
    """
    n = int(num_shards)
    hq, hkv = q.shape[1], keys.shape[1]
    if n < 1:
        raise ValueError(f"num_shards must be >= 1, got {num_shards}")
    if hq % n or hkv % n:
        raise ValueError(f"heads (q {hq}, kv {hkv}) do not split evenly into {n} shards")
    if n == 1:
        out, _ = compact_and_attend(q, keys, values, block_mask, block_size=block_size)
        return out
    sq, sk = hq // n, hkv // n
    outs = []
    for s in range(n):
        out, _ = compact_and_attend(q[:, s * sq:(s + 1) * sq].contiguous(), keys[:, s * sk:(s + 1) * sk].contiguous(),
                                    values[:, s * sk:(s + 1) * sk].contiguous(),
                                    block_mask[:, s * sk:(s + 1) * sk].contiguous(), block_size=block_size)
        outs.append(out)
    return torch.cat(outs, dim=1)
