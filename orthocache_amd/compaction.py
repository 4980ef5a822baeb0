"""Stream compaction on the GPU (reference: src/orthocache/compaction.py).

The mask reduction, prefix sum and permutation run in one HIP kernel with no
host synchronisation; ``num_active`` stays a device scalar.  compact_and_attend
attends the retained blocks in place (indirect attention over the original
K/V) instead of attending a materialised compacted copy; the softmax is over
the same tokens, so the result is the same up to fp32 rounding.
"""

from __future__ import annotations

import torch

from . import _ops
from ._native import require_gpu


def _blocks(keys: torch.Tensor, block_size: int) -> int:
    if keys.dim() != 3:
        raise ValueError(f"keys must be (seq_len, num_heads, head_dim), got {tuple(keys.shape)}")
    if keys.shape[0] % block_size:
        raise ValueError(f"seq_len {keys.shape[0]} is not a multiple of block_size {block_size}")
    return keys.shape[0] // block_size


def stream_compact(keys: torch.Tensor, values: torch.Tensor, block_mask: torch.Tensor, block_size: int = 512):
    """Compact KV blocks retained by any head: ``compaction.py:28-100``.

    Returns (compact_keys (nb, bs, H, D), compact_values, active_indices (nb,)
    int32, num_active 0-d int32).  active_indices is the full active-first
    stable permutation; compacted positions >= num_active are zero.
    """
    require_gpu(keys, values, block_mask)
    nb = _blocks(keys, block_size)
    _, h, d = keys.shape
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=keys.device, mask_in=block_mask)
    ck = torch.empty((nb, block_size, h, d), dtype=keys.dtype, device=keys.device)
    cv = torch.empty((nb, block_size, h, d), dtype=values.dtype, device=values.device)
    _ops.copy_blocks(keys.contiguous().reshape(nb, -1), ck, c.indices, c.num_active, nb, scatter=False)
    _ops.copy_blocks(values.contiguous().reshape(nb, -1), cv, c.indices, c.num_active, nb, scatter=False)
    return ck, cv, c.indices, c.num_active[0]


def stream_decompact(compact_output: torch.Tensor, active_indices: torch.Tensor, num_active,
                     num_blocks_original: int, block_size: int = 512) -> torch.Tensor:
    """Scatter compacted blocks back: ``compaction.py:103-154``.

    out[active_indices[i]] = compact_output[i] for i < num_active; every other
    block is zero.  With the permutation from stream_compact that is the
    reference's result.  Other lists are safe: entries outside
    [0, num_blocks_original) are dropped (JAX drops out-of-bounds scatter
    updates; negative entries count from the end first), and when several
    positions name one block the last of them wins (a JAX scatter leaves
    that order to the implementation).
    """
    require_gpu(compact_output, active_indices)
    nb = num_blocks_original
    if compact_output.shape[0] != nb or active_indices.shape[0] != nb:
        raise ValueError("compact_output and active_indices must have num_blocks_original entries")
    if not isinstance(num_active, torch.Tensor):
        num_active = torch.tensor([int(num_active)], dtype=torch.int32, device=compact_output.device)
    na = num_active.reshape(1).to(torch.int32)
    idx = active_indices.to(torch.int32).contiguous()
    out = torch.empty_like(compact_output.contiguous())
    _ops.copy_blocks(compact_output.contiguous().reshape(nb, -1), out, idx, na, nb, scatter=True)
    return out


def compact_and_attend(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, block_mask: torch.Tensor,
                       block_size: int = 512):
    """Compaction + attention over the retained blocks: ``compaction.py:157-222``.

    Returns (output (Sq, Hq, D) in q's dtype, {num_active, num_blocks,
    eviction_rate}); num_active and eviction_rate are 0-d device tensors, as
    the reference returns traced arrays from its jitted function.
    """
    require_gpu(q, keys, values, block_mask)
    nb = _blocks(keys, block_size)
    h = keys.shape[1]
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=keys.device, mask_in=block_mask)
    out = _ops.attend(q, keys, values, c.indices, c.num_active, block_size=block_size, out_dtype=q.dtype)
    num_active = c.num_active[0]
    return out, {
        "num_active": num_active,
        "num_blocks": nb,
        "eviction_rate": 1.0 - num_active.to(torch.float32) / nb,
    }
