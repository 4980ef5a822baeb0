"""Loop-indirection decode attention on the GPU (reference: src/orthocache/adaptive_attention.py).

The reference loops ``fori_loop(0, num_active)`` over dynamic slices and
recompiles per distinct num_active; here one HIP kernel reads the active list
and its count from device memory and splits every retained block into
128-token work items across the whole GPU, then a combine kernel merges the
partial softmax states.  Output is bf16, as in the reference.
"""

from __future__ import annotations

import torch

from . import _ops
from ._native import require_gpu

BS = 512
_SEQ_THRESHOLD = 16384  # adaptive_attention.py:126 (reported as the dispatch path label)


def stream_compact(block_mask: torch.Tensor):
    """(active-first permutation (nb,) int32, num_active Python int):
    ``adaptive_attention.py:29-40``.  Reading num_active synchronises, as
    in the reference."""
    require_gpu(block_mask)
    if block_mask.dim() != 1:
        raise ValueError("block_mask must be (num_blocks,)")
    nb = block_mask.shape[0]
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=1, device=block_mask.device, mask_in=block_mask)
    return c.indices, int(c.num_active[0].item())


def _path(seq_k: int, batched: bool = False) -> str:
    base = "vmap_heads" if seq_k <= _SEQ_THRESHOLD else "multihead_loop"
    return ("batch_" + base) if batched else base


def orthocache_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                         block_mask: torch.Tensor, block_size: int = 512):
    """Indirect attention over the blocks where block_mask is True:
    ``adaptive_attention.py:138-184``.

    q (Sq, Hq, D), k/v (S, Hkv, D) with Hq a multiple of Hkv, block_mask
    (nb,) bool (a (nb, Hkv) mask is OR-reduced over heads).  Returns
    (output bf16 (Sq, Hq, D), stats).  No retained block gives zeros.
    """
    require_gpu(q, k_cache, v_cache, block_mask)
    seq_k = k_cache.shape[0]
    if seq_k % block_size:
        raise ValueError(f"seq_len {seq_k} is not a multiple of block_size {block_size}")
    nb = seq_k // block_size
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=k_cache.shape[1], device=q.device, mask_in=block_mask)
    out = _ops.attend(q, k_cache, v_cache, c.indices, c.num_active, block_size=block_size,
                      out_dtype=torch.bfloat16)
    n = int(c.num_active[0].item())
    if n == 0:
        # adaptive_attention.py:164-167 returns zeros_like(q) (q's dtype)
        return torch.zeros_like(q), {"num_active": 0, "eviction_rate": 1.0, "path": "zero"}
    return out, {"num_active": n, "num_blocks": nb, "eviction_rate": 1.0 - n / nb, "path": _path(seq_k)}


def orthocache_attention_batched(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                 block_mask: torch.Tensor, block_size: int = 512):
    """Batched form with one mask shared by the batch: ``adaptive_attention.py:212-260``.

    q (B, Sq, Hq, D), k/v (B, S, Hkv, D), block_mask (nb,).
    """
    require_gpu(q, k_cache, v_cache, block_mask)
    b, seq_k = k_cache.shape[0], k_cache.shape[1]
    if seq_k % block_size:
        raise ValueError(f"seq_len {seq_k} is not a multiple of block_size {block_size}")
    nb = seq_k // block_size
    hkv, d = k_cache.shape[2], k_cache.shape[3]
    mask = block_mask if block_mask.dim() == 1 else block_mask.any(dim=-1)
    # One segment per batch element, each with the same mask.
    mask_b = mask.reshape(1, nb).expand(b, nb).reshape(b * nb)
    cu = torch.arange(0, (b + 1) * nb, nb, dtype=torch.int32, device=q.device)
    c = _ops.mask_compact(num_blocks=b * nb, num_kv_heads=hkv, device=q.device, mask_in=mask_b,
                          cu_blocks=cu, num_segments=b)
    k = k_cache.reshape(b * seq_k, hkv, d)
    v = v_cache.reshape(b * seq_k, hkv, d)
    out = _ops.attend(q, k, v, c.indices, c.num_active, block_size=block_size, out_dtype=torch.bfloat16,
                      cu_blocks=cu, num_segments=b)
    n = int(c.num_active[0].item())
    if n == 0:
        return torch.zeros_like(q), {"num_active": 0, "eviction_rate": 1.0, "path": "zero"}
    return out, {"num_active": n, "num_blocks": nb, "eviction_rate": 1.0 - n / nb, "batch_size": b,
                 "path": _path(seq_k, batched=True)}


# The reference package __init__ imports this name (src/orthocache/__init__.py:20)
# without defining it; it is the adaptive dispatcher above.
adaptive_sparse_attention = orthocache_attention
