"""Indirect attention on the GPU (reference: src/orthocache/indirect_attention.py).

The reference pads the active list to a power-of-two bucket and then attends
``sort_order[:bucket]``, which includes evicted blocks whenever bucket >
num_active (``indirect_attention.py:157-158``).  Here the kernel attends
exactly the num_active retained blocks; ``bucket`` is still reported in the
metadata for callers that read it.
"""

from __future__ import annotations

import torch

from . import _ops
from ._native import require_gpu

BUCKETS = [1, 2, 4, 8, 16, 32, 64, 128, 256, 512]


def _next_bucket(n: int) -> int:
    """``indirect_attention.py:22-26``."""
    for b in BUCKETS:
        if b >= n:
            return b
    return n


def indirect_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, block_mask: torch.Tensor,
                       block_size: int = 512):
    """Zero-copy indirect attention, heads sharing the OR-reduced mask:
    ``indirect_attention.py:127-170``.  Returns (output in q's dtype, meta)."""
    require_gpu(q, keys, values, block_mask)
    seq_k, h, _ = keys.shape
    if seq_k % block_size:
        raise ValueError(f"seq_len {seq_k} is not a multiple of block_size {block_size}")
    nb = seq_k // block_size
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=q.device, mask_in=block_mask)
    out = _ops.attend(q, keys, values, c.indices, c.num_active, block_size=block_size, out_dtype=q.dtype)
    n = int(c.num_active[0].item())
    if n == 0:
        return out, {"num_active": 0, "bucket": 0, "eviction_rate": 1.0}
    return out, {"num_active": n, "bucket": _next_bucket(n), "num_blocks": nb, "eviction_rate": 1.0 - n / nb}


def indirect_attention_fori(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, block_mask: torch.Tensor,
                            block_size: int = 512):
    """Loop-indirection attention (the reference package ``__init__`` imports
    this name, src/orthocache/__init__.py:19, without defining it; its
    benchmark form is ``indirect_loop_attn`` in benchmarks/phase_d_indirect_dma.py:52-111).

    Attends exactly the retained blocks; output bf16 like the loop it names.
    The retained count stays on the device (no host synchronisation).
    """
    require_gpu(q, keys, values, block_mask)
    seq_k, h, _ = keys.shape
    if seq_k % block_size:
        raise ValueError(f"seq_len {seq_k} is not a multiple of block_size {block_size}")
    nb = seq_k // block_size
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=q.device, mask_in=block_mask)
    return _ops.attend(q, keys, values, c.indices, c.num_active, block_size=block_size,
                       out_dtype=torch.bfloat16)
