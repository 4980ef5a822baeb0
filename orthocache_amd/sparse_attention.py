"""Per-head block-sparse attention on the GPU (reference: src/orthocache/sparse_attention.py).

Both entry points attend only the blocks each head keeps (per-head lists
from the compaction kernel), instead of computing logits for every key and
masking them.
"""

from __future__ import annotations

import torch

from . import _ops
from ._native import require_gpu


def _per_head(q, keys, values, block_mask, block_size, empty_head_all):
    require_gpu(q, keys, values, block_mask)
    if keys.dim() != 3 or keys.shape[0] % block_size:
        raise ValueError("keys must be (seq_len, num_heads, head_dim) with seq_len a multiple of block_size")
    nb = keys.shape[0] // block_size
    h = keys.shape[1]
    if block_mask.dim() != 2 or tuple(block_mask.shape) != (nb, h):
        raise ValueError(f"block_mask must be (num_blocks, num_heads) = ({nb}, {h}), got {tuple(block_mask.shape)}")
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=keys.device, mask_in=block_mask,
                          want_indices=False, want_head_lists=True, empty_head_all=empty_head_all)
    return _ops.attend(q, keys, values, c.head_indices, c.head_num_active, block_size=block_size,
                       per_head=True, uniform=c.head_uniform, out_dtype=q.dtype)


def jax_block_sparse_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                               block_mask: torch.Tensor, block_size: int = 512) -> torch.Tensor:
    """Per-head predicated attention: ``sparse_attention.py:5-64``.

    Each head attends the tokens of its kept blocks.  A head with every block
    masked gets equal weights over all keys (the reference's softmax over
    logits that are all -1e9), i.e. the mean of V.
    """
    return _per_head(q, keys, values, block_mask, block_size, empty_head_all=True)


def compile_pallas_sparse_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                                    block_mask: torch.Tensor, block_size: int = 512) -> torch.Tensor:
    """The gated block-sparse kernel: ``sparse_attention.py:67-180``.

    Same as jax_block_sparse_attention except for a head with every block
    masked, which returns zeros (the kernel's gated accumulators stay zero and
    it divides by max(l, 1e-9)).
    """
    return _per_head(q, keys, values, block_mask, block_size, empty_head_all=False)
