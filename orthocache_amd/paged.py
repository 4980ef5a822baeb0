"""Paged KV caches: block tables instead of contiguous sequences.

The reference's compaction already produces a page list (``active_indices``,
``compaction.py:65-82``); serving engines keep K/V in a pool of fixed-size
pages addressed through per-sequence block tables (vLLM's layout).  Here a
page is one 512-token OrthoCache block: the pools are ``(num_pages * 512,
Hkv, D)``, and every kernel that reads keys or values takes a flattened page
list -- the physical page of each logical block, segments concatenated in
``cu_blocks`` order.  Scores, masks and block lists stay in logical block
numbering.  Page numbers are clamped into the pool by the kernels.
"""

from __future__ import annotations

import torch

from . import _ops
from ._native import require_gpu
from .varlen import cu_blocks_from_seqlens


def flatten_block_table(block_table: torch.Tensor, cu_blocks: torch.Tensor, total_blocks: int) -> torch.Tensor:
    """(B, max_blocks) int block table + (B + 1) block offsets -> (total_blocks,)
    int32 page list (logical block j of sequence s at ``cu_blocks[s] + j``).
    Device-side, no host synchronisation."""
    require_gpu(block_table, cu_blocks)
    if block_table.dim() != 2:
        raise ValueError("block_table must be (num_sequences, max_blocks)")
    dev = block_table.device
    j = torch.arange(total_blocks, device=dev, dtype=torch.int64)
    cu = cu_blocks.to(torch.int64)
    seg = torch.searchsorted(cu[1:].contiguous(), j, right=True)
    local = j - cu[seg]
    return block_table.to(torch.int32)[seg, local].contiguous()


def orthocache_decode_paged(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                            block_table: torch.Tensor, cu_seqlens: torch.Tensor, tau, zeta_max, *,
                            total_blocks: int, out: torch.Tensor | None = None, out_dtype=None):
    """Score -> two-gate mask -> compaction -> attention for a ragged batch
    whose K/V live in page pools.  q (B, Sq, Hq, D); pools (P*512, Hkv, D);
    block_table (B, max_blocks); cu_seqlens (B + 1) token offsets of the
    logical sequences (multiples of 512); ``total_blocks`` = cu_seqlens[-1] /
    512 (a host int, so no synchronisation is needed).  Returns (output,
    {tau_max, zeta, indices, num_active}) on the device."""
    require_gpu(q, k_pool, v_pool, block_table, cu_seqlens)
    b = cu_seqlens.shape[0] - 1
    cu_blocks = cu_blocks_from_seqlens(cu_seqlens)
    pages = flatten_block_table(block_table, cu_blocks, total_blocks)
    layer = _ops.DecodeLayer(q, k_pool, v_pool, tau, zeta_max, cu_blocks=cu_blocks, num_segments=b, out=out,
                             out_dtype=out_dtype, pages=pages)
    o = layer.run()
    return o, {"tau_max": layer.tau_max, "zeta": layer.zeta, "indices": layer.indices,
               "num_active": layer.num_active, "pages": pages}
