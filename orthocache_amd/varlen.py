"""Ragged batches and multi-layer sweeps: many segments in one launch per kernel.

A segment is one sequence of a ragged decode batch, or one layer of a
multi-layer scoring sweep.  Keys/values of all segments are packed along the
token axis, (total_tokens, Hkv, D), with ``cu_seqlens`` (B+1) token offsets
(each a multiple of 512; FlashAttention's varlen convention).  Every segment
has its own queries (B, Sq, Hq, D) and its own thresholds.  The reference
batches only with one shared mask (src/orthocache/adaptive_attention.py:212-260)
and scores one sequence per call; here one launch scores every block of every
segment, one compacts every segment, one attends every retained block.
"""

from __future__ import annotations

import torch

from . import _ops
from ._native import BLOCK, require_gpu


def cu_blocks_from_seqlens(cu_seqlens: torch.Tensor) -> torch.Tensor:
    if cu_seqlens.dtype not in (torch.int32, torch.int64):
        raise ValueError("cu_seqlens must be an integer tensor")
    return (cu_seqlens // BLOCK).to(torch.int32).contiguous()


def score_varlen(q: torch.Tensor, keys: torch.Tensor, cu_seqlens: torch.Tensor):
    """(tau_max (nb_total, Hkv), zeta (nb_total, Hkv)) for every block of every segment."""
    require_gpu(q, keys, cu_seqlens)
    b = cu_seqlens.shape[0] - 1
    if q.dim() != 4 or q.shape[0] != b:
        raise ValueError("q must be (segments, seq_q, q_heads, head_dim)")
    sc = _ops.score(keys, q, cu_blocks=cu_blocks_from_seqlens(cu_seqlens), num_segments=b)
    return sc.tau_max[0], sc.zeta


def mask_compact_varlen(tau_max: torch.Tensor, zeta: torch.Tensor, cu_seqlens: torch.Tensor, tau, zeta_max):
    """Per-segment two-gate mask and compaction.  tau / zeta_max: floats or (B,) tensors.

    Returns (mask (nb_total, Hkv) bool, indices (nb_total,) int32 with each
    segment's local active-first permutation at its block offset,
    num_active (B,) int32)."""
    b = cu_seqlens.shape[0] - 1
    nb, h = tau_max.shape
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=tau_max.device, tau_max=tau_max.reshape(1, nb, h),
                          zeta=zeta, tau=tau, zeta_max=zeta_max, want_mask=True,
                          cu_blocks=cu_blocks_from_seqlens(cu_seqlens), num_segments=b)
    return c.mask, c.indices, c.num_active


def orthocache_decode_varlen(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, cu_seqlens: torch.Tensor,
                             tau, zeta_max, *, out: torch.Tensor | None = None, out_dtype=None):
    """Score -> two-gate mask -> compaction -> attention for a ragged batch.

    Returns (output (B, Sq, Hq, D), {tau_max, zeta, indices, num_active}) with
    every tensor on the device (no host synchronisation)."""
    require_gpu(q, keys, values, cu_seqlens)
    b = cu_seqlens.shape[0] - 1
    if q.dim() != 4 or q.shape[0] != b:
        raise ValueError("q must be (segments, seq_q, q_heads, head_dim)")
    layer = _ops.DecodeLayer(q, keys, values, tau, zeta_max, cu_blocks=cu_blocks_from_seqlens(cu_seqlens),
                             num_segments=b, out=out, out_dtype=out_dtype)
    o = layer.run()
    return o, {"tau_max": layer.tau_max, "zeta": layer.zeta, "indices": layer.indices,
               "num_active": layer.num_active}
