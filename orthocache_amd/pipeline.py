"""End-to-end OrthoCache forward on the GPU (reference: src/orthocache/pipeline.py).

One fused scoring pass (zeta and the query-aware bound together), one
mask + compaction kernel, one attention launch.  Metadata keys are the
reference's; timings are wall-clock with device synchronisation.
"""

from __future__ import annotations

import time

import torch

from . import _ops
from ._native import BLOCK, require_gpu


def _sync(dev):
    torch.cuda.synchronize(dev)


def orthocache_forward(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, block_size: int = 512,
                       zeta_max: float = 5.0, tau: float | None = None, mode: str = "compact"):
    """Spectral scoring -> two-gate eviction -> attention: ``pipeline.py:33-157``.

    mode: 'compact' (attend the blocks any head keeps), 'sparse' (each head
    attends its own kept blocks; a head keeping none returns zeros, as the
    gated kernel does) or 'dense' (all blocks).  tau=None picks
    mean - std of the per-(block, head) max bound (``pipeline.py:168-176``).
    Returns (output in q's dtype, metadata dict).
    """
    require_gpu(q, keys, values)
    seq_len_k, num_heads, head_dim = keys.shape
    seq_len_q = q.shape[0]
    num_blocks = seq_len_k // block_size
    dev = keys.device
    metadata = {
        "mode": mode,
        "seq_len_q": seq_len_q,
        "seq_len_k": seq_len_k,
        "num_blocks": num_blocks,
        "num_heads": num_heads,
        "head_dim": head_dim,
        "block_size": block_size,
        "zeta_max": zeta_max,
    }

    if mode == "dense":
        t0 = time.perf_counter()
        output = _dense_attention(q, keys, values, head_dim, block_size)
        _sync(dev)
        metadata["latency_ms"] = (time.perf_counter() - t0) * 1000
        metadata["eviction_rate"] = 0.0
        return output, metadata
    if mode not in ("compact", "sparse"):
        raise ValueError(f"Unknown mode: {mode!r}. Use 'dense', 'sparse', or 'compact'.")
    if block_size != BLOCK:
        raise ValueError(f"the FWHT scoring path needs block_size == 512, got {block_size}")
    if seq_len_k % block_size:
        raise ValueError(f"seq_len {seq_len_k} is not a multiple of block_size {block_size}")

    t_spectral = time.perf_counter()
    sc = _ops.score(keys, q, want_zeta=True)
    zeta = sc.zeta
    if tau is None:
        tau = _compute_auto_tau_from(sc.tau_max)
        metadata["tau_auto"] = True
    else:
        metadata["tau_auto"] = False
    metadata["tau"] = tau
    c = _ops.mask_compact(num_blocks=num_blocks, num_kv_heads=num_heads, device=dev, tau_max=sc.tau_max,
                          zeta=zeta, tau=tau, zeta_max=zeta_max, want_mask=True,
                          want_indices=(mode == "compact"), want_head_lists=(mode == "sparse"),
                          empty_head_all=False)
    _sync(dev)
    metadata["spectral_ms"] = (time.perf_counter() - t_spectral) * 1000

    zeta_any_head = zeta.mean(dim=-1)
    stats = torch.stack([zeta_any_head.mean(), zeta_any_head.std(unbiased=False), zeta_any_head.min(),
                         zeta_any_head.max()]).tolist()
    metadata["zeta_mean"], metadata["zeta_std"], metadata["zeta_min"], metadata["zeta_max_observed"] = stats
    blocks_retained = int(c.mask.any(dim=-1).sum().item())
    metadata["blocks_retained"] = blocks_retained
    metadata["blocks_evicted"] = num_blocks - blocks_retained
    metadata["eviction_rate"] = float(1.0 - blocks_retained / num_blocks)

    t_attn = time.perf_counter()
    if mode == "compact":
        output = _ops.attend(q, keys, values, c.indices, c.num_active, block_size=block_size, out_dtype=q.dtype)
        metadata["compact_num_active"] = blocks_retained
    else:
        output = _ops.attend(q, keys, values, c.head_indices, c.head_num_active, block_size=block_size,
                             per_head=True, uniform=c.head_uniform, out_dtype=q.dtype)
    _sync(dev)
    t_attn_end = time.perf_counter()
    metadata["attention_ms"] = (t_attn_end - t_attn) * 1000
    metadata["total_ms"] = (t_attn_end - t_spectral) * 1000
    return output, metadata


def _dense_attention(q: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, head_dim: int,
                     block_size: int = 512) -> torch.Tensor:
    """Full softmax attention over every key: ``pipeline.py:160-165``."""
    seq_k = keys.shape[0]
    bs = block_size if seq_k % block_size == 0 else seq_k
    nb = seq_k // bs
    idx = torch.arange(nb, dtype=torch.int32, device=keys.device)
    cnt = torch.tensor([nb], dtype=torch.int32, device=keys.device)
    return _ops.attend(q, keys, values, idx, cnt, block_size=bs, out_dtype=q.dtype)


def _compute_auto_tau_from(tau_max_parts: torch.Tensor) -> float:
    """mean - std (population) of the max bound per (block, head): ``pipeline.py:168-176``."""
    mb = tau_max_parts.amax(dim=0) if tau_max_parts.shape[0] > 1 else tau_max_parts[0]
    return float((mb.mean() - mb.std(unbiased=False)).item())


def _compute_auto_tau(q: torch.Tensor, keys: torch.Tensor, block_size: int = 512) -> float:
    """``pipeline.py:168-176``."""
    return _compute_auto_tau_from(_ops.score(keys, q, want_zeta=False).tau_max)
