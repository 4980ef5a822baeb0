"""Decode with the scoring hoisted to cache-write time.

The reference computes zeta, the block mean and E_AC from a full FWHT of every
key block on every call (``pipeline.py:96-145``), although its own design
notes make zeta query-independent and meant to be computed once, when a block
enters the KV cache (``docs/mathematical_framework.md:242-250``,
``docs/technical_report.md:74``).  This module keeps those per-(block, head)
statistics next to the cache:

* ``block_stats(keys)`` / ``BlockStats.update(keys, first_block)`` -- one pass
  of the scoring kernel over the keys of new blocks only (dc, E_AC, zeta);
* ``CachedDecodeLayer`` -- a decode step that reads the statistics instead of
  the keys: the bound tau_j(q) = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d)
  (``spectral_energy.py:141-177``), the two-gate mask on the cached zeta,
  compaction and attention (``oc_decode_layer_cached``).

Results equal ``DecodeLayer`` on the same keys up to the fp32 rounding of the
bound (the dot product is summed in another order).
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _native as N
from ._native import check, dtype_code, lib, ptr, require_gpu, stream_ptr
from ._ops import BLOCK, DecodeLayer, _kv_view, _pages_view


@dataclass
class BlockStats:
    """Write-time statistics of every (block, kv head): dc (nb, Hkv, D) -- the
    FWHT coefficient 0 per column (kbar = dc / sqrt(512)) --, e_ac (nb, Hkv)
    and zeta (nb, Hkv), all fp32 on the device."""

    dc: torch.Tensor
    e_ac: torch.Tensor
    zeta: torch.Tensor

    @property
    def num_blocks(self) -> int:
        return self.zeta.shape[0]

    def update(self, keys: torch.Tensor, first_block: int, num_blocks: int | None = None,
               pages: torch.Tensor | None = None) -> "BlockStats":
        """(Re)compute the statistics of blocks [first_block, first_block + num_blocks)
        of ``keys`` (S, Hkv, D) in place -- e.g. the blocks a decode step just
        filled.  Only those blocks' keys are read.  With ``pages`` (int32, one
        physical page of the pool ``keys`` per logical block) the blocks are
        logical blocks of a paged cache."""
        keys = _kv_view(keys, "keys")
        s, hkv, d = keys.shape
        nb = s // BLOCK
        pages = _pages_view(pages, keys)
        if pages is not None:
            nb = pages.shape[0]
        n = nb - first_block if num_blocks is None else num_blocks
        if first_block < 0 or n < 0 or first_block + n > min(nb, self.num_blocks):
            raise ValueError(f"blocks [{first_block}, {first_block + n}) outside the cache ({nb} blocks)")
        if tuple(self.dc.shape[1:]) != (hkv, d):
            raise ValueError("keys do not match the statistics' heads / head_dim")
        if n == 0:
            return self
        a = N.ScoreArgs()
        esz = keys.element_size()
        if pages is None:
            a.keys = ptr(keys) + first_block * BLOCK * keys.stride(0) * esz
        else:
            a.keys = ptr(keys)
            a.pages = ptr(pages) + first_block * 4
            a.num_pages = s // BLOCK
        a.keys_dtype = dtype_code(keys.dtype)
        a.keys_tok_stride = keys.stride(0); a.keys_head_stride = keys.stride(1)
        a.head_dim = d; a.num_kv_heads = hkv; a.total_blocks = n; a.num_segments = 1
        a.zeta = ptr(self.zeta) + first_block * hkv * 4
        a.dc = ptr(self.dc) + first_block * hkv * d * 4
        a.e_ac = ptr(self.e_ac) + first_block * hkv * 4
        check(lib().oc_score_blocks(C.byref(a), stream_ptr(keys.device)), "oc_score_blocks")
        return self


def block_stats(keys: torch.Tensor, capacity_blocks: int | None = None,
                pages: torch.Tensor | None = None) -> BlockStats:
    """Statistics of every block of ``keys`` (S, Hkv, D), S a multiple of 512,
    in buffers sized for ``capacity_blocks`` (default: the blocks present).
    With ``pages``, ``keys`` is a page pool and the blocks are the logical
    blocks the page list names."""
    require_gpu(keys, pages)
    keys = _kv_view(keys, "keys")
    s, hkv, d = keys.shape
    if s % BLOCK:
        raise ValueError(f"seq_len {s} is not a multiple of the block size {BLOCK}")
    nb = s // BLOCK if pages is None else pages.shape[0]
    cap = nb if capacity_blocks is None else capacity_blocks
    if cap < nb:
        raise ValueError("capacity_blocks is smaller than the blocks present")
    f32 = dict(dtype=torch.float32, device=keys.device)
    st = BlockStats(torch.empty((cap, hkv, d), **f32), torch.empty((cap, hkv), **f32),
                    torch.empty((cap, hkv), **f32))
    return st.update(keys, 0, nb, pages=pages)


class CachedDecodeLayer(DecodeLayer):
    """``DecodeLayer`` whose scoring phase reads write-time ``BlockStats``
    (bounds, cached zeta) instead of the keys.  ``zeta`` is not an output."""

    def __init__(self, q, k, v, stats: BlockStats, tau, zeta_max, **kw):
        kw.setdefault("keep_scores", True)
        super().__init__(q, k, v, tau, zeta_max, **kw)
        nb = self.args.total_blocks
        if stats.num_blocks < nb or tuple(stats.dc.shape[1:]) != (self.args.num_kv_heads, self.args.head_dim):
            raise ValueError("block statistics do not cover the keys")
        self.stats = stats
        self._stats_c = N.BlockStats(ptr(stats.dc), ptr(stats.e_ac), ptr(stats.zeta))
        self.zeta = None
        self.args.zeta = None
        L = lib()
        ws = int(L.oc_decode_layer_cached_workspace_size(C.byref(self.args)))
        if ws > self._ws_bytes:
            self.workspace = torch.empty((ws,), dtype=torch.uint8, device=self.device)
            self._ws_ptr = ptr(self.workspace)
            self._ws_bytes = ws
        sp = C.byref(self._stats_c)
        f = L.oc_decode_layer_cached
        self._fn = lambda argp, wsp, wsb, s: f(argp, sp, wsp, wsb, s)

    def run(self, stream: int | None = None) -> torch.Tensor:
        s = stream_ptr(self.device) if stream is None else stream
        check(self._fn(self._argp, self._ws_ptr, self._ws_bytes, s), "oc_decode_layer_cached")
        return self.out

    def phases(self):
        raise NotImplementedError("per-phase launches are provided by DecodeLayer only")
