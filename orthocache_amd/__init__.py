"""OrthoCache block-eviction attention on AMD MI355X (gfx950).

Drop-in for the reference package's hot path (``orthocache`` v0.3.0,
src/orthocache/__init__.py:5-23): the same function names, arguments and
outputs, taking torch tensors on a ROCm device and running hand-written HIP
kernels from ``_lib/liborthocache_hip.so``:

  FWHT-512 -> band energies / zeta / block mean / query-aware bound
  -> two-gate mask -> stream compaction -> indirect block-sparse attention.

There is no CPU path: the functions raise if the HIP library is missing or
a tensor is not on the GPU.  The reference's multi-device layer
(alltoallv_kv_exchange, distributed_orthocache_attention, ICI byte models) is
not part of this package.
"""

__version__ = "0.1.0"

from .fwht import fwht_512
from .spectral_energy import (
    BAND_DC,
    BAND_HIGH,
    BAND_LOW,
    BAND_MID,
    compute_block_energy_jax,
    compute_multiband_mask,
    compute_query_aware_bounds,
    compute_query_aware_mask,
    compute_spectral_bands,
    compute_spectral_decay_ratio,
    generate_threshold_mask,
)
from .sparse_attention import compile_pallas_sparse_attention, jax_block_sparse_attention
from .compaction import compact_and_attend, stream_compact, stream_decompact
from .partitioning import orthocache_attention_partitioned
from .pipeline import orthocache_forward
from .indirect_attention import indirect_attention, indirect_attention_fori
from .adaptive_attention import adaptive_sparse_attention, orthocache_attention, orthocache_attention_batched
from .varlen import mask_compact_varlen, orthocache_decode_varlen, score_varlen
from .hoisted import BlockStats, CachedDecodeLayer, block_stats
from .paged import flatten_block_table, orthocache_decode_paged

__all__ = [
    "fwht_512",
    "BAND_DC", "BAND_LOW", "BAND_MID", "BAND_HIGH",
    "compute_block_energy_jax", "generate_threshold_mask", "compute_query_aware_bounds",
    "compute_query_aware_mask", "compute_spectral_bands", "compute_spectral_decay_ratio",
    "compute_multiband_mask",
    "jax_block_sparse_attention", "compile_pallas_sparse_attention",
    "stream_compact", "stream_decompact", "compact_and_attend",
    "orthocache_attention_partitioned", "orthocache_forward",
    "indirect_attention", "indirect_attention_fori",
    "adaptive_sparse_attention", "orthocache_attention", "orthocache_attention_batched",
    "score_varlen", "mask_compact_varlen", "orthocache_decode_varlen",
    "BlockStats", "block_stats", "CachedDecodeLayer",
    "flatten_block_table", "orthocache_decode_paged",
]
