"""CPU oracle for the OrthoCache block-eviction path (TEST INFRASTRUCTURE ONLY).

This module restates, in NumPy, what the reference computes on the path
score -> mask -> compact -> attend.  It is the checker the GPU kernels are
compared against; it is never the thing measured or shipped.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package (``orthocache_amd``) never
imports it and fails loudly when its HIP library is missing.

Every function cites the reference file:line it follows (paths relative to
the reference repository root).  Arithmetic is float64 by default so the
oracle is the "truth" the fp32 GPU kernels are held to within a tolerance;
``dtype=np.float32`` gives the fp32 restatement used as the CPU baseline.

Pinning (what checks each function independently of its own formula):

* ``fwht_512`` / ``run_fwht_on_blocks``: closed form ``H_512 / sqrt(512)``
  from ``scipy.linalg.hadamard`` (the reference notebook's Gate 1 check),
  involution, Parseval, unit-vector and alternating-sign known answers.
* ``spectral_bands`` / ``spectral_decay_ratio``: brute force from the
  Hadamard matrix on small inputs; the reference's published Gate-6 golden
  values (zeta_A == 0.0, mean zeta_B == 4.037281036376953, mean AC energies
  7645.267578125 / 7629.59033203125); the reference tests' known answers
  (Walsh-coherent block zeta < 0.01, alternating block zeta > 1).
* ``query_aware_bounds``: closed form E_AC = sum ||k_i||^2 - 512 ||kbar||^2
  and the Cauchy-Schwarz invariant bound >= max_i q.k_i / sqrt(d).
* ``mask_from_scores`` / masks: the reference tests' threshold-mask known
  answer, NaN semantics, and the two-gate test of
  ``tests/test_spectral_bands.py:177-213`` regenerated from its seed (exact
  mask, and a variant with the reference's Walsh-coherent block that the zeta
  gate keeps).
* ``query_aware_mask`` / ``multiband_mask``: literal masks on keys built from
  natural-order Walsh rows 1 and 256 plus a mean, whose band energies, zeta,
  kbar and E_AC follow from the construction (orthogonality of the rows); a
  sequency-ordered transform fails them.
* ``auto_tau`` / ``auto_tau_from_max_bounds``: the known answer mean - population
  std of [1, 2, 3, 4] = 2.5 - sqrt(1.25) (a sample std fails it), and the
  Walsh construction's bounds in closed form.
* ``stream_compact_indices``: the compaction known answers of
  ``tests/test_alltoallv.py:60-67``, ``tests/test_distributed.py:57-64`` and
  ``tests/test_adaptive_attention.py:60-67`` plus brute-force stable
  partition; an unstable (Hoare) partition fails the first known answer.
* ``stream_decompact``: the compact -> decompact round trip on a permutation;
  lists that are not one follow JAX's scatter rules (negative entries count
  from the end, out-of-bounds entries are dropped) with positions applied in
  order.
* ``attention_*``: float64 closed-form softmax over the retained tokens, and
  the reference's own C++ CPU attention (``notebooks/phase_d_kaggle.py``
  custom call) when ``oracle/_ref`` has been built from the reference.
* ``block_logits``: a softmax over the retained blocks' logits, times their
  values, must reproduce ``attention_active_blocks`` (which the reference's
  C++ attention pins); the logits of a key equal to the query are
  ||q||^2 / sqrt(d).
"""

from __future__ import annotations

import numpy as np

BLOCK = 512
SQRT512 = 22.627416997969522  # fwht.py:61 divides by this literal
# spectral_energy.py:15-18: natural-order (Hadamard-index) band boundaries.
BAND_DC = 0
BAND_LOW = (1, 64)
BAND_MID = (64, 256)
BAND_HIGH = (256, 512)
ZETA_EPS = 1e-6  # spectral_energy.py:138


# --------------------------------------------------------------------------
# FWHT
# --------------------------------------------------------------------------
def fwht_512(x: np.ndarray, dtype=np.float64) -> np.ndarray:
    """512-point FWHT along axis 0, natural (Hadamard) order, scaled 1/sqrt(512).

    Follows ``src/orthocache/fwht.py:4-65``: nine radix-2 stages with stride
    h = 1, 2, ..., 256, each viewing the rows as (512/2h, 2, h) and replacing
    the pair (a, b) with (a + b, a - b); then a division by sqrt(512)
    (``fwht.py:61``).  1-D input is treated as one column (``fwht.py:17-19``).
    """
    x = np.asarray(x)
    one_d = x.ndim == 1
    y = x.astype(dtype).reshape(BLOCK, -1)
    if y.shape[0] != BLOCK:
        raise ValueError("fwht_512 needs 512 rows")
    cols = y.shape[1]
    h = 1
    while h < BLOCK:
        v = y.reshape(BLOCK // (2 * h), 2, h, cols)
        y = np.stack([v[:, 0] + v[:, 1], v[:, 0] - v[:, 1]], axis=1).reshape(BLOCK, cols)
        h *= 2
    y = y / dtype(SQRT512)
    return y[:, 0] if one_d else y


def run_fwht_on_blocks(keys: np.ndarray, block_size: int = BLOCK, dtype=np.float64) -> np.ndarray:
    """(S, H, D) -> spectral coefficients (nb, 512, H, D).

    Follows ``spectral_energy.py:38-66``: block, move the token axis first,
    flatten the rest, FWHT, and undo the transpose.
    """
    s, h, d = keys.shape
    if block_size != BLOCK:
        raise ValueError("the FWHT path needs block_size == 512")
    nb = s // block_size
    blocks = keys[: nb * block_size].reshape(nb, block_size, h, d).astype(dtype)
    flat = np.transpose(blocks, (1, 0, 2, 3)).reshape(block_size, nb * h * d)
    spec = fwht_512(flat, dtype=dtype).reshape(block_size, nb, h, d)
    return np.transpose(spec, (1, 0, 2, 3))


# --------------------------------------------------------------------------
# Scores
# --------------------------------------------------------------------------
def block_energy(keys: np.ndarray, block_size: int = BLOCK, dtype=np.float64) -> np.ndarray:
    """Sum of squares per (block, head): ``spectral_energy.py:21-35``."""
    s, h, d = keys.shape
    nb = s // block_size
    b = keys[: nb * block_size].reshape(nb, block_size, h, d).astype(dtype)
    return np.sum(b * b, axis=(1, 3))


def spectral_bands(keys, block_size=BLOCK, band_low=BAND_LOW, band_mid=BAND_MID,
                   band_high=BAND_HIGH, dtype=np.float64):
    """(dc, e_low, e_mid, e_high): ``spectral_energy.py:69-106``.

    dc is coefficient 0 (nb, H, D); each band energy is the sum of squared
    coefficients over the band's natural-index range and over head_dim.
    """
    spec = run_fwht_on_blocks(keys, block_size, dtype)
    dc = spec[:, BAND_DC]
    lo = np.sum(spec[:, band_low[0]:band_low[1]] ** 2, axis=(1, 3))
    mi = np.sum(spec[:, band_mid[0]:band_mid[1]] ** 2, axis=(1, 3))
    hi = np.sum(spec[:, band_high[0]:band_high[1]] ** 2, axis=(1, 3))
    return dc, lo, mi, hi


def spectral_decay_ratio(keys, block_size=BLOCK, band_low=BAND_LOW, band_high=BAND_HIGH,
                         dtype=np.float64):
    """zeta = E_high / (E_low + 1e-6): ``spectral_energy.py:109-138``.

    The middle band passed down is (band_low[1], band_high[0]) as at
    ``spectral_energy.py:135-136``; it is computed and discarded.
    """
    _, lo, _, hi = spectral_bands(keys, block_size, band_low, (band_low[1], band_high[0]),
                                  band_high, dtype)
    return hi / (lo + dtype(ZETA_EPS))


def query_aware_bounds(q, keys, block_size=BLOCK, dtype=np.float64):
    """tau_j(q) = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d), shape (Sq, nb, H).

    Follows ``spectral_energy.py:141-177``: kbar = DC / sqrt(block_size)
    (``:166``), E_AC = sum over coefficients 1..511 and head_dim (``:162-163``).
    """
    _, h, d = keys.shape
    if q.shape[1] != h or q.shape[2] != d:
        raise ValueError("q and keys must share (num_heads, head_dim)")
    spec = run_fwht_on_blocks(keys, block_size, dtype)
    dc = spec[:, 0]
    e_ac = np.sum(spec[:, 1:] ** 2, axis=(1, 3))
    kbar = dc / np.sqrt(dtype(block_size))
    qd = q.astype(dtype)
    align = np.einsum("qhd,bhd->qbh", qd, kbar) / np.sqrt(dtype(d))
    qn = np.linalg.norm(qd, axis=-1)
    resid = (qn[:, None, :] * np.sqrt(e_ac)[None, :, :]) / np.sqrt(dtype(d))
    return align + resid


def fold_gqa(q: np.ndarray, num_kv_heads: int) -> np.ndarray:
    """(Sq, G*Hkv, D) -> (Sq*G, Hkv, D): query head h*G+g reads kv head h.

    The reference scores need equal head counts (``spectral_energy.py:169``);
    the mask is a max over axis 0 (``:195``), so folding the group into the
    query axis gives the same per-(block, kv head) maximum.
    """
    sq, hq, d = q.shape
    g = hq // num_kv_heads
    if g * num_kv_heads != hq:
        raise ValueError("query heads must be a multiple of kv heads")
    return q.reshape(sq, num_kv_heads, g, d).transpose(0, 2, 1, 3).reshape(sq * g, num_kv_heads, d)


def nanmax_axis0(x: np.ndarray) -> np.ndarray:
    """``jnp.max`` semantics (NaN propagates), restated with ``np.max``."""
    return np.max(x, axis=0)


def mask_from_scores(tau_max, zeta, tau, zeta_max):
    """Two-gate mask on fp32 scores: ``spectral_energy.py:180-234``.

    keep = (tau_max >= fp32(tau)) & (zeta <= fp32(zeta_max)).  JAX rounds a
    Python-float threshold to the array's fp32 (weak typing); any comparison
    with NaN is False.
    """
    tm = np.asarray(tau_max, dtype=np.float32)
    z = np.asarray(zeta, dtype=np.float32)
    with np.errstate(invalid="ignore"):
        return (tm >= np.float32(tau)) & (z <= np.float32(zeta_max))


def query_aware_mask(q, keys, tau, block_size=BLOCK, dtype=np.float64):
    """``spectral_energy.py:180-196``."""
    b = query_aware_bounds(q, keys, block_size, dtype)
    return nanmax_axis0(b) >= tau


def multiband_mask(q, keys, tau, zeta_max, block_size=BLOCK, dtype=np.float64):
    """``spectral_energy.py:199-234`` (float64 truth; see mask_from_scores)."""
    tm = nanmax_axis0(query_aware_bounds(q, keys, block_size, dtype))
    z = spectral_decay_ratio(keys, block_size, dtype=dtype)
    return (tm >= tau) & (z <= zeta_max)


def threshold_mask(energies, epsilon):
    """``spectral_energy.py:237-239``."""
    return np.asarray(energies) >= epsilon


# --------------------------------------------------------------------------
# Compaction
# --------------------------------------------------------------------------
def stream_compact_indices(block_mask: np.ndarray):
    """Active-first stable permutation and count.

    ``compaction.py:65-82`` (OR over heads, ``argsort(-active, stable)``) and
    ``adaptive_attention.py:29-40`` (``argsort(where(mask, iota, nb+iota))``)
    give the same permutation: active blocks ascending, then inactive ones
    ascending.
    """
    m = np.asarray(block_mask, dtype=bool)
    active = m.any(axis=-1) if m.ndim == 2 else m
    order = np.argsort(-active.astype(np.int32), kind="stable").astype(np.int32)
    return order, int(active.sum())


def stream_compact(keys, values, block_mask, block_size=BLOCK):
    """Materialised compaction: ``compaction.py:28-100``."""
    s, h, d = keys.shape
    nb = s // block_size
    order, n = stream_compact_indices(block_mask)
    kb = keys[: nb * block_size].reshape(nb, block_size, h, d)[order].copy()
    vb = values[: nb * block_size].reshape(nb, block_size, h, d)[order].copy()
    kb[n:] = 0
    vb[n:] = 0
    return kb, vb, order, n


def stream_decompact(compact, active_indices, num_active, num_blocks):
    """``compaction.py:103-154``: out[active[i]] = compact[i] if i < n else 0.

    The reference scatters with ``output.at[active_indices].set(...)``: a
    negative entry counts from the end (NumPy indexing), an entry still out
    of bounds is dropped (JAX scatter), and for repeated entries the order is
    left to the implementation; here positions are applied in order, so the
    last position i < n naming a block wins.
    """
    out = np.zeros((num_blocks,) + compact.shape[1:], dtype=compact.dtype)
    n = max(0, min(int(num_active), num_blocks))
    for i, j in enumerate(np.asarray(active_indices)[:n]):
        j = int(j)
        if -num_blocks <= j < 0:
            j += num_blocks
        if 0 <= j < num_blocks:
            out[j] = compact[i]
    return out


def exclusive_scan(counts):
    """``alltoallv.py:113-145`` known answer helper: [3,2,5,1] -> [0,3,5,10], 11."""
    c = np.asarray(counts, dtype=np.int64)
    off = np.concatenate([[0], np.cumsum(c)[:-1]])
    return off, int(c.sum())


# --------------------------------------------------------------------------
# Attention
# --------------------------------------------------------------------------
def attention_active_blocks(q, k, v, active_blocks, block_size=BLOCK, dtype=np.float64):
    """Softmax attention over the tokens of the given blocks, GQA aware.

    Semantics of ``adaptive_attention.py:46-120`` (loop over active blocks,
    logits q.k / sqrt(d), online softmax, o / l): in closed form, softmax over
    exactly the retained tokens.  No retained block gives zeros
    (``adaptive_attention.py:164-167``).  q: (Sq, Hq, D); k, v: (S, Hkv, D);
    query head hq reads kv head hq // (Hq / Hkv).  Returns (Sq, Hq, D).
    """
    sq, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    blocks = list(active_blocks)
    out = np.zeros((sq, hq, d), dtype=dtype)
    if not blocks:
        return out
    tok = np.concatenate([np.arange(b * block_size, (b + 1) * block_size) for b in blocks])
    kk = k[tok].astype(dtype)
    vv = v[tok].astype(dtype)
    qq = q.astype(dtype)
    for h in range(hq):
        kh = kk[:, h // g]
        logits = qq[:, h] @ kh.T / np.sqrt(dtype(d))
        logits -= logits.max(axis=1, keepdims=True)
        p = np.exp(logits)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h] = p @ vv[:, h // g]
    return out


def block_logits(q, keys, block_size=BLOCK, dtype=np.float64):
    """Attention logits q.k / sqrt(d) of every key row, per block and kv head.

    The logits of ``adaptive_attention.py:60-61`` (one head) and ``:103-104``
    (all heads) for every token instead of the retained blocks only.
    q: (Sq, Hq, D) with Hq a multiple of Hkv; keys: (S, Hkv, D).  Returns
    (nb, Hkv, block_size, Sq*G) with query row i = t*G + g (query head
    h*G + g of token t), the folded order of ``fold_gqa``.
    """
    s, hkv, d = keys.shape
    nb = s // block_size
    qf = fold_gqa(q, hkv).astype(dtype)          # (Sq*G, Hkv, D)
    kb = keys.astype(dtype).reshape(nb, block_size, hkv, d)
    return np.einsum("brhd,ihd->bhri", kb, qf) / np.sqrt(dtype(d))


def attention_per_head_predicated(q, k, v, block_mask, block_size=BLOCK, dtype=np.float64):
    """``sparse_attention.py:5-64``: per-head mask, masked logits -> -1e9.

    A head whose blocks are all masked gets uniform weights over every key,
    i.e. the mean of V (all logits equal -1e9).  block_mask: (nb, Hkv).
    """
    sq, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    nb = k.shape[0] // block_size
    m = np.asarray(block_mask, dtype=bool)
    out = np.zeros((sq, hq, d), dtype=dtype)
    qq = q.astype(dtype)
    kk = k.astype(dtype)
    vv = v.astype(dtype)
    for h in range(hq):
        hk = h // g
        keep = np.repeat(m[:, hk], block_size)[: nb * block_size]
        logits = qq[:, h] @ kk[: nb * block_size, hk].T / np.sqrt(dtype(d))
        logits = np.where(keep[None, :], logits, -1e9)
        logits -= logits.max(axis=1, keepdims=True)
        p = np.exp(logits)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h] = p @ vv[: nb * block_size, hk]
    return out


def attention_per_head_gated(q, k, v, block_mask, block_size=BLOCK, dtype=np.float64):
    """``sparse_attention.py:67-138`` kernel semantics: masked blocks gate the
    accumulators off, so an all-masked head returns 0 (r_out / max(r_sum, 1e-9))."""
    out = attention_per_head_predicated(q, k, v, block_mask, block_size, dtype)
    hkv = k.shape[1]
    g = q.shape[1] // hkv
    m = np.asarray(block_mask, dtype=bool)
    for h in range(q.shape[1]):
        if not m[:, h // g].any():
            out[:, h] = 0
    return out


def online_softmax_loop_fp32(q, k, v, active_indices, num_active, block_size=BLOCK):
    """fp32 restatement of ``adaptive_attention.py:90-120`` (``_multihead_loop``).

    m starts at -1e30; per active block: logits = q.k / sqrt(d) in fp32,
    running max, rescale, accumulate; result o / l cast to bf16 by the caller.
    GQA: kv head h serves query heads h*G .. h*G+G-1.  Used as the CPU
    restatement timed beside the GPU.
    """
    sq, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    q32 = q.astype(np.float32).reshape(sq, hkv, g, d)
    scale = np.sqrt(np.float32(d))
    m = np.full((sq, hkv, g), -1e30, dtype=np.float32)
    l = np.zeros((sq, hkv, g), dtype=np.float32)
    o = np.zeros((sq, hkv, g, d), dtype=np.float32)
    for i in range(num_active):
        b = int(active_indices[i])
        kb = k[b * block_size:(b + 1) * block_size].astype(np.float32)  # (BS, Hkv, D)
        vb = v[b * block_size:(b + 1) * block_size].astype(np.float32)
        logits = np.einsum("qhgd,khd->qhgk", q32, kb) / scale
        mb = logits.max(axis=-1)
        mn = np.maximum(m, mb)
        el = np.exp(logits - mn[..., None])
        ep = np.exp(m - mn)
        l = l * ep + el.sum(axis=-1)
        o = o * ep[..., None] + np.einsum("qhgk,khd->qhgd", el, vb)
        m = mn
    if num_active == 0:
        return np.zeros((sq, hq, d), dtype=np.float32)
    return (o / l[..., None]).reshape(sq, hq, d)


def next_bucket(n, buckets=(1, 2, 4, 8, 16, 32, 64, 128, 256, 512)):
    """``indirect_attention.py:20-26``."""
    for b in buckets:
        if b >= n:
            return b
    return n


def auto_tau_from_max_bounds(max_bounds):
    """mean - std over every (block, head) entry of the max bound:
    ``pipeline.py:174-176``.  ``jnp.std`` defaults to ddof=0, the population
    standard deviation, as ``np.std`` does."""
    mb = np.asarray(max_bounds, dtype=np.float64)
    return float(np.mean(mb) - np.std(mb))


def auto_tau(q, keys, block_size=BLOCK, dtype=np.float64):
    """mean - std of the per-(block, head) max bound: ``pipeline.py:168-176``
    (the max over queries is ``:173``)."""
    return auto_tau_from_max_bounds(nanmax_axis0(query_aware_bounds(q, keys, block_size, dtype)))


# --------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even), for building inputs the GPU sees
# --------------------------------------------------------------------------
def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = np.isnan(x)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 and return them as float32."""
    return bf16_bits_to_f32(to_bf16_bits(np.asarray(x, dtype=np.float32)))
