"""GPU: the reference's drop-in entry points, called through ``orthocache_amd``.

Each test calls a reference-named function (src/orthocache/__init__.py:5-23)
the way a reference caller would and compares its result with the oracle:

* masks (compute_query_aware_mask, compute_multiband_mask,
  generate_threshold_mask) bit for bit against ``O.mask_from_scores`` on the
  GPU's own fp32 scores, and against the literal masks of keys whose scores
  follow from their Walsh construction;
* attention entry points (indirect_attention_fori, adaptive_sparse_attention,
  orthocache_attention_partitioned, orthocache_forward(mode='sparse'))
  against the float64 oracle over the retained tokens;
* auto-tau (orthocache_forward(tau=None)) against the oracle's pinned
  mean - population-std on the same fp32 scores;
* the reference's C custom-call entry point (orthocache_compacted_attention)
  against the oracle and the reference's compiled CPU function.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from oracle import oc_oracle as O

pytestmark = pytest.mark.gpu


def np32(t):
    return t.detach().float().cpu().numpy()


def close(out, ref, rel):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(out - ref).max() / max(np.abs(ref).max(), 1e-6)
    assert err <= rel, f"max error {err:.3e} (tolerance {rel})"


def gap_threshold(scores, quantile):
    """A threshold halfway between two neighbouring distinct fp32 scores near
    the quantile, with a gap wide enough that fp32-vs-float64 rounding of the
    scores (rtol 1e-5) cannot move any score across it."""
    s = np.unique(np.asarray(scores, np.float64).ravel())
    i = int(quantile * (len(s) - 1))
    for j in sorted(range(1, len(s)), key=lambda j: abs(j - i)):
        lo, hi = s[j - 1], s[j]
        if hi - lo > 1e-4 * max(abs(lo), abs(hi), 1.0):
            return float((lo + hi) / 2)
    raise AssertionError("no separated pair of scores")


# ---------------------------------------------------------------- masks
def walsh_keys(dev, blocks, d):
    """K[t, :] = m + a w_1[t] s + c w_256[t] r per block (m, a, c), as in
    tests/test_oracle.py::walsh_keys: E_low = 512 a^2 d, E_high = 512 c^2 d,
    E_AC = 512 (a^2 + c^2) d, kbar = m."""
    t = np.arange(512)
    w1 = np.where(t % 2 == 0, 1.0, -1.0)
    w256 = np.where(t < 256, 1.0, -1.0)
    s = np.where(np.arange(d) % 3 == 0, -1.0, 1.0)
    r = np.where(np.arange(d) % 2 == 0, 1.0, -1.0)
    k = np.concatenate([np.asarray(m, np.float64)[None, :] + a * np.outer(w1, s) + c * np.outer(w256, r)
                        for m, a, c in blocks])
    return torch.from_numpy(k[:, None, :].astype(np.float32)).to(dev)


def test_masks_walsh_construction(dev):
    """q = [2, 0, ...], d = 64 (sqrt(d) = 8): with m0 = +-40 the bounds are
    [e, e, 10 + e, -10 + e], e = 2 sqrt(512 * 1.25 * 64) / 8 = 50.596, and
    zeta = [0.25, 4, 0.25, 0.25] (up to the 1e-6 in the denominator)."""
    import orthocache_amd as oc

    d = 64
    m = np.zeros(d)
    mp, mn = m.copy(), m.copy()
    mp[0], mn[0] = 40.0, -40.0
    k = walsh_keys(dev, [(m, 1.0, 0.5), (m, 0.5, 1.0), (mp, 1.0, 0.5), (mn, 1.0, 0.5)], d)
    q = torch.zeros(1, 1, d, device=dev)
    q[0, 0, 0] = 2.0
    e = 2 * math.sqrt(512 * 1.25 * 64) / 8
    np.testing.assert_allclose(np32(oc.compute_query_aware_bounds(q, k))[0, :, 0], [e, e, 10 + e, -10 + e],
                               rtol=1e-5)
    assert np32(oc.compute_query_aware_mask(q, k, 55.0))[:, 0].tolist() == [False, False, True, False]
    assert np32(oc.compute_query_aware_mask(q, k, 45.0))[:, 0].tolist() == [True, True, True, False]
    assert np32(oc.compute_multiband_mask(q, k, 45.0, 1.0))[:, 0].tolist() == [True, False, True, False]
    assert np32(oc.compute_multiband_mask(q, k, 45.0, 5.0))[:, 0].tolist() == [True, True, True, False]
    q2 = torch.cat([q, -q])
    assert np32(oc.compute_multiband_mask(q2, k, 55.0, 1.0))[:, 0].tolist() == [False, False, True, True]
    m_gpu = oc.compute_multiband_mask(q, k, 45.0, 1.0)
    assert m_gpu.dtype == torch.bool and tuple(m_gpu.shape) == (4, 1)


def test_masks_two_gate_reference_case(dev):
    """tests/test_spectral_bands.py:177-213 regenerated from its seed, with
    block 1 replaced by the reference's Walsh-coherent block
    (tests/test_spectral_bands.py:89-117); exact masks as in the oracle test."""
    import orthocache_amd as oc
    from scipy.linalg import hadamard

    np.random.seed(42)
    keys = np.random.randn(1024, 1, 64).astype(np.float32)
    for i in range(512):
        keys[i, 0, :] *= (1.0 if i % 2 == 0 else -1.0) * 5.0
    q = np.random.randn(1, 1, 64).astype(np.float32)
    kg, qg = torch.from_numpy(keys).to(dev), torch.from_numpy(q).to(dev)
    assert np32(oc.compute_multiband_mask(qg, kg, -100.0, 1.0)).tolist() == [[False], [False]]
    h = hadamard(512).astype(np.float64)
    rng = np.random.RandomState(42)
    coh = np.zeros((512, 64))
    for j in range(1, 16):
        coh += np.outer(h[:, j], rng.randn(64) * 0.5)
    keys[512:, 0, :] = coh.astype(np.float32)
    kg = torch.from_numpy(keys).to(dev)
    assert np32(oc.compute_multiband_mask(qg, kg, -100.0, 1.0)).tolist() == [[False], [True]]
    assert np32(oc.compute_query_aware_mask(qg, kg, -100.0)).tolist() == [[True], [True]]
    np.testing.assert_array_equal(np32(oc.compute_multiband_mask(qg, kg, -100.0, 1.0)).astype(bool),
                                  O.multiband_mask(q, keys, -100.0, 1.0))


@pytest.mark.parametrize("evict", [0.5, 0.9])
def test_masks_c2_shape(dev, evict):
    """C2 (64K tokens, 32 q / 16 kv heads, d = 256, bf16): the API masks equal
    the oracle's two-gate compare on the GPU's own fp32 scores, bit for bit;
    the scores of sampled blocks agree with the float64 oracle."""
    import orthocache_amd as oc
    from orthocache_amd import _ops, workloads

    wl = workloads.c2(dev)
    sc = _ops.score(wl.k, wl.q)
    tm, z = np32(sc.tau_max[0]), np32(sc.zeta)
    tau = gap_threshold(tm, evict)
    zmax = gap_threshold(z, 0.6)  # gate 2 evicts ~40% of the entries
    qa = oc.compute_query_aware_mask(wl.q, wl.k, tau)
    mb = oc.compute_multiband_mask(wl.q, wl.k, tau, zmax)
    torch.cuda.synchronize()
    assert qa.dtype == torch.bool and tuple(qa.shape) == (128, 16)
    np.testing.assert_array_equal(np32(qa).astype(bool), O.mask_from_scores(tm, np.zeros_like(z), tau, 0.0))
    np.testing.assert_array_equal(np32(mb).astype(bool), O.mask_from_scores(tm, z, tau, zmax))
    assert 0 < np32(mb).sum() <= np32(qa).sum() < qa.numel()
    if evict == 0.5:
        # both gates bite (at 90% eviction the kept tiles are the noise-injected
        # blocks, whose energy sits in the low band: gate 2 passes them all)
        assert np32(mb).sum() < np32(qa).sum()
    # the float64 oracle agrees on sampled blocks
    kk = wl.k.reshape(128, 512, 16, 256)
    qf = O.fold_gqa(np32(wl.q), 16)
    for b in (0, 41, 127):
        kb = np32(kk[b])
        np.testing.assert_allclose(z[b], O.spectral_decay_ratio(kb)[0], rtol=1e-5)
        np.testing.assert_allclose(tm[b], O.query_aware_bounds(qf, kb).max(axis=0)[0], rtol=1e-5, atol=1e-5)
        np.testing.assert_array_equal(np32(mb)[b].astype(bool), O.multiband_mask(qf, kb, tau, zmax)[0])


def test_masks_many_queries(dev):
    """512 queries (C4's chunk, 8 kv heads, d = 128): the bound runs on the
    tiled kernel and the mask reduces 64-query tile maxima with a
    NaN-propagating max.  One query of head 3 is NaN, so every block of head
    3 is evicted (jnp.max propagates NaN; NaN >= tau is False)."""
    import orthocache_amd as oc
    from orthocache_amd import workloads

    wl = workloads.c4(dev)
    q = wl.q.clone()
    q[300, 3, :] = float("nan")
    b = oc.compute_query_aware_bounds(q, wl.k)
    z = oc.compute_spectral_decay_ratio(wl.k)
    torch.cuda.synchronize()
    bn = np32(b)
    assert bn.shape == (512, 256, 8)
    tmax = O.nanmax_axis0(bn)
    assert np.isnan(tmax[:, 3]).all() and not np.isnan(np.delete(tmax, 3, axis=1)).any()
    ok = np.delete(tmax, 3, axis=1)
    tau = gap_threshold(ok, 0.75)
    zmax = gap_threshold(np32(z), 0.9)
    qa = np32(oc.compute_query_aware_mask(q, wl.k, tau)).astype(bool)
    mb = np32(oc.compute_multiband_mask(q, wl.k, tau, zmax)).astype(bool)
    np.testing.assert_array_equal(qa, O.mask_from_scores(tmax, np.zeros_like(tmax), tau, 0.0))
    np.testing.assert_array_equal(mb, O.mask_from_scores(tmax, np32(z), tau, zmax))
    assert not qa[:, 3].any() and qa.any()
    # bounds of sampled blocks against the float64 oracle (NaN where the oracle has NaN)
    kk = wl.k.reshape(256, 512, 8, 128)
    qn = np32(q)
    for blk in (0, 128, 255):
        ref = O.query_aware_bounds(qn, np32(kk[blk]))[:, 0, :]
        got = bn[:, blk, :]
        assert np.array_equal(np.isnan(got), np.isnan(ref))
        fin = ~np.isnan(ref)
        np.testing.assert_allclose(got[fin], ref[fin], rtol=1e-5, atol=1e-5)


def test_generate_threshold_mask_kat(dev):
    """tests/test_energy.py:73-79, then chained after compute_block_energy_jax."""
    import orthocache_amd as oc

    e = torch.tensor([[10.5, 2.3], [1.1, 15.6]], device=dev)
    assert oc.generate_threshold_mask(e, 5.0).cpu().tolist() == [[True, False], [False, True]]
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    k = torch.randn(4 * 512, 2, 64, generator=g, device=dev)
    k[512:1024, 1] *= 0.1
    en = oc.compute_block_energy_jax(k)
    kn = np32(k)
    np.testing.assert_allclose(np32(en), O.block_energy(kn), rtol=1e-5)
    eps = gap_threshold(np32(en), 0.3)
    np.testing.assert_array_equal(np32(oc.generate_threshold_mask(en, eps)).astype(bool),
                                  O.threshold_mask(O.block_energy(kn), eps))


# ------------------------------------------------------------ attention
def _qkv(dev, nb, sq, hq, hkv, d, dtype, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = (torch.randn(sq, hq, d, generator=g, device=dev) / math.sqrt(d)).to(dtype)
    k = torch.randn(nb * 512, hkv, d, generator=g, device=dev).to(dtype)
    v = torch.randn(nb * 512, hkv, d, generator=g, device=dev).to(dtype)
    return q, k, v


@pytest.mark.parametrize("sq,hq,hkv,d", [(1, 8, 4, 128), (2, 4, 4, 64), (64, 8, 2, 128)])
def test_indirect_attention_fori(dev, sq, hq, hkv, d):
    """The loop-indirection entry point the reference __init__ names
    (src/orthocache/__init__.py:19): bf16 output over exactly the blocks any
    head keeps.  64 queries x 4 rows per kv head take the MFMA kernels."""
    import orthocache_amd as oc

    nb = 10
    q, k, v = _qkv(dev, nb, sq, hq, hkv, d, torch.bfloat16, seed=sq * 7 + hq)
    rng = np.random.default_rng(sq + hq)
    m = rng.random((nb, hkv)) < 0.25
    m[3, 0] = True
    out = oc.indirect_attention_fori(q, k, v, torch.from_numpy(m).to(dev))
    assert out.dtype == torch.bfloat16 and out.shape == q.shape
    order, n = O.stream_compact_indices(m)
    close(np32(out), O.attention_active_blocks(np32(q), np32(k), np32(v), order[:n]), 1e-2)
    zero = oc.indirect_attention_fori(q, k, v, torch.zeros(nb, hkv, dtype=torch.bool, device=dev))
    assert float(zero.float().abs().sum()) == 0.0


def test_adaptive_sparse_attention(dev):
    """``adaptive_sparse_attention`` (src/orthocache/__init__.py:20, the
    adaptive dispatcher): 1-D block mask, bf16 output and the reference's
    stats keys; full eviction gives zeros and path 'zero'."""
    import orthocache_amd as oc

    nb, hkv, d = 40, 4, 128  # 20480 tokens > _SEQ_THRESHOLD: the multi-head path label
    q, k, v = _qkv(dev, nb, 1, 8, hkv, d, torch.bfloat16, seed=3)
    m = np.zeros(nb, bool)
    m[[0, 7, 8, 21, 39]] = True
    out, stats = oc.adaptive_sparse_attention(q, k, v, torch.from_numpy(m).to(dev))
    assert stats["num_active"] == 5 and stats["num_blocks"] == nb and stats["path"] == "multihead_loop"
    assert stats["eviction_rate"] == pytest.approx(1 - 5 / nb)
    assert out.dtype == torch.bfloat16
    close(np32(out), O.attention_active_blocks(np32(q), np32(k), np32(v), [0, 7, 8, 21, 39]), 1e-2)
    q2, k2, v2 = _qkv(dev, 8, 1, 2, 2, 64, torch.bfloat16, seed=4)
    m2 = torch.tensor([True, False, False, True, False, False, False, True], device=dev)
    out2, st2 = oc.adaptive_sparse_attention(q2, k2, v2, m2)
    assert st2["path"] == "vmap_heads" and st2["num_active"] == 3
    close(np32(out2), O.attention_active_blocks(np32(q2), np32(k2), np32(v2), [0, 3, 7]), 1e-2)
    out3, st3 = oc.adaptive_sparse_attention(q2, k2, v2, torch.zeros(8, dtype=torch.bool, device=dev))
    assert st3 == {"num_active": 0, "eviction_rate": 1.0, "path": "zero"}
    assert float(out3.float().abs().sum()) == 0.0


def test_orthocache_attention_partitioned(dev):
    """src/orthocache/partitioning.py:38-44: compact_and_attend's output, in
    q's dtype, over the blocks any head keeps."""
    import orthocache_amd as oc

    q, k, v = _qkv(dev, 6, 3, 4, 2, 64, torch.float32, seed=9)
    m = torch.tensor([[True, False], [False, False], [False, True], [False, False], [True, True], [False, False]],
                     device=dev)
    out = oc.orthocache_attention_partitioned(q, k, v, m)
    assert out.dtype == torch.float32 and out.shape == q.shape
    close(np32(out), O.attention_active_blocks(np32(q), np32(k), np32(v), [0, 2, 4]), 1e-4)
    ref, _ = oc.compact_and_attend(q, k, v, m)
    assert torch.equal(out, ref)


def test_orthocache_attention_partitioned_head_shards(dev):
    """partitioning.py:20-50's sharding rule 'q h d, k h d, k h d, b h -> q h d':
    with two head shards each shard compacts over its own kv head's mask, so
    shard 0 (q heads 0-1, kv head 0) attends blocks {0, 4} and shard 1 (q heads
    2-3, kv head 1) blocks {2, 4}; uneven splits are refused."""
    import orthocache_amd as oc

    q, k, v = _qkv(dev, 6, 3, 4, 2, 64, torch.float32, seed=9)
    m = torch.tensor([[True, False], [False, False], [False, True], [False, False], [True, True], [False, False]],
                     device=dev)
    out = oc.orthocache_attention_partitioned(q, k, v, m, num_shards=2)
    assert out.dtype == torch.float32 and out.shape == q.shape
    qn, kn, vn = np32(q), np32(k), np32(v)
    close(np32(out[:, :2]), O.attention_active_blocks(qn[:, :2], kn[:, :1], vn[:, :1], [0, 4]), 1e-4)
    close(np32(out[:, 2:]), O.attention_active_blocks(qn[:, 2:], kn[:, 1:], vn[:, 1:], [2, 4]), 1e-4)
    whole = oc.orthocache_attention_partitioned(q, k, v, m, num_shards=1)
    assert not torch.equal(out, whole)
    with pytest.raises(ValueError, match="split evenly"):
        oc.orthocache_attention_partitioned(q, k, v, m, num_shards=3)


def test_forward_sparse_mode_output(dev):
    """orthocache_forward(mode='sparse') (pipeline.py:146-148): each head
    attends its own kept blocks; a head keeping none returns zeros (the gated
    kernel).  Compared with the oracle's per-head gated attention on the mask
    the oracle draws from the GPU's own scores."""
    import orthocache_amd as oc
    from orthocache_amd import _ops

    g = torch.Generator(device=dev)
    g.manual_seed(17)
    nb, h, d = 8, 4, 64
    q = torch.randn(2, h, d, generator=g, device=dev)
    k = torch.randn(nb * 512, h, d, generator=g, device=dev)
    v = torch.randn(nb * 512, h, d, generator=g, device=dev)
    k[:, 2] *= 0.01  # head 2's bounds sit far below the others: it keeps nothing
    sc = _ops.score(k, q)
    tm, z = np32(sc.tau_max[0]), np32(sc.zeta)
    tau = gap_threshold(np.delete(tm, 2, axis=1), 0.5)
    zmax = gap_threshold(z, 0.8)
    out, meta = oc.orthocache_forward(q, k, v, zeta_max=zmax, tau=tau, mode="sparse")
    mask = O.mask_from_scores(tm, z, tau, zmax)
    assert not mask[:, 2].any() and mask.any()
    assert meta["blocks_retained"] == int(mask.any(axis=1).sum())
    ref = O.attention_per_head_gated(np32(q), np32(k), np32(v), mask)
    close(np32(out), ref, 1e-4)
    assert float(out[:, 2].abs().sum()) == 0.0
    # the compact mode on the same scores attends the union of the heads' blocks
    outc, _ = oc.orthocache_forward(q, k, v, zeta_max=zmax, tau=tau, mode="compact")
    order, n = O.stream_compact_indices(mask)
    close(np32(outc), O.attention_active_blocks(np32(q), np32(k), np32(v), order[:n]), 1e-4)


def test_forward_auto_tau(dev):
    """tau=None: mean - population std of the max bound per (block, head)
    (pipeline.py:168-176), from the GPU's fp32 scores; the oracle's pinned
    statistic on the same scores, and the float64 oracle end to end."""
    import orthocache_amd as oc
    from orthocache_amd import _ops

    g = torch.Generator(device=dev)
    g.manual_seed(23)
    nb, h, d = 6, 2, 64
    q = torch.randn(3, h, d, generator=g, device=dev)
    k = torch.randn(nb * 512, h, d, generator=g, device=dev) + 0.2
    v = torch.randn(nb * 512, h, d, generator=g, device=dev)
    out, meta = oc.orthocache_forward(q, k, v, zeta_max=10.0, tau=None, mode="compact")
    assert meta["tau_auto"] is True
    sc = _ops.score(k, q)
    tm, z = np32(sc.tau_max[0]), np32(sc.zeta)
    assert meta["tau"] == pytest.approx(O.auto_tau_from_max_bounds(tm), rel=1e-5)
    assert meta["tau"] == pytest.approx(O.auto_tau(np32(q), np32(k)), rel=1e-4)
    mask = O.mask_from_scores(tm, z, meta["tau"], 10.0)
    order, n = O.stream_compact_indices(mask)
    assert meta["blocks_retained"] == n
    close(np32(out), O.attention_active_blocks(np32(q), np32(k), np32(v), order[:n]), 1e-4)


class _CADesc(ctypes.Structure):
    # notebooks/phase_d_kaggle.py:211-217 (CompactedAttentionDescriptor)
    _fields_ = [("seq_len_q", ctypes.c_int32), ("seq_len_k", ctypes.c_int32), ("head_dim", ctypes.c_int32),
                ("block_size", ctypes.c_int32), ("num_blocks", ctypes.c_int32)]


def _custom_call(q, k, v, m, bs, out):
    from orthocache_amd import _native as N

    L = N.lib()
    desc = _CADesc(q.shape[0], k.shape[0], q.shape[1], bs, m.shape[0])
    ins = (ctypes.c_void_p * 5)(q.data_ptr(), k.data_ptr(), v.data_ptr(), m.data_ptr(), ctypes.addressof(desc))
    L.orthocache_compacted_attention(ctypes.c_void_p(out.data_ptr()), ins)


@pytest.mark.parametrize("sq,d,bs,nb", [(1, 128, 512, 8), (7, 64, 128, 12), (33, 256, 64, 5), (4, 32, 512, 3),
                                        (600, 128, 256, 4), (2, 64, 64, 3000)])
def test_reference_custom_call_entry_point(dev, sq, d, bs, nb):
    """orthocache_compacted_attention under the reference's own signature
    (notebooks/phase_d_kaggle.py:211-222) on device buffers: against the
    float64 oracle and, where it is built, the reference's compiled CPU
    function on the same inputs."""
    from oracle import native

    g = torch.Generator(device=dev)
    g.manual_seed(sq * 31 + nb)
    q = torch.randn(sq, d, generator=g, device=dev) / math.sqrt(d)
    k = torch.randn(nb * bs, d, generator=g, device=dev)
    v = torch.randn(nb * bs, d, generator=g, device=dev)
    rng = np.random.default_rng(nb + d)
    m = (rng.random(nb) < 0.5).astype(np.int32) * rng.integers(1, 5, nb).astype(np.int32)  # any nonzero is active
    m[rng.integers(nb)] = -3
    md = torch.from_numpy(m).to(dev)
    out = torch.full((sq, d), float("nan"), device=dev)
    _custom_call(q, k, v, md, bs, out)
    active = np.flatnonzero(m)
    ref = O.attention_active_blocks(np32(q)[:, None], np32(k)[:, None], np32(v)[:, None], active, block_size=bs)[:, 0]
    close(np32(out), ref, 1e-4)
    if native.ref_available():
        close(np32(out), native.ref_compacted_attention(np32(q), np32(k), np32(v), m, block_size=bs), 1e-4)


def test_reference_custom_call_no_active_block(dev):
    """No active block (and no block at all) gives zero rows, as the
    reference's r_sum guard does; a descriptor whose seq_len_k is not
    num_blocks * block_size is refused and out is left alone."""
    from orthocache_amd import _native as N

    q = torch.randn(3, 64, device=dev)
    k = torch.randn(4 * 128, 64, device=dev)
    v = torch.randn(4 * 128, 64, device=dev)
    out = torch.full((3, 64), float("nan"), device=dev)
    _custom_call(q, k, v, torch.zeros(4, dtype=torch.int32, device=dev), 128, out)
    assert float(out.abs().sum()) == 0.0
    out.fill_(float("nan"))
    _custom_call(q, k[:0], v[:0], torch.zeros(0, dtype=torch.int32, device=dev), 128, out)
    assert float(out.abs().sum()) == 0.0
    out.fill_(float("nan"))
    _custom_call(q, k[:300], v[:300], torch.ones(4, dtype=torch.int32, device=dev), 128, out)
    assert torch.isnan(out).all()
    assert b"seq_len_k" in N.lib().oc_last_error()
