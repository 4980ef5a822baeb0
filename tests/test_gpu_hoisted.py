"""GPU parity: decode with the scoring hoisted to cache-write time.

Write-time statistics (dc, E_AC, zeta from one scoring pass over new blocks)
are checked against the float64 oracle and must be the same bits whether the
cache is scored at once or block range by block range.  The cached decode
step (oc_decode_layer_cached) must publish bounds within the scores'
tolerance of the oracle, a mask and permutation bit-exact with the oracle's on
its own fp32 scores, and attention within the bf16 tolerance.
"""

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
    scale = max(np.abs(ref).max(), 1e-6)
    err = np.abs(out - ref).max() / scale
    assert err <= rel, f"max error {err:.3e} relative to output scale (tolerance {rel})"


def test_block_stats_vs_oracle(dev):
    import orthocache_amd as oc
    from orthocache_amd import workloads

    k = workloads.make_keys(6, 4, 128, seed=31, device=dev, noise_frac=0.3)
    st = oc.block_stats(k)
    kn = np32(k)
    np.testing.assert_allclose(np32(st.zeta), O.spectral_decay_ratio(kn), rtol=1e-5, atol=1e-6)
    dc, lo, mi, hi = O.spectral_bands(kn.astype(np.float64))
    np.testing.assert_allclose(np32(st.dc), dc, rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(np32(st.e_ac), lo + mi + hi, rtol=1e-5)


def test_incremental_update_is_bit_identical(dev):
    import orthocache_amd as oc
    from orthocache_amd import workloads

    k = workloads.make_keys(10, 2, 256, seed=32, device=dev)
    full = oc.block_stats(k)
    inc = oc.block_stats(k[: 3 * 512], capacity_blocks=10)
    inc.update(k, 3, 4)   # blocks 3..6
    inc.update(k, 7)      # the rest
    torch.cuda.synchronize()
    for a, b in ((full.dc, inc.dc), (full.e_ac, inc.e_ac), (full.zeta, inc.zeta)):
        assert torch.equal(a, b)
    with pytest.raises(ValueError):
        inc.update(k, 9, 2)


@pytest.mark.parametrize("evict", [0.5, 0.9])
def test_cached_layer_c2(dev, evict):
    import orthocache_amd as oc
    from orthocache_amd import _ops, workloads

    wl = workloads.c2(dev, seq=16384)
    sc = _ops.score(wl.k, wl.q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, evict)
    st = oc.block_stats(wl.k)
    layer = oc.CachedDecodeLayer(wl.q, wl.k, wl.v, st, tau, zmax, out_dtype=torch.float32)
    out = layer.run()
    torch.cuda.synchronize()
    qf = O.fold_gqa(np32(wl.q), wl.k.shape[1])
    kn = np32(wl.k)
    tm = np32(layer.tau_max)
    np.testing.assert_allclose(tm, O.query_aware_bounds(qf, kn).max(axis=0), rtol=1e-5, atol=1e-5)
    # cached zeta is the scoring kernel's, bit for bit
    assert torch.equal(st.zeta, sc.zeta)
    mask = O.mask_from_scores(tm, np32(st.zeta), tau, zmax)
    order, n = O.stream_compact_indices(mask)
    np.testing.assert_array_equal(np32(layer.indices).astype(np.int64), order)
    assert int(layer.num_active[0]) == n
    ref = O.attention_active_blocks(np32(wl.q), kn, np32(wl.v), order[:n])
    close(np32(out), ref, 2e-3)
    # and the keys-reading layer on the same inputs gives the same result
    full = _ops.DecodeLayer(wl.q, wl.k, wl.v, tau, zmax, out_dtype=torch.float32)
    out_full = full.run()
    torch.cuda.synchronize()
    if torch.equal(full.indices, layer.indices):
        close(np32(out), np32(out_full), 1e-5)


def test_cached_layer_ragged_segments(dev):
    import orthocache_amd as oc
    from orthocache_amd import varlen, workloads

    wl = workloads.c3(dev, batch=6, lo=2048, hi=8192)
    cu = wl.cu_seqlens.cpu().numpy() // 512
    tm0, z0 = varlen.score_varlen(wl.q, wl.k, wl.cu_seqlens)
    taus, zmaxs = [], []
    for s in range(len(wl.meta["lens"])):
        t, zm = workloads.calibrate_unified(tm0[cu[s]:cu[s + 1]], z0[cu[s]:cu[s + 1]], wl.meta["evict"][s])
        taus.append(t)
        zmaxs.append(zm)
    tau_t = torch.tensor(taus, dtype=torch.float32, device=dev)
    zmax_t = torch.tensor(zmaxs, dtype=torch.float32, device=dev)
    st = oc.block_stats(wl.k)
    layer = oc.CachedDecodeLayer(wl.q, wl.k, wl.v, st, tau_t, zmax_t, cu_blocks=varlen.cu_blocks_from_seqlens(wl.cu_seqlens),
                                 num_segments=len(wl.meta["lens"]), out_dtype=torch.float32)
    out = layer.run()
    torch.cuda.synchronize()
    tm, zn, idx = np32(layer.tau_max), np32(st.zeta), np32(layer.indices).astype(np.int64)
    for s in range(len(wl.meta["lens"])):
        lo, hi = cu[s], cu[s + 1]
        kseg = np32(wl.k[lo * 512:hi * 512])
        qf = O.fold_gqa(np32(wl.q[s]), wl.k.shape[1])
        np.testing.assert_allclose(tm[lo:hi], O.query_aware_bounds(qf, kseg).max(axis=0), rtol=1e-5, atol=1e-5)
        mask = O.mask_from_scores(tm[lo:hi], zn[lo:hi], taus[s], zmaxs[s])
        order, n = O.stream_compact_indices(mask)
        np.testing.assert_array_equal(idx[lo:hi], order)
        assert int(layer.num_active[s]) == n
        ref = O.attention_active_blocks(np32(wl.q[s]), kseg, np32(wl.v[lo * 512:hi * 512]), order[:n])
        close(np32(out[s]), ref, 2e-3)


def test_cached_layer_rejects_short_stats(dev):
    import orthocache_amd as oc
    from orthocache_amd import workloads

    wl = workloads.c2(dev, seq=4096)
    st = oc.block_stats(wl.k[:2048])
    with pytest.raises(ValueError):
        oc.CachedDecodeLayer(wl.q, wl.k, wl.v, st, 0.0, 1.0)
