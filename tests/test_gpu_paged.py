"""GPU parity: paged K/V caches (page pools + block tables).

The page list only changes where a block's keys and values are read, never
the arithmetic, so every paged result must equal the contiguous-cache result
bit for bit: scores, masks, permutations, counts and attention outputs, for
the decode layer, the MFMA prefill kernels, write-time statistics and the
cached decode step.  The paged results are also checked against the oracle
directly, on the logical blocks gathered from the pool on the host
(active_indices is a page list, src/orthocache/compaction.py:65-82), so a
page-addressing mistake shared by the paged and contiguous paths would fail.
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
    err = np.abs(out - ref).max() / max(np.abs(ref).max(), 1e-6)
    assert err <= rel, f"max error {err:.3e} (tolerance {rel})"


def _logical(pool, pages):
    """(total_blocks * 512, H, D) float32 host array: logical block j is
    pool page pages[j], gathered on the host."""
    p = np32(pool)
    pg = pages.cpu().numpy().astype(np.int64)
    return p.reshape(-1, 512, *p.shape[1:])[pg].reshape(-1, *p.shape[1:])


def _pool(dev, k, v, extra_pages, seed):
    """Scatter the contiguous caches' blocks over a larger pool in a random
    order; return (k_pool, v_pool, pages)."""
    nb = k.shape[0] // 512
    g = torch.Generator()
    g.manual_seed(seed)
    npages = nb + extra_pages
    pages = torch.randperm(npages, generator=g)[:nb].to(torch.int32).to(dev)
    shape = (npages * 512,) + tuple(k.shape[1:])
    k_pool = torch.randn(shape, device=dev).to(k.dtype)   # unused pages hold noise
    v_pool = torch.randn(shape, device=dev).to(v.dtype)
    k_pool.view(npages, 512, *k.shape[1:])[pages.long()] = k.view(nb, 512, *k.shape[1:])
    v_pool.view(npages, 512, *v.shape[1:])[pages.long()] = v.view(nb, 512, *v.shape[1:])
    return k_pool, v_pool, pages


def _thresholds(dev, wl, tm, z, cu):
    from orthocache_amd import workloads

    taus, zmaxs = [], []
    for s in range(len(wl.meta["lens"])):
        t, zm = workloads.calibrate_unified(tm[cu[s]:cu[s + 1]], z[cu[s]:cu[s + 1]], wl.meta["evict"][s])
        taus.append(t)
        zmaxs.append(zm)
    return (torch.tensor(taus, dtype=torch.float32, device=dev), torch.tensor(zmaxs, dtype=torch.float32, device=dev))


def test_flatten_block_table(dev):
    import orthocache_amd as oc

    bt = torch.tensor([[7, 3, -1, -1], [0, 9, 4, 2], [5, -1, -1, -1]], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 2, 6, 7], dtype=torch.int32, device=dev)
    pages = oc.flatten_block_table(bt, cu, 7)
    assert pages.dtype == torch.int32
    assert pages.cpu().tolist() == [7, 3, 0, 9, 4, 2, 5]


def test_paged_decode_layer_equals_contiguous(dev):
    import orthocache_amd as oc
    from orthocache_amd import _ops, varlen, workloads

    wl = workloads.c3(dev, batch=5, lo=2048, hi=6144)
    cu = wl.cu_seqlens.cpu().numpy() // 512
    nb = int(cu[-1])
    tm, z = varlen.score_varlen(wl.q, wl.k, wl.cu_seqlens)
    tau_t, zmax_t = _thresholds(dev, wl, tm, z, cu)
    cu_blocks = varlen.cu_blocks_from_seqlens(wl.cu_seqlens)
    ref = _ops.DecodeLayer(wl.q, wl.k, wl.v, tau_t, zmax_t, cu_blocks=cu_blocks, num_segments=5,
                           out_dtype=torch.float32)
    ref_out = ref.run()
    k_pool, v_pool, pages = _pool(dev, wl.k, wl.v, extra_pages=11, seed=41)
    # the same pages as a vLLM-style block table, padded with -1
    lens_b = np.diff(cu)
    bt = torch.full((5, int(lens_b.max()) + 2), -1, dtype=torch.int32)
    pl = pages.cpu()
    for s in range(5):
        bt[s, :lens_b[s]] = pl[cu[s]:cu[s + 1]]
    out, meta = oc.orthocache_decode_paged(wl.q, k_pool, v_pool, bt.to(dev), wl.cu_seqlens, tau_t, zmax_t,
                                           total_blocks=nb, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(meta["pages"], pages)
    assert torch.equal(meta["tau_max"], ref.tau_max)
    assert torch.equal(meta["zeta"], ref.zeta)
    assert torch.equal(meta["indices"], ref.indices)
    assert torch.equal(meta["num_active"], ref.num_active)
    assert torch.equal(out, ref_out)


def test_paged_prefill_equals_contiguous(dev):
    from orthocache_amd import _ops, workloads

    nb, hkv, d = 12, 4, 128
    k = workloads.make_keys(nb, hkv, d, seed=42, device=dev)
    v = workloads.make_values(nb * 512, hkv, d, seed=43, device=dev)
    q = workloads.make_queries((96, 8, d), d, seed=44, device=dev)
    mask = torch.tensor([1, 0, 1, 1, 0, 1, 0, 0, 1, 1, 0, 1], dtype=torch.bool, device=dev)
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=mask)
    k_pool, v_pool, pages = _pool(dev, k, v, extra_pages=5, seed=45)
    assert _ops.attend_plan(q, k_pool, v_pool, c.indices, c.num_active, pages=pages)[0] == "prefill_mfma"
    ref = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    got = _ops.attend(q, k_pool, v_pool, c.indices, c.num_active, out_dtype=torch.float32, pages=pages)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_paged_stats_and_cached_layer(dev):
    import orthocache_amd as oc
    from orthocache_amd import _ops, workloads

    wl = workloads.c2(dev, seq=8192)
    sc = _ops.score(wl.k, wl.q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, 0.75)
    st = oc.block_stats(wl.k)
    k_pool, v_pool, pages = _pool(dev, wl.k, wl.v, extra_pages=3, seed=46)
    stp = oc.block_stats(k_pool, pages=pages)
    torch.cuda.synchronize()
    assert torch.equal(stp.dc, st.dc) and torch.equal(stp.e_ac, st.e_ac) and torch.equal(stp.zeta, st.zeta)
    ref = oc.CachedDecodeLayer(wl.q, wl.k, wl.v, st, tau, zmax, out_dtype=torch.float32)
    got = oc.CachedDecodeLayer(wl.q, k_pool, v_pool, stp, tau, zmax, out_dtype=torch.float32, pages=pages)
    a, b = ref.run(), got.run()
    torch.cuda.synchronize()
    assert torch.equal(ref.indices, got.indices)
    assert torch.equal(a, b)
    # scores straight from the pool equal the contiguous scores
    scp = _ops.score(k_pool, wl.q, pages=pages)
    torch.cuda.synchronize()
    assert torch.equal(scp.tau_max, sc.tau_max) and torch.equal(scp.zeta, sc.zeta)


def test_pages_validation(dev):
    from orthocache_amd import _ops

    k = torch.zeros(1024, 2, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        _ops.score(k, pages=torch.zeros(2, dtype=torch.int64, device=dev))
    with pytest.raises(ValueError):
        _ops.score(k, pages=torch.zeros((2, 1), dtype=torch.int32, device=dev))


def test_paged_decode_layer_vs_oracle(dev):
    """A ragged batch of 6 sequences whose blocks sit in a shuffled pool
    with 9 unused noise pages: scores of every block (rtol 1e-5), masks,
    permutations and counts (bit-exact on the layer's own scores) and every
    sequence's attention (bf16 inputs, fp32 output: 2e-3) against the oracle
    on the logically ordered caches."""
    import orthocache_amd as oc
    from orthocache_amd import varlen, workloads

    wl = workloads.c3(dev, seed=17, batch=6, lo=1024, hi=5120)
    cu = wl.cu_seqlens.cpu().numpy() // 512
    nb = int(cu[-1])
    tm, z = varlen.score_varlen(wl.q, wl.k, wl.cu_seqlens)
    tau_t, zmax_t = _thresholds(dev, wl, tm, z, cu)
    k_pool, v_pool, pages = _pool(dev, wl.k, wl.v, extra_pages=9, seed=53)
    lens_b = np.diff(cu)
    bt = torch.full((6, int(lens_b.max())), -1, dtype=torch.int32)
    pl = pages.cpu()
    for s in range(6):
        bt[s, :lens_b[s]] = pl[cu[s]:cu[s + 1]]
    out, meta = oc.orthocache_decode_paged(wl.q, k_pool, v_pool, bt.to(dev), wl.cu_seqlens, tau_t, zmax_t,
                                           total_blocks=nb, out_dtype=torch.float32)
    torch.cuda.synchronize()
    kl, vl = _logical(k_pool, pages), _logical(v_pool, pages)
    tmn, zn = np32(meta["tau_max"]), np32(meta["zeta"])
    idx, cnt = np32(meta["indices"]).astype(np.int64), np32(meta["num_active"]).astype(np.int64)
    taus, zmaxs = tau_t.cpu().numpy(), zmax_t.cpu().numpy()
    hkv = kl.shape[1]
    for s in range(6):
        lo, hi = cu[s], cu[s + 1]
        ks, vs = kl[lo * 512:hi * 512], vl[lo * 512:hi * 512]
        qs = np32(wl.q[s])
        np.testing.assert_allclose(zn[lo:hi], O.spectral_decay_ratio(ks), rtol=1e-5)
        np.testing.assert_allclose(tmn[lo:hi], O.query_aware_bounds(O.fold_gqa(qs, hkv), ks).max(axis=0),
                                   rtol=1e-5, atol=1e-5)
        mask = O.mask_from_scores(tmn[lo:hi], zn[lo:hi], float(taus[s]), float(zmaxs[s]))
        order, n = O.stream_compact_indices(mask)
        np.testing.assert_array_equal(idx[lo:hi], order)
        assert cnt[s] == n
        close(np32(out[s]), O.attention_active_blocks(qs, ks, vs, order[:n]), 2e-3)


def test_paged_prefill_vs_oracle(dev):
    """The MFMA prefill kernels reading a shuffled pool: output against the
    float64 oracle over the retained logical blocks (fp32 output with P
    rounded to bf16: 5e-3)."""
    from orthocache_amd import _ops, workloads

    nb, hkv, d = 10, 2, 128
    k = workloads.make_keys(nb, hkv, d, seed=61, device=dev)
    v = workloads.make_values(nb * 512, hkv, d, seed=62, device=dev)
    q = workloads.make_queries((80, 4, d), d, seed=63, device=dev)
    keep = [0, 2, 3, 7, 9]
    mask = torch.zeros(nb, dtype=torch.bool, device=dev)
    mask[keep] = True
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=mask)
    k_pool, v_pool, pages = _pool(dev, k, v, extra_pages=6, seed=64)
    assert _ops.attend_plan(q, k_pool, v_pool, c.indices, c.num_active, pages=pages)[0] == "prefill_mfma"
    got = _ops.attend(q, k_pool, v_pool, c.indices, c.num_active, out_dtype=torch.float32, pages=pages)
    torch.cuda.synchronize()
    ref = O.attention_active_blocks(np32(q), _logical(k_pool, pages), _logical(v_pool, pages), keep)
    close(np32(got), ref, 5e-3)
