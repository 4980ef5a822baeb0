"""GPU parity: paged K/V caches (page pools + block tables).

The page list only changes where a block's keys and values are read, never
the arithmetic, so every paged result must equal the contiguous-cache result
bit for bit: scores, masks, permutations, counts and attention outputs, for
the decode layer, the MFMA prefill kernels, write-time statistics and the
cached decode step.  The contiguous results themselves are pinned against the
oracle in the other test files.
"""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


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
