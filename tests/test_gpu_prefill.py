"""GPU parity: the matrix-core (MFMA) prefill attention kernels.

Same semantics as the decode kernels (softmax over exactly the retained
blocks, fp32 softmax state); checked against the float64 oracle.  The P V
product takes P rounded to the input dtype (bf16/fp16), so with fp32 output
the tolerance is 5e-3 of the output scale instead of the decode kernel's 2e-3;
with bf16 output the north-star 1e-2 applies.
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
    return err


def make(dev, nb, sq, hq, hkv, d, dtype, seed, block=512, batch=None):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    qshape = (sq, hq, d) if batch is None else (batch, sq, hq, d)
    q = torch.randn(qshape, generator=g, device=dev).to(dtype)
    k = torch.randn(nb * block, hkv, d, generator=g, device=dev).to(dtype)
    v = torch.randn(nb * block, hkv, d, generator=g, device=dev).to(dtype)
    return q, k, v


def compact(dev, mask, hkv, **kw):
    from orthocache_amd import _ops

    return _ops.mask_compact(num_blocks=mask.shape[0], num_kv_heads=hkv, device=dev, mask_in=mask, **kw)


@pytest.mark.parametrize("sq,hq,hkv,d,dtype,nb", [
    (512, 8, 8, 128, torch.bfloat16, 16),   # C4 shape at reduced length
    (300, 4, 2, 128, torch.bfloat16, 9),    # GQA, 600 rows: last query tile partial
    (40, 2, 2, 64, torch.float16, 7),
    (33, 1, 1, 128, torch.bfloat16, 5),     # just above the 32-row threshold
    (32, 4, 1, 64, torch.bfloat16, 6),      # group 4: 128 rows, one tile
    (64, 16, 2, 128, torch.float16, 4),
    (128, 2, 2, 128, torch.bfloat16, 1),    # one block, fewer tiles than splits
])
def test_unified_vs_oracle(dev, sq, hq, hkv, d, dtype, nb):
    from orthocache_amd import _ops

    q, k, v = make(dev, nb, sq, hq, hkv, d, dtype, seed=sq + hq + d)
    rng = np.random.default_rng(sq)
    m = rng.random(nb) < 0.6
    m[rng.integers(nb)] = True
    mask = torch.from_numpy(m).to(dev)
    c = compact(dev, mask, hkv)
    plan = _ops.attend_plan(q, k, v, c.indices, c.num_active)
    assert plan[0] == "prefill_mfma" and plan[1] >= 1
    out = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    ref = O.attention_active_blocks(np32(q), np32(k), np32(v), np.flatnonzero(m))
    close(np32(out), ref, 5e-3)
    out16 = _ops.attend(q, k, v, c.indices, c.num_active)
    assert out16.dtype == dtype
    close(np32(out16), ref, 1e-2)


def test_half_partials_beyond_fp16_range(dev):
    """16-bit outputs merge the splits from fp16 partials scaled by each row's
    largest |o|: value columns near 4e4 (their unnormalised sums far beyond
    fp16's 65504) beside columns near 1 stay within the bf16 tolerance of the
    output scale, and the bf16 output agrees with the fp32-partial path."""
    from orthocache_amd import _ops

    nb, hkv = 12, 2
    q, k, v = make(dev, nb, 256, 2, hkv, 128, torch.bfloat16, seed=41)
    v = v.float()
    v[..., :64] *= 4e4
    v = v.to(torch.bfloat16)
    mask = torch.ones(nb, dtype=torch.bool, device=dev)
    c = compact(dev, mask, hkv)
    plan = _ops.attend_plan(q, k, v, c.indices, c.num_active)
    assert plan[0] == "prefill_mfma" and plan[1] > 1
    out16 = _ops.attend(q, k, v, c.indices, c.num_active)
    out32 = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    assert torch.isfinite(out16.float()).all()
    ref = O.attention_active_blocks(np32(q), np32(k), np32(v), range(nb))
    close(np32(out16), ref, 1e-2)
    close(np32(out16), np32(out32), 4e-3)


@pytest.mark.parametrize("ntiles", [1, 2, 3, 5, 7])
def test_short_tile_ranges(dev, ntiles):
    # 64-token blocks are one key tile each, and this shape gets a single
    # split, so the kernel walks exactly `ntiles` tiles: the software
    # pipeline's prologue, odd and even counts and its last two steps.
    from orthocache_amd import _ops

    bs = 64
    q, k, v = make(dev, ntiles, 64, 2, 2, 128, torch.bfloat16, seed=30 + ntiles, block=bs)
    mask = torch.ones(ntiles, dtype=torch.bool, device=dev)
    c = compact(dev, mask, 2)
    assert _ops.attend_plan(q, k, v, c.indices, c.num_active, block_size=bs) == ("prefill_mfma", 1)
    out = _ops.attend(q, k, v, c.indices, c.num_active, block_size=bs, out_dtype=torch.float32)
    ref = O.attention_active_blocks(np32(q), np32(k), np32(v), range(ntiles), block_size=bs)
    close(np32(out), ref, 5e-3)


def test_matches_decode_kernel(dev):
    # The same bf16 values through both kernel families: fp32 queries take the
    # decode kernel, bf16 queries the MFMA kernel.
    from orthocache_amd import _ops

    nb, hkv = 8, 2
    q, k, v = make(dev, nb, 96, 4, hkv, 128, torch.bfloat16, seed=11)
    mask = torch.tensor([1, 0, 1, 1, 0, 1, 0, 1], dtype=torch.bool, device=dev)
    c = compact(dev, mask, hkv)
    assert _ops.attend_plan(q.float(), k, v, c.indices, c.num_active)[0] == "decode"
    dec = _ops.attend(q.float(), k, v, c.indices, c.num_active, out_dtype=torch.float32)
    mma = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    close(np32(mma), np32(dec), 5e-3)


def test_empty_list_gives_zeros(dev):
    from orthocache_amd import _ops

    q, k, v = make(dev, 4, 64, 2, 2, 128, torch.bfloat16, seed=12)
    c = compact(dev, torch.zeros(4, dtype=torch.bool, device=dev), 2)
    out = _ops.attend(q, k, v, c.indices, c.num_active)
    assert float(out.float().abs().sum()) == 0.0


def test_per_head_predicated_and_gated(dev):
    import orthocache_amd as oc

    nb, hkv = 6, 2
    q, k, v = make(dev, nb, 64, 8, hkv, 128, torch.bfloat16, seed=13)
    m = np.zeros((nb, hkv), bool)
    m[[0, 2, 5], 0] = True  # kv head 1 keeps nothing
    mt = torch.from_numpy(m).to(dev)
    pred = oc.jax_block_sparse_attention(q, k, v, mt)
    gated = oc.compile_pallas_sparse_attention(q, k, v, mt)
    qn, kn, vn = np32(q), np32(k), np32(v)
    close(np32(pred), O.attention_per_head_predicated(qn, kn, vn, m), 1e-2)
    close(np32(gated), O.attention_per_head_gated(qn, kn, vn, m), 1e-2)
    assert float(gated[:, 4:].float().abs().sum()) == 0.0


def test_ragged_segments(dev):
    from orthocache_amd import _ops

    hkv, hq, d, sq = 2, 4, 128, 40
    seg_nb = [3, 1, 4, 2]
    cu = np.concatenate([[0], np.cumsum(seg_nb)]).astype(np.int32)
    nb = int(cu[-1])
    g = torch.Generator(device=dev)
    g.manual_seed(14)
    q = torch.randn(len(seg_nb), sq, hq, d, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(nb * 512, hkv, d, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(nb * 512, hkv, d, generator=g, device=dev).to(torch.bfloat16)
    m = np.array([1, 0, 1, 0, 1, 1, 0, 1, 0, 1], bool)
    m[cu[1]] = False  # segment 1 (one block) keeps nothing
    cu_t = torch.from_numpy(cu).to(dev)
    c = compact(dev, torch.from_numpy(m).to(dev), hkv, cu_blocks=cu_t, num_segments=len(seg_nb))
    kw = dict(cu_blocks=cu_t, num_segments=len(seg_nb), out_dtype=torch.float32)
    assert _ops.attend_plan(q, k, v, c.indices, c.num_active, **kw)[0] == "prefill_mfma"
    out = _ops.attend(q, k, v, c.indices, c.num_active, **kw)
    for s in range(len(seg_nb)):
        lo, hi = cu[s], cu[s + 1]
        act = [j for j in range(hi - lo) if m[lo + j]]
        if not act:
            assert float(out[s].abs().sum()) == 0.0
            continue
        ref = O.attention_active_blocks(np32(q[s]), np32(k[lo * 512:hi * 512]), np32(v[lo * 512:hi * 512]), act)
        close(np32(out[s]), ref, 5e-3)


def test_c4_full_size_sampled_rows(dev):
    """C4: 512 queries x 131072 keys (256 blocks), 8 kv heads, d=128, bf16,
    75% of blocks evicted.  Every row is computed; a seeded sample of query
    rows is checked against the float64 oracle, and a second launch must
    reproduce the first bit for bit."""
    from orthocache_amd import _ops

    nb, hkv, d, sq = 256, 8, 128, 512
    q, k, v = make(dev, nb, sq, hkv, hkv, d, torch.bfloat16, seed=15)
    rng = np.random.default_rng(15)
    m = np.zeros(nb, bool)
    m[rng.choice(nb, nb // 4, replace=False)] = True
    c = compact(dev, torch.from_numpy(m).to(dev), hkv)
    assert int(c.num_active[0]) == 64
    assert _ops.attend_plan(q, k, v, c.indices, c.num_active) == ("prefill_mfma", 16)
    out = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    again = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    assert torch.equal(out, again)
    rows = np.sort(rng.choice(sq, 24, replace=False))
    act = np.flatnonzero(m)
    ref = O.attention_active_blocks(np32(q[rows]), np32(k), np32(v), act)
    close(np32(out[rows]), ref, 5e-3)
    assert torch.isfinite(out).all()


def test_c4_prefill_layer_as_benched(dev):
    """C4 as bench.py times it: PrefillLayer (scoring -> bounds of all 512
    queries on the tiled kernel -> two-gate mask + compaction over the
    64-query tile maxima -> MFMA attention) on workloads.c4 at full size
    (131072 keys, 8 kv heads, d = 128, bf16), 75% evicted.  Tile maxima of
    sampled blocks against the float64 oracle; mask, permutation and count
    bit-exact against the oracle on the layer's own fp32 scores; sampled
    query rows against the float64 oracle over the retained blocks."""
    from orthocache_amd import _ops, workloads

    wl = workloads.c4(dev)
    sc = _ops.score(wl.k, wl.q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max.amax(dim=0), sc.zeta, 0.75)
    layer = _ops.PrefillLayer(wl.q, wl.k, wl.v, tau, zmax)
    out = layer.run()
    torch.cuda.synchronize()
    nb, hkv, d = 256, 8, 128
    parts = np32(layer.tau_max)
    assert parts.shape == (8, nb, hkv)
    z = np32(layer.zeta)
    mask = O.mask_from_scores(O.nanmax_axis0(parts), z, tau, zmax)
    order, n = O.stream_compact_indices(mask)
    assert n == int(layer.num_active[0]) == 64
    np.testing.assert_array_equal(np32(layer.indices).astype(np.int64), order)
    kk = wl.k.reshape(nb, 512, hkv, d)
    qn = np32(wl.q)
    for b in sorted({0, int(order[0]), int(order[n - 1]), int(order[n]), nb - 1}):
        kb = np32(kk[b])
        bounds = O.query_aware_bounds(qn, kb)[:, 0, :]          # (512 queries, hkv)
        np.testing.assert_allclose(parts[:, b, :], bounds.reshape(8, 64, hkv).max(axis=1), rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(z[b], O.spectral_decay_ratio(kb)[0], rtol=1e-5)
    rows = np.sort(np.random.default_rng(4).choice(512, 16, replace=False))
    sel = torch.from_numpy(order[:n].astype(np.int64)).to(dev)
    k_act = kk.index_select(0, sel).reshape(n * 512, hkv, d)
    v_act = wl.v.reshape(nb, 512, hkv, d).index_select(0, sel).reshape(n * 512, hkv, d)
    ref = O.attention_active_blocks(qn[rows], np32(k_act), np32(v_act), range(n))
    close(np32(out[rows]), ref, 1e-2)
    # a second run of the layer reproduces the first bit for bit
    again = layer.run().clone()
    torch.cuda.synchronize()
    assert torch.equal(again, out)
