"""GPU parity: the two-gate mask written by the scoring pass, and attention
that takes a block mask of one segment instead of a compacted list.

The scoring kernel's mask must equal, bit for bit, what the mask + compaction
kernel and the oracle derive from the same fp32 scores.  Attention from a
mask must give the same output bits as attention from the compaction's list
(same items in the same order), and write the same permutation and count.
"""

import numpy as np
import pytest
import torch

from oracle import oc_oracle as O

pytestmark = pytest.mark.gpu


def np32(t):
    return t.detach().float().cpu().numpy()


def make(dev, nb, sq, hq, hkv, d, dtype, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn(sq, hq, d, generator=g, device=dev).to(dtype)
    k = torch.randn(nb * 512, hkv, d, generator=g, device=dev).to(dtype)
    v = torch.randn(nb * 512, hkv, d, generator=g, device=dev).to(dtype)
    return q, k, v


@pytest.mark.parametrize("hkv,hq,d", [(16, 32, 256), (8, 32, 128), (3, 6, 64), (4, 4, 128), (1, 1, 128)])
def test_score_mask_matches_compaction(dev, hkv, hq, d):
    from orthocache_amd import _ops, workloads

    nb = 12
    k = workloads.make_keys(nb, hkv, d, seed=hkv + d, device=dev, noise_blocks=3)
    q = workloads.make_queries((1, hq, d), d, seed=7, device=dev)
    plain = _ops.score(k, q)
    tau, zmax = workloads.calibrate_unified(plain.tau_max[0], plain.zeta, evict=0.5)
    res = _ops.score(k, q, gate=(tau, zmax), want_logits=_ops.layer_uses_logits(k.dtype, d, hq // hkv, q.dtype))
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, tau_max=res.tau_max, zeta=res.zeta,
                          tau=tau, zeta_max=zmax, want_mask=True)
    torch.cuda.synchronize()
    assert torch.equal(res.mask, c.mask)
    ref = O.mask_from_scores(np32(res.tau_max[0]), np32(res.zeta), tau, zmax)
    np.testing.assert_array_equal(res.mask.cpu().numpy(), ref)


def test_score_mask_per_segment_thresholds(dev):
    from orthocache_amd import _ops

    hkv, d = 4, 128
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    k = torch.randn(6 * 512, hkv, d, generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn(2, 1, 8, d, generator=gen, device=dev).to(torch.bfloat16)
    cu = torch.tensor([0, 4, 6], dtype=torch.int32, device=dev)
    plain = _ops.score(k, q, cu_blocks=cu, num_segments=2)
    tm = plain.tau_max[0]
    tau = torch.stack([tm[:4].median(), tm[4:].median()]).float()
    zmax = torch.stack([plain.zeta[:4].max(), plain.zeta[4:].median()]).float()
    res = _ops.score(k, q, cu_blocks=cu, num_segments=2, gate=(tau, zmax))
    c = _ops.mask_compact(num_blocks=6, num_kv_heads=hkv, device=dev, tau_max=res.tau_max, zeta=res.zeta,
                          tau=tau, zeta_max=zmax, want_mask=True, cu_blocks=cu, num_segments=2)
    torch.cuda.synchronize()
    assert torch.equal(res.mask, c.mask)


MASKS = {
    "mixed": lambda nb, h, r: r.random((nb, h)) < 0.15,
    "none": lambda nb, h, r: np.zeros((nb, h), bool),
    "all": lambda nb, h, r: np.ones((nb, h), bool),
    "one_head": lambda nb, h, r: np.eye(nb, h, k=0, dtype=bool),
}


@pytest.mark.parametrize("nb,hkv,hq,d,dtype", [
    (128, 16, 32, 256, torch.bfloat16), (300, 4, 8, 128, torch.bfloat16), (1, 2, 2, 64, torch.float32),
    (9, 3, 3, 128, torch.float16), (40, 8, 32, 128, torch.bfloat16), (5, 32, 32, 64, torch.bfloat16)])
@pytest.mark.parametrize("kind", sorted(MASKS))
def test_attend_from_mask_equals_list(dev, nb, hkv, hq, d, dtype, kind):
    from orthocache_amd import _ops

    q, k, v = make(dev, nb, 1, hq, hkv, d, dtype, seed=nb + hkv)
    m_np = MASKS[kind](nb, hkv, np.random.default_rng(nb * hkv))
    mask = torch.from_numpy(m_np).to(dev)
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=mask)
    ref = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    idx = torch.full((nb,), -7, dtype=torch.int32, device=dev)
    cnt = torch.full((1,), -7, dtype=torch.int32, device=dev)
    out = _ops.attend(q, k, v, None, None, mask=mask, indices_out=idx, num_active_out=cnt, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(idx, c.indices) and torch.equal(cnt, c.num_active)
    assert torch.equal(out, ref)
    order, n = O.stream_compact_indices(m_np.any(axis=1))
    np.testing.assert_array_equal(idx.cpu().numpy(), order)
    assert int(cnt[0]) == n
    if n == 0:
        assert np.all(np32(out) == 0)


def test_attend_from_mask_with_logits(dev):
    from orthocache_amd import _ops

    nb, hkv, hq, d = 20, 8, 32, 128
    q, k, v = make(dev, nb, 1, hq, hkv, d, torch.bfloat16, seed=4)
    sc = _ops.score(k, q, want_logits=True)
    mask = torch.from_numpy(np.random.default_rng(2).random((nb, hkv)) < 0.1).to(dev)
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=mask)
    ref = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32, logits=sc.logits)
    out = _ops.attend(q, k, v, None, None, mask=mask, out_dtype=torch.float32, logits=sc.logits)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_mask_input_limits(dev):
    from orthocache_amd import _native, _ops

    q, k, v = make(dev, 4, 1, 4, 2, 64, torch.bfloat16, seed=1)
    with pytest.raises(_native.OrthoCacheError):
        # per-head lists cannot come from a mask input
        _ops.attend(q, k, v, None, None, mask=torch.ones(4, 2, dtype=torch.bool, device=dev), per_head=True)
    q2, k2, v2 = make(dev, 4, 64, 4, 2, 64, torch.bfloat16, seed=2)  # 128 rows per kv head: prefill shapes
    with pytest.raises(_native.OrthoCacheError):
        _ops.attend(q2, k2, v2, None, None, mask=torch.ones(4, 2, dtype=torch.bool, device=dev))


def test_layer_graph_replays_match_eager(dev):
    """The captured layer replayed several times, with eager work and host
    synchronisation in between and a new query each time, equals the eager
    layer bit for bit on every replay."""
    from orthocache_amd import _ops, workloads

    nb, hkv, hq, d = 24, 4, 8, 128
    k = workloads.make_keys(nb, hkv, d, seed=41, device=dev, noise_blocks=3)
    v = workloads.make_values(nb * 512, hkv, d, seed=42, device=dev)
    q = workloads.make_queries((1, hq, d), d, seed=43, device=dev)
    sc = _ops.score(k, q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, evict=0.75)
    layer = _ops.DecodeLayer(q, k, v, tau, zmax)
    g = layer.capture()
    for rep in range(4):
        layer.q.copy_(workloads.make_queries((1, hq, d), d, seed=50 + rep, device=dev))
        g.replay()
        torch.cuda.synchronize()
        got = (layer.out.clone(), layer.indices.clone(), layer.num_active.clone())
        _ops.score(k, layer.q)  # unrelated eager work between replays
        layer.run()
        torch.cuda.synchronize()
        assert torch.equal(got[0], layer.out), rep
        assert torch.equal(got[1], layer.indices) and torch.equal(got[2], layer.num_active), rep
