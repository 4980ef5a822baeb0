"""GPU parity: indirect block-sparse attention vs the float64 oracle.

Tolerances: fp32 inputs 1e-4 (the reference's compacted-vs-predicated check
uses 1e-3, tests/test_compaction.py:178-184); bf16 inputs with bf16 output
1e-2 relative to the output scale.
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


def make(dev, nb, sq, hq, hkv, d, dtype, seed, block=512):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn(sq, hq, d, generator=g, device=dev).to(dtype)
    k = torch.randn(nb * block, hkv, d, generator=g, device=dev).to(dtype)
    v = torch.randn(nb * block, hkv, d, generator=g, device=dev).to(dtype)
    return q, k, v


class TestUnified:
    @pytest.mark.parametrize("sq,hq,hkv,d,dtype", [
        (1, 1, 1, 128, torch.bfloat16), (1, 32, 16, 256, torch.bfloat16), (1, 32, 8, 128, torch.bfloat16),
        (4, 4, 4, 64, torch.float32), (2, 8, 2, 256, torch.float32), (3, 6, 2, 128, torch.float16),
        (16, 2, 1, 64, torch.float32), (1, 1, 1, 512, torch.bfloat16), (1, 2, 1, 32, torch.float32),
        # 5-16 query rows per kv head (split form reading keys and values, groups of 8 rows)
        (1, 64, 8, 128, torch.bfloat16), (1, 48, 8, 128, torch.bfloat16), (5, 1, 1, 128, torch.float16),
        (2, 4, 1, 64, torch.bfloat16), (1, 16, 2, 256, torch.float32), (1, 128, 8, 128, torch.bfloat16),
        (1, 96, 8, 128, torch.bfloat16), (2, 8, 1, 64, torch.float16), (3, 4, 1, 128, torch.bfloat16)])
    def test_vs_oracle(self, dev, sq, hq, hkv, d, dtype):
        from orthocache_amd import _ops

        nb = 9
        q, k, v = make(dev, nb, sq, hq, hkv, d, dtype, seed=d + hq)
        mask = torch.tensor([1, 0, 1, 1, 0, 0, 1, 0, 1], dtype=torch.bool, device=dev)
        c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=mask)
        out = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
        ref = O.attention_active_blocks(np32(q), np32(k), np32(v), [0, 2, 3, 6, 8])
        close(np32(out), ref, 1e-4 if dtype == torch.float32 else 2e-3)

    def test_bf16_output_tolerance(self, dev):
        import orthocache_amd as oc

        q, k, v = make(dev, 8, 1, 4, 4, 128, torch.bfloat16, seed=3)
        mask = torch.tensor([1, 0, 0, 1, 1, 0, 1, 0], dtype=torch.bool, device=dev)
        out, stats = oc.orthocache_attention(q, k, v, mask)
        assert out.dtype == torch.bfloat16 and stats["num_active"] == 4
        ref = O.attention_active_blocks(np32(q), np32(k), np32(v), [0, 3, 4, 6])
        close(np32(out), ref, 1e-2)

    def test_empty_gives_zeros(self, dev):
        import orthocache_amd as oc

        q, k, v = make(dev, 4, 2, 2, 2, 64, torch.bfloat16, seed=4)
        out, stats = oc.orthocache_attention(q, k, v, torch.zeros(4, dtype=torch.bool, device=dev))
        assert float(out.float().abs().sum()) == 0.0
        assert stats == {"num_active": 0, "eviction_rate": 1.0, "path": "zero"}

    @pytest.mark.parametrize("block", [64, 100, 128, 256, 1024])
    def test_other_block_sizes(self, dev, block):
        from orthocache_amd import _ops

        nb = 6
        q, k, v = make(dev, nb, 2, 2, 1, 64, torch.float32, seed=block, block=block)
        mask = torch.tensor([0, 1, 1, 0, 0, 1], dtype=torch.bool, device=dev)
        c = _ops.mask_compact(num_blocks=nb, num_kv_heads=1, device=dev, mask_in=mask)
        out = _ops.attend(q, k, v, c.indices, c.num_active, block_size=block)
        ref = O.attention_active_blocks(np32(q), np32(k), np32(v), [1, 2, 5], block_size=block)
        close(np32(out), ref, 1e-4)

    def test_zero_eviction_matches_dense(self, dev):
        import orthocache_amd as oc
        from orthocache_amd.pipeline import _dense_attention

        q, k, v = make(dev, 4, 4, 4, 4, 64, torch.float32, seed=5)
        out, meta = oc.compact_and_attend(q, k, v, torch.ones(4, 4, dtype=torch.bool, device=dev))
        dense = _dense_attention(q, k, v, 64)
        assert float(meta["eviction_rate"]) == 0.0
        torch.testing.assert_close(out, dense, atol=1e-5, rtol=1e-5)
        ref = O.attention_active_blocks(np32(q), np32(k), np32(v), range(4))
        close(np32(dense), ref, 1e-4)

    def test_dense_non_block_multiple(self, dev):
        from orthocache_amd.pipeline import _dense_attention

        q = torch.randn(3, 2, 64, device=dev)
        k = torch.randn(700, 2, 64, device=dev)
        v = torch.randn(700, 2, 64, device=dev)
        out = _dense_attention(q, k, v, 64)
        ref = O.attention_active_blocks(np32(q), np32(k), np32(v), [0], block_size=700)
        close(np32(out), ref, 1e-4)


class TestPerHead:
    def test_predicated_and_gated(self, dev):
        import orthocache_amd as oc

        nb, h = 6, 3
        q, k, v = make(dev, nb, 4, h, h, 64, torch.float32, seed=6)
        m = np.zeros((nb, h), bool)
        m[[0, 4], 0] = True
        m[[1, 2, 3, 5], 1] = True  # head 2 keeps nothing
        mt = torch.from_numpy(m).to(dev)
        pred = oc.jax_block_sparse_attention(q, k, v, mt)
        gated = oc.compile_pallas_sparse_attention(q, k, v, mt)
        qn, kn, vn = np32(q), np32(k), np32(v)
        close(np32(pred), O.attention_per_head_predicated(qn, kn, vn, m), 1e-4)
        close(np32(gated), O.attention_per_head_gated(qn, kn, vn, m), 1e-4)
        assert float(gated[:, 2].abs().sum()) == 0.0

    def test_gqa_per_head(self, dev):
        import orthocache_amd as oc

        nb, hkv = 5, 2
        q, k, v = make(dev, nb, 2, 8, hkv, 128, torch.bfloat16, seed=7)
        m = np.array([[1, 0], [0, 1], [1, 1], [0, 0], [1, 0]], bool)
        out = oc.jax_block_sparse_attention(q, k, v, torch.from_numpy(m).to(dev))
        close(np32(out), O.attention_per_head_predicated(np32(q), np32(k), np32(v), m), 1e-2)

    def test_compact_matches_sparse(self, dev):
        # tests/test_compaction.py:162-184: compacted vs predicated at 1e-3
        import orthocache_amd as oc

        nb, h = 8, 4
        q, k, v = make(dev, nb, 4, h, h, 64, torch.float32, seed=8)
        m1 = torch.tensor([i % 2 == 0 for i in range(nb)], device=dev)
        mask = m1[:, None].expand(nb, h).contiguous()
        sparse = oc.jax_block_sparse_attention(q, k, v, mask)
        compact, meta = oc.compact_and_attend(q, k, v, mask)
        torch.testing.assert_close(compact, sparse, atol=1e-3, rtol=1e-3)
        assert int(meta["num_active"]) == 4 and int(meta["num_blocks"]) == 8
        assert abs(float(meta["eviction_rate"]) - 0.5) < 0.01


class TestBatched:
    def test_shared_mask_batch(self, dev):
        import orthocache_amd as oc

        b, nb, h, d = 3, 4, 2, 64
        g = torch.Generator(device=dev)
        g.manual_seed(9)
        q = torch.randn(b, 1, h, d, generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn(b, nb * 512, h, d, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(b, nb * 512, h, d, generator=g, device=dev).to(torch.bfloat16)
        mask = torch.tensor([1, 0, 1, 1], dtype=torch.bool, device=dev)
        out, stats = oc.orthocache_attention_batched(q, k, v, mask)
        assert out.shape == q.shape and stats["batch_size"] == 3 and stats["num_active"] == 3
        for i in range(b):
            ref = O.attention_active_blocks(np32(q[i]), np32(k[i]), np32(v[i]), [0, 2, 3])
            close(np32(out[i]), ref, 1e-2)

    def test_ragged_segments(self, dev):
        from orthocache_amd import _ops

        hkv, hq, d = 2, 4, 128
        seg_nb = [2, 5, 1, 3]
        cu = np.concatenate([[0], np.cumsum(seg_nb)]).astype(np.int32)
        nb = int(cu[-1])
        g = torch.Generator(device=dev)
        g.manual_seed(10)
        q = torch.randn(len(seg_nb), 1, hq, d, generator=g, device=dev)
        k = torch.randn(nb * 512, hkv, d, generator=g, device=dev)
        v = torch.randn(nb * 512, hkv, d, generator=g, device=dev)
        rng = np.random.default_rng(10)
        m = rng.random(nb) < 0.5
        m[cu[2]] = False  # segment 2 (one block) keeps nothing -> zeros
        cu_t = torch.from_numpy(cu).to(dev)
        c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=torch.from_numpy(m).to(dev),
                              cu_blocks=cu_t, num_segments=len(seg_nb))
        out = _ops.attend(q, k, v, c.indices, c.num_active, cu_blocks=cu_t, num_segments=len(seg_nb))
        for s in range(len(seg_nb)):
            lo, hi = cu[s], cu[s + 1]
            act = [j for j in range(hi - lo) if m[lo + j]]
            ref = O.attention_active_blocks(np32(q[s]), np32(k[lo * 512:hi * 512]), np32(v[lo * 512:hi * 512]), act)
            close(np32(out[s]), ref, 1e-4) if act else None
            if not act:
                assert float(out[s].abs().sum()) == 0.0
