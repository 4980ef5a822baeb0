"""GPU parity: two-gate masks and stream compaction, bit-exact vs the oracle."""

import numpy as np
import pytest
import torch

from oracle import oc_oracle as O

pytestmark = pytest.mark.gpu


def np32(t):
    return t.detach().cpu().numpy()


def dev_f32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def run_mask(dev, tau_max, zeta, tau, zmax, **kw):
    from orthocache_amd import _ops

    nb, h = tau_max.shape[-2:]
    tm = dev_f32(tau_max, dev)
    if tm.dim() == 2:
        tm = tm.unsqueeze(0)
    return _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=dev, tau_max=tm,
                             zeta=None if zeta is None else dev_f32(zeta, dev), tau=tau, zeta_max=zmax,
                             want_mask=True, want_active=True, **kw)


class TestMask:
    @pytest.mark.parametrize("nb,h", [(1, 1), (16, 1), (128, 16), (257, 8), (1000, 3), (4096, 2)])
    def test_bit_exact_on_identical_scores(self, dev, nb, h):
        rng = np.random.default_rng(nb * 31 + h)
        tm = rng.standard_normal((nb, h)).astype(np.float32)
        z = rng.exponential(2.0, (nb, h)).astype(np.float32)
        tau = float(np.percentile(tm, 60))
        zmax = float(np.percentile(z, 80))
        c = run_mask(dev, tm, z, tau, zmax)
        exp = O.mask_from_scores(tm, z, tau, zmax)
        np.testing.assert_array_equal(np32(c.mask), exp)
        np.testing.assert_array_equal(np32(c.active), exp.any(axis=1))
        order, n = O.stream_compact_indices(exp)
        np.testing.assert_array_equal(np32(c.indices), order)
        assert int(c.num_active[0]) == n

    def test_special_values(self, dev):
        t32 = np.float32(0.1)
        below = np.nextafter(t32, np.float32(-1))
        tm = np.array([[t32], [below], [np.nan], [np.inf], [-np.inf], [t32]], dtype=np.float32)
        z = np.array([[0.0], [0.0], [0.0], [0.0], [0.0], [np.nan]], dtype=np.float32)
        c = run_mask(dev, tm, z, 0.1, 1.0)
        np.testing.assert_array_equal(np32(c.mask)[:, 0], [True, False, False, True, False, False])
        # tie on zeta_max keeps, NaN threshold keeps nothing
        c = run_mask(dev, np.ones((2, 1), np.float32), np.array([[2.5], [2.5000002]], np.float32), 0.0, 2.5)
        np.testing.assert_array_equal(np32(c.mask)[:, 0], [True, False])
        c = run_mask(dev, np.ones((3, 1), np.float32), np.zeros((3, 1), np.float32), float("nan"), 1.0)
        assert not np32(c.mask).any() and int(c.num_active[0]) == 0

    def test_partial_maxima_propagate_nan(self, dev):
        parts = np.array([[[1.0]], [[np.nan]], [[0.0]]], dtype=np.float32)  # (P=3, nb=1, h=1)
        c = run_mask(dev, parts, None, 0.5, 0.0)
        assert not np32(c.mask)[0, 0]
        parts = np.array([[[0.1]], [[0.7]]], dtype=np.float32)
        c = run_mask(dev, parts, None, 0.5, 0.0)
        assert np32(c.mask)[0, 0]

    def test_gate_two_off(self, dev):
        tm = np.array([[1.0], [0.0]], np.float32)
        c = run_mask(dev, tm, None, 0.5, None)
        np.testing.assert_array_equal(np32(c.mask)[:, 0], [True, False])


class TestCompaction:
    @pytest.mark.parametrize("mask,active", [
        ([False, True, False, True, True, False], [1, 3, 4]),
        ([True, False, True, True, False], [0, 2, 3]),
        ([True, False, True, False, True, False, False, True], [0, 2, 4, 7]),
    ])
    def test_reference_kats(self, dev, mask, active):
        from orthocache_amd import adaptive_attention

        idx, n = adaptive_attention.stream_compact(torch.tensor(mask, device=dev))
        order, n_ref = O.stream_compact_indices(np.array(mask))
        assert n == n_ref == len(active)
        np.testing.assert_array_equal(np32(idx), order)

    @pytest.mark.parametrize("nb", [1, 2, 63, 64, 65, 255, 256, 257, 1023, 5000])
    @pytest.mark.parametrize("p", [0.0, 0.1, 0.5, 1.0])
    def test_random_masks(self, dev, nb, p):
        from orthocache_amd import _ops

        rng = np.random.default_rng(nb + int(p * 100))
        m = rng.random((nb, 4)) < p / 4
        c = _ops.mask_compact(num_blocks=nb, num_kv_heads=4, device=dev,
                              mask_in=torch.from_numpy(m).to(dev), want_head_lists=True)
        order, n = O.stream_compact_indices(m)
        np.testing.assert_array_equal(np32(c.indices), order)
        assert int(c.num_active[0]) == n
        for h in range(4):
            oh, nh = O.stream_compact_indices(m[:, h])
            np.testing.assert_array_equal(np32(c.head_indices[h]), oh)
            assert int(c.head_num_active[0, h]) == nh

    def test_empty_head_policy(self, dev):
        from orthocache_amd import _ops

        m = np.zeros((5, 2), bool)
        m[[1, 3], 0] = True
        c = _ops.mask_compact(num_blocks=5, num_kv_heads=2, device=dev, mask_in=torch.from_numpy(m).to(dev),
                              want_indices=False, want_head_lists=True, empty_head_all=True)
        np.testing.assert_array_equal(np32(c.head_num_active)[0], [2, 5])
        np.testing.assert_array_equal(np32(c.head_uniform)[0], [0, 1])
        np.testing.assert_array_equal(np32(c.head_indices)[1], np.arange(5))

    def test_segments(self, dev):
        from orthocache_amd import _ops

        rng = np.random.default_rng(7)
        seg_nb = [3, 1, 300, 17, 64]
        cu = np.concatenate([[0], np.cumsum(seg_nb)]).astype(np.int32)
        nb = int(cu[-1])
        tm = rng.standard_normal((nb, 2)).astype(np.float32)
        z = rng.random((nb, 2)).astype(np.float32)
        taus = np.array([0.0, 10.0, 0.5, -0.5, 1.0], np.float32)
        zmaxs = np.array([0.5, 0.9, 0.8, 1.0, 0.3], np.float32)
        c = _ops.mask_compact(num_blocks=nb, num_kv_heads=2, device=dev, tau_max=dev_f32(tm, dev).unsqueeze(0),
                              zeta=dev_f32(z, dev), tau=dev_f32(taus, dev), zeta_max=dev_f32(zmaxs, dev),
                              want_mask=True, cu_blocks=torch.from_numpy(cu).to(dev), num_segments=len(seg_nb))
        idx = np32(c.indices)
        for s in range(len(seg_nb)):
            lo, hi = cu[s], cu[s + 1]
            exp = O.mask_from_scores(tm[lo:hi], z[lo:hi], float(taus[s]), float(zmaxs[s]))
            np.testing.assert_array_equal(np32(c.mask)[lo:hi], exp)
            order, n = O.stream_compact_indices(exp)
            np.testing.assert_array_equal(idx[lo:hi], order)
            assert int(c.num_active[s]) == n


class TestMaterialised:
    def test_stream_compact_and_decompact(self, dev):
        import orthocache_amd as oc

        nb, h, d = 8, 4, 64
        k = torch.randn(nb * 512, h, d, device=dev)
        v = torch.randn(nb * 512, h, d, device=dev)
        m1 = torch.tensor([i % 2 == 0 for i in range(nb)], device=dev)
        mask = m1[:, None].expand(nb, h)
        ck, cv, idx, n = oc.stream_compact(k, v, mask)
        assert int(n) == 4 and ck.shape == (nb, 512, h, d)
        kb = k.reshape(nb, 512, h, d)
        for i in range(4):
            assert torch.equal(ck[i], kb[int(idx[i])])
        assert float(ck[4:].abs().sum()) == 0.0
        back = oc.stream_decompact(ck, idx, n, nb)
        keep = m1.cpu().numpy()
        for b in range(nb):
            if keep[b]:
                assert torch.equal(back[b], kb[b])
            else:
                assert float(back[b].abs().sum()) == 0.0

    def test_full_and_zero_eviction(self, dev):
        import orthocache_amd as oc

        k = torch.randn(4 * 512, 2, 32, device=dev)
        ck, _, _, n = oc.stream_compact(k, k, torch.zeros(4, 2, dtype=torch.bool, device=dev))
        assert int(n) == 0 and float(ck.abs().sum()) == 0.0
        _, _, idx, n = oc.stream_compact(k, k, torch.ones(4, 2, dtype=torch.bool, device=dev))
        assert int(n) == 4 and np32(idx).tolist() == [0, 1, 2, 3]
        _, _, _, n = oc.stream_compact(k[:512], k[:512], torch.ones(1, 2, dtype=torch.bool, device=dev))
        assert int(n) == 1

    @pytest.mark.parametrize("idx,n", [
        ([3, 1, 3, 0, 5, 2], 4),         # block 3 named twice: the later position (2) wins
        ([7, -1, 9, 2, -6, 0], 6),       # out of range (7, 9, -7..) dropped; -1 -> 5, -6 -> 0
        ([1, 1, 1, 1, 1, 1], 6),         # every position names block 1: position 5 wins
        ([4, 0, 2, 1, 3, 5], 9),         # num_active beyond the block count is clamped to 6
        ([4, 0, 2, 1, 3, 5], -2),        # and below zero to 0: all zeros
    ])
    def test_decompact_arbitrary_lists(self, dev, idx, n):
        """stream_decompact on lists that are not stream_compact's permutation:
        every destination block is written once, out-of-range entries are
        dropped, repeated entries take the last position (the oracle's
        in-order scatter); the gather clamps its entries."""
        import orthocache_amd as oc
        from orthocache_amd import _ops

        nb, h, d = 6, 2, 32
        src = torch.randn(nb, 512, h, d, device=dev)
        ind = torch.tensor(idx, dtype=torch.int32, device=dev)
        out = oc.stream_decompact(src, ind, n, nb)
        torch.cuda.synchronize()
        ref = O.stream_decompact(np32(src), np.array(idx), n, nb)
        np.testing.assert_array_equal(np32(out), ref)
        # gather form: dst[i] = src[clamp(wrap(idx[i]))] for i < n
        dst = torch.empty_like(src)
        na = torch.tensor([n], dtype=torch.int32, device=dev)
        _ops.copy_blocks(src.reshape(nb, -1), dst, ind, na, nb, scatter=False)
        torch.cuda.synchronize()
        nn = max(0, min(n, nb))
        s = np32(src)
        for i in range(nb):
            if i < nn:
                j = idx[i] + nb if -nb <= idx[i] < 0 else idx[i]
                np.testing.assert_array_equal(np32(dst[i]), s[min(max(j, 0), nb - 1)])
            else:
                assert float(dst[i].abs().sum()) == 0.0
