"""GPU parity: FWHT and block scores vs the CPU oracle and the reference's golden values."""

import numpy as np
import pytest
import torch
from scipy.linalg import hadamard

from oracle import oc_oracle as O

pytestmark = pytest.mark.gpu

H512 = hadamard(512).astype(np.float64) / np.sqrt(512)


def np32(t):
    return t.detach().float().cpu().numpy()


def to_dev(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(dtype)


# ------------------------------------------------------------------ FWHT
class TestFWHT:
    def test_reference_case(self, dev):
        import orthocache_amd as oc

        np.random.seed(42)  # tests/test_fwht.py:8-20
        a = np.random.randn(512, 128).astype(np.float32)
        y = np32(oc.fwht_512(to_dev(a, dev)))
        np.testing.assert_allclose(y, O.fwht_512(a), rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(y, H512 @ a, rtol=1e-5, atol=1e-5)

    def test_1d_and_odd_widths(self, dev):
        import orthocache_amd as oc

        rng = np.random.default_rng(0)
        for n in (1, 3, 31, 33, 100):
            a = rng.standard_normal((512, n)).astype(np.float32)
            np.testing.assert_allclose(np32(oc.fwht_512(to_dev(a, dev))), H512 @ a, rtol=1e-5, atol=1e-5)
        a = rng.standard_normal(512).astype(np.float32)
        y = oc.fwht_512(to_dev(a, dev))
        assert tuple(y.shape) == (512,)
        np.testing.assert_allclose(np32(y), H512 @ a, rtol=1e-5, atol=1e-5)

    def test_parseval_and_involution(self, dev):
        import orthocache_amd as oc

        a = torch.randn(512, 257, device=dev)
        y = oc.fwht_512(a)
        rel = (y.pow(2).sum() - a.pow(2).sum()).abs() / a.pow(2).sum()
        assert rel.item() <= 1e-5
        back = oc.fwht_512(y)
        assert ((back - a).norm() / a.norm()).item() <= 1e-5

    def test_bf16_input(self, dev):
        import orthocache_amd as oc

        a = torch.randn(512, 64, device=dev).to(torch.bfloat16)
        y = oc.fwht_512(a)
        assert y.dtype == torch.bfloat16
        ref = H512 @ np32(a)
        np.testing.assert_allclose(np32(y), ref, rtol=1e-2, atol=1e-2)

    def test_blocks_spectrum(self, dev):
        from orthocache_amd.spectral_energy import _run_fwht_on_blocks

        k = np.random.default_rng(1).standard_normal((1024, 3, 64)).astype(np.float32)
        spec = np32(_run_fwht_on_blocks(to_dev(k, dev)))
        np.testing.assert_allclose(spec, O.run_fwht_on_blocks(k), rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- scores
class TestBands:
    def test_reference_case_bands(self, dev):
        import orthocache_amd as oc

        np.random.seed(42)  # tests/test_spectral_bands.py:28-51
        keys = np.random.randn(1024, 2, 64).astype(np.float32)
        dc, lo, mi, hi = oc.compute_spectral_bands(to_dev(keys, dev))
        rdc, rlo, rmi, rhi = O.spectral_bands(keys)
        np.testing.assert_allclose(np32(dc), rdc, rtol=1e-5, atol=1e-5)
        for g, r in ((lo, rlo), (mi, rmi), (hi, rhi)):
            np.testing.assert_allclose(np32(g), r, rtol=1e-5)

    def test_reference_case_zeta(self, dev):
        import orthocache_amd as oc

        np.random.seed(123)  # tests/test_spectral_bands.py:54-67
        keys = np.random.randn(1024, 2, 64).astype(np.float32)
        z = oc.compute_spectral_decay_ratio(to_dev(keys, dev))
        np.testing.assert_allclose(np32(z), O.spectral_decay_ratio(keys), rtol=1e-5)

    @pytest.mark.parametrize("d,dtype", [(64, torch.float32), (128, torch.float32), (256, torch.float32),
                                          (512, torch.float32), (64, torch.bfloat16), (128, torch.bfloat16),
                                          (256, torch.bfloat16), (512, torch.bfloat16), (1024, torch.bfloat16),
                                          (128, torch.float16), (32, torch.float32)])
    @pytest.mark.parametrize("hkv", [3, 4])  # 4: heads with 128- or 256-byte rows are scored two per tile
    def test_all_layouts(self, dev, d, dtype, hkv):
        import orthocache_amd as oc

        rng = np.random.default_rng(d + hkv)
        keys = (rng.standard_normal((1536, hkv, d)) +
                rng.standard_normal((3, 1, hkv, d)).repeat(512, 0).reshape(1536, hkv, d)).astype(np.float32)
        kd = to_dev(keys, dev, dtype)
        kref = np32(kd)  # the values the GPU sees
        dc, lo, mi, hi = oc.compute_spectral_bands(kd)
        rdc, rlo, rmi, rhi = O.spectral_bands(kref)
        np.testing.assert_allclose(np32(dc), rdc, rtol=1e-5, atol=1e-4)
        for g, r in ((lo, rlo), (mi, rmi), (hi, rhi)):
            np.testing.assert_allclose(np32(g), r, rtol=1e-5)
        z = oc.compute_spectral_decay_ratio(kd)
        np.testing.assert_allclose(np32(z), O.spectral_decay_ratio(kref), rtol=1e-5)

    @pytest.mark.parametrize("d,dtype", [(128, torch.bfloat16), (64, torch.float32)])
    def test_head_major_storage(self, dev, d, dtype):
        """Keys stored head-major ((H, S, D) memory, viewed as (S, H, D)): the
        tile's second head is a head stride away rather than the next D
        elements.  Scores and bounds equal the contiguous layout's bit for bit
        (same values, same summation order)."""
        from orthocache_amd import _ops

        rng = np.random.default_rng(d)
        keys = to_dev(rng.standard_normal((2048, 4, d)) + 0.3, dev, dtype)
        q = to_dev(rng.standard_normal((1, 8, d)), dev, dtype)
        hm = keys.permute(1, 0, 2).contiguous().permute(1, 0, 2)
        assert hm.stride(1) == 2048 * d
        a, b = _ops.score(keys, q, want_bands=True), _ops.score(hm, q, want_bands=True)
        for name in ("tau_max", "zeta", "dc", "e_low", "e_mid", "e_high", "e_ac"):
            assert torch.equal(getattr(a, name), getattr(b, name)), name

    def test_gate6_golden(self, dev):
        import orthocache_amd as oc
        from tests.test_oracle import GATE6_AC_A, GATE6_AC_B, GATE6_ZETA_B_MEAN, gate6_blocks

        a, b = gate6_blocks()
        za = np32(oc.compute_spectral_decay_ratio(to_dev(a, dev)))
        zb = np32(oc.compute_spectral_decay_ratio(to_dev(b, dev)))
        assert np.all(za < 1e-9)
        np.testing.assert_allclose(np.mean(zb), GATE6_ZETA_B_MEAN, rtol=2e-6)
        _, la, ma, ha = oc.compute_spectral_bands(to_dev(a, dev))
        _, lb, mb, hb = oc.compute_spectral_bands(to_dev(b, dev))
        np.testing.assert_allclose(np.mean(np32(la + ma + ha)), GATE6_AC_A, rtol=2e-6)
        np.testing.assert_allclose(np.mean(np32(lb + mb + hb)), GATE6_AC_B, rtol=2e-6)

    def test_large_mean_low_band(self, dev):
        import orthocache_amd as oc

        rng = np.random.default_rng(3)
        keys = (rng.standard_normal((512, 1, 128)) * 0.05 + 40.0).astype(np.float32)
        _, lo, _, _ = oc.compute_spectral_bands(to_dev(keys, dev))
        _, rlo, _, _ = O.spectral_bands(keys)
        np.testing.assert_allclose(np32(lo), rlo, rtol=1e-4)

    def test_custom_bands(self, dev):
        import orthocache_amd as oc

        keys = np.random.default_rng(4).standard_normal((1024, 2, 64)).astype(np.float32)
        dc, lo, mi, hi = oc.compute_spectral_bands(to_dev(keys, dev), 512, (1, 32), (32, 300), (300, 512))
        rdc, rlo, rmi, rhi = O.spectral_bands(keys, 512, (1, 32), (32, 300), (300, 512))
        for g, r in ((lo, rlo), (mi, rmi), (hi, rhi)):
            np.testing.assert_allclose(np32(g), r, rtol=1e-5)
        z = oc.compute_spectral_decay_ratio(to_dev(keys, dev), 512, (1, 16), (400, 512))
        np.testing.assert_allclose(np32(z), O.spectral_decay_ratio(keys, 512, (1, 16), (400, 512)), rtol=1e-5)

    def test_block_energy(self, dev):
        import orthocache_amd as oc

        np.random.seed(42)  # tests/test_energy.py:16-52
        keys = np.random.randn(1024, 4, 64).astype(np.float32)
        e = oc.compute_block_energy_jax(to_dev(keys, dev), 512)
        np.testing.assert_allclose(np32(e), O.block_energy(keys), rtol=1e-5, atol=1e-5)
        e = oc.compute_block_energy_jax(to_dev(keys, dev), 128)
        np.testing.assert_allclose(np32(e), O.block_energy(keys, 128), rtol=1e-5, atol=1e-5)


class TestBounds:
    def test_reference_case(self, dev):
        import orthocache_amd as oc

        np.random.seed(42)  # tests/test_energy.py:55-72
        q = np.random.randn(8, 4, 64).astype(np.float32)
        keys = np.random.randn(1024, 4, 64).astype(np.float32)
        b = oc.compute_query_aware_bounds(to_dev(q, dev), to_dev(keys, dev))
        np.testing.assert_allclose(np32(b), O.query_aware_bounds(q, keys), rtol=1e-5, atol=1e-5)

    @pytest.mark.parametrize("sq,hq,hkv,d", [(1, 1, 1, 128), (1, 32, 16, 256), (3, 8, 2, 64), (40, 2, 2, 128),
                                               (100, 4, 1, 64)])
    def test_gqa_and_many_queries(self, dev, sq, hq, hkv, d):
        import orthocache_amd as oc

        rng = np.random.default_rng(sq * 7 + hq)
        q = rng.standard_normal((sq, hq, d)).astype(np.float32)
        keys = (rng.standard_normal((1024, hkv, d)) + 0.5).astype(np.float32)
        b = np32(oc.compute_query_aware_bounds(to_dev(q, dev), to_dev(keys, dev)))
        ref = O.query_aware_bounds(O.fold_gqa(q, hkv), keys)
        np.testing.assert_allclose(b, ref, rtol=1e-5, atol=1e-5)

    @pytest.mark.parametrize("sq,hq,hkv,d,nblk", [(100, 4, 2, 128, 70), (37, 8, 1, 64, 3), (65, 2, 2, 256, 5),
                                                    (512, 4, 1, 128, 130), (17, 4, 4, 128, 1)])
    def test_bf16_queries_many_rows(self, dev, sq, hq, hkv, d, nblk):
        """Many bf16 query rows take the bf16 matrix-core bound (kbar split
        into three bf16 terms): full bounds and per-64-row tile maxima against
        the float64 oracle, and against the fp32 kernel on the same values.
        Ragged query tiles (odd tile counts leave a workgroup's second tile
        empty) and block counts that are not multiples of 64."""
        import orthocache_amd as oc
        from orthocache_amd import _ops

        rng = np.random.default_rng(sq * 31 + nblk)
        qd = to_dev(rng.standard_normal((sq, hq, d)).astype(np.float32), dev, torch.bfloat16)
        kd = to_dev((rng.standard_normal((nblk * 512, hkv, d)) + 0.25).astype(np.float32), dev, torch.bfloat16)
        q, keys = np32(qd), np32(kd)  # the values the GPU sees
        ref = O.query_aware_bounds(O.fold_gqa(q, hkv), keys)
        b = np32(oc.compute_query_aware_bounds(qd, kd))
        np.testing.assert_allclose(b, ref, rtol=1e-5, atol=1e-5)
        b32 = np32(oc.compute_query_aware_bounds(qd.float(), kd))
        np.testing.assert_allclose(b, b32, rtol=2e-6, atol=2e-6)
        parts = np32(_ops.score(kd, qd).tau_max)
        nq = ref.shape[0]
        nt = (nq + 63) // 64
        pad = np.full((nt * 64 - nq,) + ref.shape[1:], -np.inf)
        ref_parts = np.concatenate([ref, pad]).reshape(nt, 64, *ref.shape[1:]).max(axis=1)
        assert parts.shape == ref_parts.shape
        np.testing.assert_allclose(parts, ref_parts, rtol=1e-5, atol=1e-5)

    def test_bf16_queries_nonfinite_keys(self, dev):
        """Infinite and NaN keys: the bf16 split kernel's bounds equal the
        fp32 kernel's (NaN where it gives NaN, the same infinities)."""
        import orthocache_amd as oc

        rng = np.random.default_rng(11)
        k = rng.standard_normal((6 * 512, 2, 128)).astype(np.float32)
        k[3, 0, 5] = np.inf
        k[512 + 7, 1, 100] = -np.inf
        k[2 * 512, 0, 0] = np.nan
        k[4 * 512 + 1, 1, 64:] = 3e38
        qd = to_dev(rng.standard_normal((70, 4, 128)).astype(np.float32), dev, torch.bfloat16)
        kd = to_dev(k, dev, torch.bfloat16)
        b = np32(oc.compute_query_aware_bounds(qd, kd))
        b32 = np32(oc.compute_query_aware_bounds(qd.float(), kd))
        assert np.array_equal(np.isnan(b), np.isnan(b32))
        assert np.array_equal(np.isinf(b), np.isinf(b32))
        np.testing.assert_allclose(b, b32, rtol=2e-6, atol=2e-6)

    @pytest.mark.parametrize("sq,hq,hkv", [(1, 32, 16), (2, 8, 2), (64, 4, 4), (1, 32, 8), (3, 9, 3)])
    @pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
    def test_tau_max_inline_and_tiled(self, dev, sq, hq, hkv, dtype):
        from orthocache_amd import _ops

        d = 128
        rng = np.random.default_rng(sq + hq)
        q = rng.standard_normal((sq, hq, d)).astype(np.float32)
        keys = rng.standard_normal((2048, hkv, d)).astype(np.float32)
        kd, qd = to_dev(keys, dev, dtype), to_dev(q, dev, dtype)
        keys, q = np32(kd), np32(qd)  # the values the GPU sees
        sc = _ops.score(kd, qd)
        tm = np32(sc.tau_max).max(axis=0)
        ref = O.nanmax_axis0(O.query_aware_bounds(O.fold_gqa(q, hkv), keys))
        np.testing.assert_allclose(tm, ref, rtol=1e-5, atol=1e-5)
