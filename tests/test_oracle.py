"""Pin the CPU oracle (oracle/oc_oracle.py) before trusting it.

Checks come from outside the oracle's own formulas: the reference's
published golden values (Gate 6), closed forms (Hadamard matrix, Parseval,
bias-variance identity), brute force on tiny inputs, and the known answers
of the reference's own tests, regenerated from their seeds.  The last tests
plant typical mistakes in copies of oracle functions and confirm a check
fails for each.
"""

import numpy as np
import pytest
from scipy.linalg import hadamard

from oracle import oc_oracle as O

H512 = hadamard(512).astype(np.float64)


def gate6_blocks():
    """Gate-6 inputs, built exactly as the reference notebook (cell 10)."""
    n, nh, hd = 512, 4, 512
    rng = np.random.RandomState(123)
    a = np.zeros((n, nh, hd))
    for h in range(nh):
        for j in range(1, 16):
            c = rng.randn(hd)
            a[:, h, :] += np.outer(H512[:, j], c) / np.sqrt(n)
    var_a = np.sum(a ** 2)
    br = rng.randn(n, nh, hd)
    b = br * np.sqrt(var_a / np.sum(br ** 2))
    return a.astype(np.float32), b.astype(np.float32)


# Reference golden values: benchmarks/results/orthocache_v4_31b_results.json:1387-1394
GATE6_ZETA_A = 0.0
GATE6_ZETA_B_MEAN = 4.037281036376953
GATE6_AC_A = 7645.267578125
GATE6_AC_B = 7629.59033203125


class TestFWHT:
    def test_closed_form_hadamard(self):
        x = np.random.default_rng(0).standard_normal((512, 33))
        np.testing.assert_allclose(O.fwht_512(x), H512 @ x / np.sqrt(512), rtol=0, atol=1e-12)

    def test_reference_test_case(self):
        # tests/test_fwht.py:8-20: 512x128 from np.random.seed(42), rtol/atol 1e-5
        np.random.seed(42)
        a = np.random.randn(512, 128).astype(np.float32)
        np.testing.assert_allclose(O.fwht_512(a, dtype=np.float32), H512 @ a / np.sqrt(512), rtol=1e-5, atol=1e-5)

    def test_1d(self):
        x = np.random.default_rng(1).standard_normal(512)
        y = O.fwht_512(x)
        assert y.shape == (512,)
        np.testing.assert_allclose(y, H512 @ x / np.sqrt(512), atol=1e-12)

    def test_involution_and_parseval(self):
        x = np.random.default_rng(2).standard_normal((512, 8))
        y = O.fwht_512(x)
        np.testing.assert_allclose(O.fwht_512(y), x, atol=1e-12)
        np.testing.assert_allclose((y ** 2).sum(0), (x ** 2).sum(0), rtol=1e-12)

    def test_known_answers(self):
        const = np.ones(512)
        y = O.fwht_512(const)
        assert np.isclose(y[0], np.sqrt(512)) and np.allclose(y[1:], 0)
        alt = np.where(np.arange(512) % 2 == 0, 1.0, -1.0)
        y = O.fwht_512(alt)
        assert np.isclose(y[1], np.sqrt(512)) and np.allclose(np.delete(y, 1), 0)
        step = np.where(np.arange(512) < 256, 1.0, -1.0)
        y = O.fwht_512(step)
        assert np.isclose(y[256], np.sqrt(512)) and np.allclose(np.delete(y, 256), 0)

    def test_blocks_layout(self):
        rng = np.random.default_rng(3)
        k = rng.standard_normal((1024, 3, 5))
        spec = O.run_fwht_on_blocks(k)
        assert spec.shape == (2, 512, 3, 5)
        for b in range(2):
            for h in range(3):
                np.testing.assert_allclose(spec[b, :, h, :], H512 @ k[b * 512:(b + 1) * 512, h, :] / np.sqrt(512),
                                           atol=1e-12)


class TestBands:
    def test_gate6_golden_fp32(self):
        a, b = gate6_blocks()
        za = O.spectral_decay_ratio(a, dtype=np.float32)
        zb = O.spectral_decay_ratio(b, dtype=np.float32)
        assert np.all(za == GATE6_ZETA_A)
        # The fp32 restatement reproduces the published mean exactly.
        assert float(np.mean(zb)) == GATE6_ZETA_B_MEAN
        _, la, ma, ha = O.spectral_bands(a, dtype=np.float32)
        _, lb, mb, hb = O.spectral_bands(b, dtype=np.float32)
        assert float(np.mean(la + ma + ha)) == GATE6_AC_A
        np.testing.assert_allclose(float(np.mean(lb + mb + hb)), GATE6_AC_B, rtol=1e-6)

    def test_gate6_golden_fp64(self):
        a, b = gate6_blocks()
        np.testing.assert_allclose(np.mean(O.spectral_decay_ratio(b)), GATE6_ZETA_B_MEAN, rtol=1e-6)
        assert np.all(np.abs(O.spectral_decay_ratio(a)) < 1e-20)

    def test_brute_force_bands(self):
        rng = np.random.default_rng(4)
        k = rng.standard_normal((1024, 2, 7))
        dc, lo, mi, hi = O.spectral_bands(k)
        for b in range(2):
            for h in range(2):
                c = H512 @ k[b * 512:(b + 1) * 512, h, :] / np.sqrt(512)
                np.testing.assert_allclose(dc[b, h], c[0], atol=1e-12)
                np.testing.assert_allclose(lo[b, h], (c[1:64] ** 2).sum(), rtol=1e-12)
                np.testing.assert_allclose(mi[b, h], (c[64:256] ** 2).sum(), rtol=1e-12)
                np.testing.assert_allclose(hi[b, h], (c[256:] ** 2).sum(), rtol=1e-12)

    def test_walsh_coherent_block(self):
        # tests/test_spectral_bands.py:89-117
        rng = np.random.RandomState(42)
        blk = np.zeros((512, 64))
        for j in range(1, 16):
            w = np.ones(512)
            for i in range(512):
                for bit in range(9):
                    if (j >> bit) & 1 and (i >> bit) & 1:
                        w[i] *= -1
            blk += np.outer(w, rng.randn(64) * 0.5)
        z = O.spectral_decay_ratio(blk.reshape(512, 1, 64))
        assert z[0, 0] < 0.01

    def test_alternating_noise_block(self):
        # tests/test_spectral_bands.py:70-86 (its assertion: zeta > 1)
        np.random.seed(99)
        blk = np.zeros((512, 64))
        for i in range(512):
            blk[i] = (1.0 if i % 2 == 0 else -1.0) * np.random.randn(64) * 2.0
        assert O.spectral_decay_ratio(blk.reshape(512, 1, 64))[0, 0] > 1.0

    def test_white_noise_expectation(self):
        # E[zeta] -> 256/63 for white noise (high band 256 coefficients, low 63)
        k = np.random.default_rng(5).standard_normal((512 * 64, 1, 64))
        z = O.spectral_decay_ratio(k)
        assert abs(np.mean(z) - 256 / 63) < 0.05

    def test_block_energy_is_total_energy(self):
        k = np.random.default_rng(6).standard_normal((1024, 4, 64))
        dc, lo, mi, hi = O.spectral_bands(k)
        np.testing.assert_allclose(O.block_energy(k), (dc ** 2).sum(-1) + lo + mi + hi, rtol=1e-12)


class TestBounds:
    def test_closed_form(self):
        rng = np.random.default_rng(7)
        q = rng.standard_normal((8, 4, 64))
        k = rng.standard_normal((1024, 4, 64)) + 0.3
        b = O.query_aware_bounds(q, k)
        kb = k.reshape(2, 512, 4, 64)
        kbar = kb.mean(axis=1)
        eac = (kb ** 2).sum(axis=(1, 3)) - 512 * (kbar ** 2).sum(-1)
        exp = (np.einsum("qhd,bhd->qbh", q, kbar) + np.linalg.norm(q, axis=-1)[:, None, :] * np.sqrt(eac)[None]) / 8.0
        np.testing.assert_allclose(b, exp, rtol=1e-10)

    def test_cauchy_schwarz_invariant(self):
        rng = np.random.default_rng(8)
        q = rng.standard_normal((5, 2, 32))
        k = rng.standard_normal((1536, 2, 32))
        b = O.query_aware_bounds(q, k)
        logits = np.einsum("qhd,khd->qkh", q, k) / np.sqrt(32)
        mx = logits.reshape(5, 3, 512, 2).max(axis=2)
        assert np.all(b >= mx - 1e-9)

    def test_gqa_fold(self):
        rng = np.random.default_rng(9)
        q = rng.standard_normal((3, 8, 16))  # 8 q heads over 2 kv heads
        f = O.fold_gqa(q, 2)
        assert f.shape == (12, 2, 16)
        # query head h*G+g of token t lands on row t*G+g, kv head h
        np.testing.assert_array_equal(f[1 * 4 + 3, 1], q[1, 1 * 4 + 3])


class TestMasks:
    def test_threshold_mask_kat(self):
        # tests/test_energy.py:73-79
        m = O.threshold_mask(np.array([[10.5, 2.3], [1.1, 15.6]]), 5.0)
        np.testing.assert_array_equal(m, [[True, False], [False, True]])

    def test_two_gate_reference_case(self):
        # tests/test_spectral_bands.py:177-213 regenerated from its seed.  Block 0
        # is white noise times the alternating sign: in natural order that
        # multiplies by Walsh row 1, which only swaps coefficients s and s^1,
        # so its spectrum stays flat (zeta ~ 256/63 like block 1's plain
        # noise).  With tau = -100 and zeta_max = 1 both blocks fail gate 2:
        # the exact mask is all False, which the reference's `not all()` allows.
        np.random.seed(42)
        keys = np.random.randn(1024, 1, 64).astype(np.float32)
        for i in range(512):
            keys[i, 0, :] *= (1.0 if i % 2 == 0 else -1.0) * 5.0
        q = np.random.randn(1, 1, 64).astype(np.float32)
        m = O.multiband_mask(q, keys, -100.0, 1.0)
        np.testing.assert_array_equal(m, [[False], [False]])
        z = O.spectral_decay_ratio(keys)[:, 0]
        assert np.all((z > 2.5) & (z < 6.0)), z
        # The swap s <-> s^1 moves only coefficient 1 into DC and DC into the
        # low band; the high band of block 0 is the high band of the
        # unmodulated noise, coefficient by coefficient.
        raw = keys[:512, 0].astype(np.float64) * np.where(np.arange(512) % 2 == 0, 1.0, -1.0)[:, None]
        spec_raw = H512 @ raw / np.sqrt(512)
        spec_mod = H512 @ keys[:512, 0].astype(np.float64) / np.sqrt(512)
        np.testing.assert_allclose(spec_mod[256:], spec_raw[np.arange(256, 512) ^ 1], rtol=1e-9, atol=1e-9)

    def test_two_gate_separates_coherent_block(self):
        # The same case with block 1 replaced by the reference's Walsh-coherent
        # block (tests/test_spectral_bands.py:89-117: Walsh rows 1..15 with
        # RandomState(42) * 0.5 coefficients, zeta < 0.01): gate 2 now keeps
        # block 1 only, gate 1 at tau = -100 keeps both.
        np.random.seed(42)
        keys = np.random.randn(1024, 1, 64).astype(np.float32)
        for i in range(512):
            keys[i, 0, :] *= (1.0 if i % 2 == 0 else -1.0) * 5.0
        q = np.random.randn(1, 1, 64).astype(np.float32)
        rng = np.random.RandomState(42)
        coh = np.zeros((512, 64))
        for j in range(1, 16):
            coh += np.outer(H512[:, j], rng.randn(64) * 0.5)
        keys[512:, 0, :] = coh.astype(np.float32)
        np.testing.assert_array_equal(O.multiband_mask(q, keys, -100.0, 1.0), [[False], [True]])
        np.testing.assert_array_equal(O.query_aware_mask(q, keys, -100.0), [[True], [True]])
        # gate 1 alone at a tau above every bound keeps nothing
        np.testing.assert_array_equal(O.multiband_mask(q, keys, 1e6, 1.0), [[False], [False]])


def walsh_keys(blocks, d):
    """Keys whose spectra are known without a transform.

    Each block is (m, a, c): K[t, :] = m + a w_1[t] s + c w_256[t] r, with
    w_i the natural-order Walsh row i (Hadamard row i: w_1 alternates every
    token, w_256 changes sign once, at token 256), m a (d,) mean vector and
    s, r fixed +-1 vectors.  By orthogonality of the rows, per column the
    transform (scaled 1/sqrt(512)) has coefficient 0 = sqrt(512) m,
    coefficient 1 = sqrt(512) a s and coefficient 256 = sqrt(512) c r, so:
    E_low = 512 a^2 d, E_mid = 0, E_high = 512 c^2 d, E_AC = 512 (a^2 + c^2) d,
    kbar = m.
    """
    t = np.arange(512)
    w1 = np.where(t % 2 == 0, 1.0, -1.0)
    w256 = np.where(t < 256, 1.0, -1.0)
    s = np.where(np.arange(d) % 3 == 0, -1.0, 1.0)
    r = np.where(np.arange(d) % 2 == 0, 1.0, -1.0)
    out = []
    for m, a, c in blocks:
        out.append(np.asarray(m, np.float64)[None, :] + a * np.outer(w1, s) + c * np.outer(w256, r))
    return np.concatenate(out)[:, None, :]


class TestWalshMasks:
    """The mask entry points on keys whose scores follow from the construction.

    q = [2, 0, 0, 0] (||q|| = 2, sqrt(d) = 2).  Blocks (m, a, c):
      0: (0, 1, 0.5)         E_AC = 512*1.25*4 = 2560, tau = 0 + 2*sqrt(2560)/2 = 50.596, zeta = 0.25
      1: (0, 0.5, 1)         tau = 50.596, zeta = 4
      2: ([10,0,0,0], 1, .5) tau = 2*10/2 + 50.596 = 60.596, zeta = 0.25
      3: ([-10,0,0,0], 1,.5) tau = -10 + 50.596 = 40.596, zeta = 0.25
    """

    Q = np.array([[[2.0, 0.0, 0.0, 0.0]]])
    BLOCKS = [(np.zeros(4), 1.0, 0.5), (np.zeros(4), 0.5, 1.0), ([10.0, 0, 0, 0], 1.0, 0.5),
              ([-10.0, 0, 0, 0], 1.0, 0.5)]

    def test_scores_from_construction(self):
        k = walsh_keys(self.BLOCKS, 4)
        dc, lo, mi, hi = O.spectral_bands(k)
        np.testing.assert_allclose(lo[:, 0], [512 * 4, 128 * 4, 512 * 4, 512 * 4], rtol=1e-12)
        np.testing.assert_allclose(hi[:, 0], [128 * 4, 512 * 4, 128 * 4, 128 * 4], rtol=1e-12)
        np.testing.assert_allclose(mi, 0, atol=1e-9)
        # zeta = E_high / (E_low + 1e-6) (spectral_energy.py:138)
        z_co, z_hi = 512.0 / (2048.0 + 1e-6), 2048.0 / (512.0 + 1e-6)
        np.testing.assert_allclose(O.spectral_decay_ratio(k)[:, 0], [z_co, z_hi, z_co, z_co], rtol=1e-12)
        e = np.sqrt(2560.0)
        np.testing.assert_allclose(O.query_aware_bounds(self.Q, k)[0, :, 0], [e, e, 10 + e, -10 + e], rtol=1e-12)

    def test_query_aware_mask(self):
        k = walsh_keys(self.BLOCKS, 4)
        np.testing.assert_array_equal(O.query_aware_mask(self.Q, k, 55.0)[:, 0], [False, False, True, False])
        np.testing.assert_array_equal(O.query_aware_mask(self.Q, k, 45.0)[:, 0], [True, True, True, False])

    def test_multiband_mask(self):
        k = walsh_keys(self.BLOCKS, 4)
        np.testing.assert_array_equal(O.multiband_mask(self.Q, k, 45.0, 1.0)[:, 0], [True, False, True, False])
        np.testing.assert_array_equal(O.multiband_mask(self.Q, k, 45.0, 5.0)[:, 0], [True, True, True, False])
        np.testing.assert_array_equal(O.multiband_mask(self.Q, k, 30.0, 0.1)[:, 0], [False, False, False, False])
        # the max is over queries: a second query pointing the other way lifts block 3
        q2 = np.concatenate([self.Q, -self.Q], axis=0)
        np.testing.assert_array_equal(O.multiband_mask(q2, k, 55.0, 1.0)[:, 0], [False, False, True, True])

    def test_planted_sequency_order_flips_gate_two(self):
        # A sequency-ordered transform would put w_1 (511 sign changes) in the
        # high band and w_256 (one sign change) in the low band, inverting zeta.
        k = walsh_keys(self.BLOCKS, 4)
        nat = O.run_fwht_on_blocks(k)
        seq_idx = np.array([int(bin(i ^ (i >> 1))[2:].zfill(9)[::-1], 2) for i in range(512)])
        spec = np.empty_like(nat)
        spec[:, seq_idx] = nat  # natural index -> sequency index
        bad_zeta = (spec[:, 256:] ** 2).sum(axis=(1, 3)) / ((spec[:, 1:64] ** 2).sum(axis=(1, 3)) + 1e-6)
        bad = (O.query_aware_bounds(self.Q, k).max(0) >= 45.0) & (bad_zeta <= 1.0)
        assert list(bad[:, 0]) != [True, False, True, False]


class TestAutoTau:
    def test_known_answer(self):
        # mean 2.5, population variance 1.25 (ddof=0, jnp.std's default)
        assert O.auto_tau_from_max_bounds([[1.0, 2.0], [3.0, 4.0]]) == pytest.approx(2.5 - np.sqrt(1.25), rel=1e-15)
        assert O.auto_tau_from_max_bounds(np.full((3, 2), 7.0)) == 7.0

    def test_planted_sample_std_fails(self):
        bad = 2.5 - np.std([1.0, 2.0, 3.0, 4.0], ddof=1)
        assert bad != pytest.approx(O.auto_tau_from_max_bounds([1.0, 2.0, 3.0, 4.0]), rel=1e-6)

    def test_walsh_construction(self):
        # max bounds of TestWalshMasks: [e, e, 10 + e, -10 + e] with e = sqrt(2560):
        # mean e + 0, population std sqrt((0 + 0 + 100 + 100) / 4) = sqrt(50).
        k = walsh_keys(TestWalshMasks.BLOCKS, 4)
        assert O.auto_tau(TestWalshMasks.Q, k) == pytest.approx(np.sqrt(2560.0) - np.sqrt(50.0), rel=1e-12)
        # the max runs over queries before the statistics (pipeline.py:173)
        q2 = np.concatenate([TestWalshMasks.Q, -TestWalshMasks.Q], axis=0)
        e = np.sqrt(2560.0)
        mb = [e, e, 10 + e, 10 + e]
        assert O.auto_tau(q2, k) == pytest.approx(np.mean(mb) - np.sqrt(np.mean((np.array(mb) - np.mean(mb)) ** 2)),
                                                   rel=1e-12)

    def test_fp32_threshold_rounding_and_nan(self):
        tau = 0.1  # not representable: JAX compares against fp32(0.1)
        t32 = np.float32(tau)
        scores = np.array([[t32, np.nextafter(t32, np.float32(0))], [np.nan, np.inf]], dtype=np.float32)
        z = np.zeros_like(scores)
        m = O.mask_from_scores(scores, z, tau, 1.0)
        np.testing.assert_array_equal(m, [[True, False], [False, True]])
        m = O.mask_from_scores(np.ones((1, 2), np.float32), np.array([[np.nan, 1.0]], np.float32), 0.0, 1.0)
        np.testing.assert_array_equal(m, [[False, True]])

    def test_nanmax_propagates(self):
        x = np.array([[1.0, 2.0], [np.nan, 0.0]])
        r = O.nanmax_axis0(x)
        assert np.isnan(r[0]) and r[1] == 2.0


class TestCompaction:
    @pytest.mark.parametrize("mask,active", [
        ([False, True, False, True, True, False], [1, 3, 4]),   # tests/test_alltoallv.py:60-67
        ([True, False, True, True, False], [0, 2, 3]),          # tests/test_distributed.py:57-64
        ([True, False, True, False, True, False, False, True], [0, 2, 4, 7]),  # test_adaptive_attention.py:60-67
    ])
    def test_known_answers(self, mask, active):
        order, n = O.stream_compact_indices(np.array(mask))
        assert n == len(active)
        assert list(order[:n]) == active
        assert sorted(order) == list(range(len(mask)))
        assert list(order[n:]) == [i for i, m in enumerate(mask) if not m]

    def test_all_and_none(self):
        o, n = O.stream_compact_indices(np.ones(6, bool))
        assert n == 6 and list(o) == list(range(6))
        o, n = O.stream_compact_indices(np.zeros(6, bool))
        assert n == 0 and list(o) == list(range(6))

    def test_or_over_heads_and_brute_force(self):
        rng = np.random.default_rng(10)
        for nb in (1, 7, 64, 300):
            m = rng.random((nb, 3)) < 0.2
            o, n = O.stream_compact_indices(m)
            act = m.any(1)
            exp = [j for j in range(nb) if act[j]] + [j for j in range(nb) if not act[j]]
            assert list(o) == exp and n == act.sum()

    def test_exclusive_scan_kat(self):
        off, tot = O.exclusive_scan([3, 2, 5, 1])  # tests/test_alltoallv.py:76-81
        assert list(off) == [0, 3, 5, 10] and tot == 11

    def test_compact_decompact_roundtrip(self):
        rng = np.random.default_rng(11)
        k = rng.standard_normal((4 * 512, 2, 8))
        m = np.array([[True, False], [False, False], [False, True], [False, False]])
        ck, cv, order, n = O.stream_compact(k, k, m)
        assert n == 2 and np.all(ck[n:] == 0)
        back = O.stream_decompact(ck, order, n, 4)
        kb = k.reshape(4, 512, 2, 8)
        np.testing.assert_array_equal(back[[0, 2]], kb[[0, 2]])
        assert np.all(back[[1, 3]] == 0)


class TestAttention:
    def _data(self, nb=4, sq=2, hq=4, hkv=2, d=16, seed=12):
        rng = np.random.default_rng(seed)
        return (rng.standard_normal((sq, hq, d)), rng.standard_normal((nb * 512, hkv, d)),
                rng.standard_normal((nb * 512, hkv, d)))

    def test_all_blocks_equals_dense_softmax(self):
        q, k, v = self._data()
        out = O.attention_active_blocks(q, k, v, range(4))
        g = 2
        for h in range(4):
            lg = q[:, h] @ k[:, h // g].T / 4.0
            w = np.exp(lg - lg.max(1, keepdims=True))
            w /= w.sum(1, keepdims=True)
            np.testing.assert_allclose(out[:, h], w @ v[:, h // g], rtol=1e-12)

    def test_online_loop_matches_closed_form(self):
        q, k, v = self._data(nb=5, d=32)
        order, n = O.stream_compact_indices(np.array([True, False, True, True, False]))
        ref = O.attention_active_blocks(q, k, v, order[:n])
        loop = O.online_softmax_loop_fp32(q, k, v, order, n)
        np.testing.assert_allclose(loop, ref, rtol=2e-5, atol=2e-6)

    def test_empty_gives_zeros(self):
        q, k, v = self._data()
        assert np.all(O.attention_active_blocks(q, k, v, []) == 0)
        assert np.all(O.online_softmax_loop_fp32(q, k, v, np.arange(4), 0) == 0)

    def test_per_head_semantics(self):
        q, k, v = self._data(hq=2, hkv=2)
        m = np.array([[True, False], [False, False], [True, False], [False, False]])
        pred = O.attention_per_head_predicated(q, k, v, m)
        gated = O.attention_per_head_gated(q, k, v, m)
        np.testing.assert_allclose(pred[:, 0], O.attention_active_blocks(q[:, :1], k[:, :1], v[:, :1], [0, 2])[:, 0],
                                   rtol=1e-10)
        # head 1 keeps nothing: uniform weights -> mean of V; gated kernel -> zeros
        np.testing.assert_allclose(pred[:, 1], np.broadcast_to(v[:, 1].mean(0), pred[:, 1].shape), rtol=1e-10)
        assert np.all(gated[:, 1] == 0)


class TestBlockLogits:
    def _softmax_attend(self, lg, v, blocks, hkv, g):
        # lg: (nb, Hkv, 512, Sq*G) logits; softmax over the retained tokens, times V.
        d = v.shape[-1]
        nq = lg.shape[-1]
        sq = nq // g
        out = np.zeros((sq, hkv * g, d))
        tok = np.concatenate([np.arange(b * 512, (b + 1) * 512) for b in blocks])
        for h in range(hkv):
            l_h = np.concatenate([lg[b, h] for b in blocks], axis=0)  # (T, Sq*G)
            w = np.exp(l_h - l_h.max(0, keepdims=True))
            w /= w.sum(0, keepdims=True)
            o = w.T @ v[tok, h]                                        # (Sq*G, D)
            for i in range(nq):
                t, gg = divmod(i, g)
                out[t, h * g + gg] = o[i]
        return out

    def test_softmax_of_logits_reproduces_attention(self):
        rng = np.random.default_rng(21)
        q = rng.standard_normal((3, 4, 16))
        k = rng.standard_normal((4 * 512, 2, 16))
        v = rng.standard_normal((4 * 512, 2, 16))
        lg = O.block_logits(q, k)
        assert lg.shape == (4, 2, 512, 6)
        blocks = [0, 2, 3]
        np.testing.assert_allclose(self._softmax_attend(lg, v, blocks, 2, 2),
                                   O.attention_active_blocks(q, k, v, blocks), rtol=1e-10, atol=1e-12)

    def test_self_logit_known_answer(self):
        rng = np.random.default_rng(22)
        q = rng.standard_normal((1, 1, 64))
        k = rng.standard_normal((512, 1, 64))
        k[37, 0] = q[0, 0]
        lg = O.block_logits(q, k)
        assert np.isclose(lg[0, 0, 37, 0], (q[0, 0] ** 2).sum() / 8.0)

    def test_planted_gqa_fold_mistake_fails(self):
        # Query heads grouped the wrong way round (h + g*Hkv instead of h*G + g)
        # must not reproduce the attention.
        rng = np.random.default_rng(23)
        q = rng.standard_normal((1, 4, 8))
        k = rng.standard_normal((2 * 512, 2, 8))
        v = rng.standard_normal((2 * 512, 2, 8))
        bad_q = q[:, [0, 2, 1, 3]]
        lg_bad = O.block_logits(bad_q, k)
        assert not np.allclose(self._softmax_attend(lg_bad, v, [0, 1], 2, 2),
                               O.attention_active_blocks(q, k, v, [0, 1]))


class TestPlantedMistakes:
    """Each plants a plausible oracle mistake and checks that a pin above catches it."""

    def test_wrong_band_edge_fails_brute_force(self):
        k = np.random.default_rng(13).standard_normal((512, 1, 8))
        _, lo_bad, _, _ = O.spectral_bands(k, band_low=(0, 64))  # includes DC
        c = H512 @ k[:, 0, :] / np.sqrt(512)
        assert not np.isclose(lo_bad[0, 0], (c[1:64] ** 2).sum())

    def test_missing_scale_fails_closed_form(self):
        x = np.random.default_rng(14).standard_normal((512, 2))
        bad = O.fwht_512(x) * np.sqrt(512)  # dropped 1/sqrt(512)
        assert not np.allclose(bad, H512 @ x / np.sqrt(512))

    def test_sequency_order_fails_known_answer(self):
        # Reordering to sequency would move the alternating pattern to index 511.
        alt = np.where(np.arange(512) % 2 == 0, 1.0, -1.0)
        y = O.fwht_512(alt)
        assert abs(y[511]) < 1e-9 and abs(y[1]) > 1

    def test_unstable_partition_fails_kat(self):
        # A two-pointer (Hoare) partition puts the same blocks first but not in
        # order: the KAT of tests/test_alltoallv.py:60-67 must reject it.
        m = np.array([False, True, False, True, True, False])

        def hoare(mask):
            order = list(range(len(mask)))
            i, j = 0, len(mask) - 1
            while True:
                while i < j and mask[order[i]]:
                    i += 1
                while i < j and not mask[order[j]]:
                    j -= 1
                if i >= j:
                    return np.array(order), int(mask.sum())
                order[i], order[j] = order[j], order[i]

        def kat_ok(order, n):
            return n == 3 and list(order[:3]) == [1, 3, 4] and list(order[3:]) == [0, 2, 5]

        bad, nb = hoare(m)
        assert sorted(bad[:nb]) == [1, 3, 4]  # the right set ...
        assert not kat_ok(bad, nb)            # ... in the wrong order
        assert kat_ok(*O.stream_compact_indices(m))

    def test_wrong_sqrt_d_fails_closed_form(self):
        rng = np.random.default_rng(15)
        q = rng.standard_normal((2, 1, 16))
        k = rng.standard_normal((512, 1, 16))
        b = O.query_aware_bounds(q, k)
        kbar = k.mean(0)
        eac = (k ** 2).sum() - 512 * (kbar ** 2).sum()
        wrong = (q[:, 0] @ kbar[0] + np.linalg.norm(q[:, 0], axis=-1) * np.sqrt(eac)) / 16.0  # d, not sqrt(d)
        assert not np.allclose(b[:, 0, 0], wrong)
