"""Pin the oracle's attention against the reference's own C++ attention, and
check the C port (the CPU baseline) against the NumPy oracle."""

import numpy as np
import pytest

from oracle import oc_oracle as O
from oracle import native as ON


@pytest.fixture(scope="module")
def port():
    try:
        return ON.port()
    except RuntimeError as e:
        pytest.fail(str(e))


@pytest.mark.skipif(not ON.ref_available(), reason="oracle/_ref not built (reference tree absent)")
class TestAgainstReferenceCpp:
    @pytest.mark.parametrize("seed,mask", [(0, [1, 0, 1, 1]), (1, [0, 0, 0, 1]), (2, [1, 1, 1, 1]),
                                           (3, [0, 1, 0, 1, 0, 1, 1, 0])])
    def test_single_head_matches(self, seed, mask):
        rng = np.random.default_rng(seed)
        nb, sq, d = len(mask), 3, 64
        q = rng.standard_normal((sq, d)).astype(np.float32)
        k = rng.standard_normal((nb * 512, d)).astype(np.float32)
        v = rng.standard_normal((nb * 512, d)).astype(np.float32)
        ref = ON.ref_compacted_attention(q, k, v, np.array(mask))
        act = [i for i, m in enumerate(mask) if m]
        ours = O.attention_active_blocks(q[:, None, :], k[:, None, :], v[:, None, :], act)[:, 0]
        np.testing.assert_allclose(ours, ref, rtol=1e-4, atol=1e-5)

    def test_all_evicted_gives_zeros(self):
        rng = np.random.default_rng(4)
        q = rng.standard_normal((2, 32)).astype(np.float32)
        k = rng.standard_normal((1024, 32)).astype(np.float32)
        ref = ON.ref_compacted_attention(q, k, k, np.zeros(2, np.int32))
        assert np.all(ref == 0)
        assert np.all(O.attention_active_blocks(q[:, None], k[:, None], k[:, None], [])[:, 0] == 0)


class TestPort:
    def test_scores_match_oracle(self, port):
        rng = np.random.default_rng(5)
        k = (rng.standard_normal((1536, 3, 64)) + 0.5).astype(np.float32)
        kb = O.to_bf16_bits(k).reshape(k.shape)
        kf = O.bf16_bits_to_f32(kb).reshape(k.shape)
        q = rng.standard_normal((1, 6, 64)).astype(np.float32)
        qf = O.fold_gqa(q, 3)
        tm, z = ON.port_score(kb, qf)
        np.testing.assert_allclose(z, O.spectral_decay_ratio(kf), rtol=2e-5)
        np.testing.assert_allclose(tm, O.query_aware_bounds(qf, kf).max(axis=0), rtol=2e-5, atol=2e-5)

    def test_compact_matches_oracle(self, port):
        rng = np.random.default_rng(6)
        tm = rng.standard_normal((300, 4)).astype(np.float32)
        z = rng.random((300, 4)).astype(np.float32)
        mask, idx, n = ON.port_compact(tm, z, 0.7, 0.5)
        exp = O.mask_from_scores(tm, z, 0.7, 0.5)
        np.testing.assert_array_equal(mask, exp)
        order, n_ref = O.stream_compact_indices(exp)
        np.testing.assert_array_equal(idx, order)
        assert n == n_ref

    def test_compact_fuzz_matches_oracle(self, port):
        """Property-based: NaN, +-inf, +-0, subnormal and tied scores and
        thresholds; the port's mask, permutation and count equal the NumPy
        oracle's bit for bit."""
        from hypothesis import HealthCheck, given, settings
        from hypothesis import strategies as st
        from hypothesis.extra import numpy as hnp

        pool = [float(x) for x in (-np.inf, np.inf, np.nan, -0.0, 0.0, 1e-45, -1e-45, 1.0,
                                   np.nextafter(np.float32(1), np.float32(2)), 2.5)]
        elems = st.one_of(st.sampled_from(pool), st.floats(width=32, allow_nan=True, allow_infinity=True))

        @st.composite
        def case(draw):
            nb, h = draw(st.integers(1, 120)), draw(st.integers(1, 6))
            return (draw(hnp.arrays(np.float32, (nb, h), elements=elems)),
                    draw(hnp.arrays(np.float32, (nb, h), elements=elems)), draw(elems), draw(elems))

        @given(case())
        @settings(derandomize=True, database=None, max_examples=80, deadline=None,
                  suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])
        def check(c):
            tm, z, tau, zmax = c
            mask, idx, n = ON.port_compact(tm, z, tau, zmax)
            exp = O.mask_from_scores(tm, z, tau, zmax)
            np.testing.assert_array_equal(mask, exp)
            order, n_ref = O.stream_compact_indices(exp)
            np.testing.assert_array_equal(idx, order)
            assert n == n_ref

        check()

    def test_attend_matches_oracle(self, port):
        rng = np.random.default_rng(7)
        q = rng.standard_normal((2, 4, 64)).astype(np.float32)
        k = O.to_bf16_bits(rng.standard_normal((2048, 2, 64))).reshape(2048, 2, 64)
        v = O.to_bf16_bits(rng.standard_normal((2048, 2, 64))).reshape(2048, 2, 64)
        idx = np.array([1, 3, 0, 2], np.int32)
        out = ON.port_attend(q, k, v, idx, 2)
        ref = O.attention_active_blocks(q, O.bf16_bits_to_f32(k).reshape(k.shape),
                                        O.bf16_bits_to_f32(v).reshape(v.shape), [1, 3])
        np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)
        assert np.all(ON.port_attend(q, k, v, idx, 0) == 0)
