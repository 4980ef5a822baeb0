"""GPU parity by property-based fuzzing: the two-gate mask and compaction.

Hypothesis draws score arrays and thresholds whose values come partly from a
pool of edge cases (NaN, +-inf, +-0, subnormals, values one ulp either side of
1, the largest finite floats) and partly from all fp32 values, so ties at a
threshold, NaN scores, NaN thresholds and empty or full masks all occur.  The
GPU's mask, active-first permutation and count (oc_mask_compact) must equal
the oracle's bit for bit: mask_from_scores over the NaN-propagating maximum of
the partial maxima (spectral_energy.py:180-234: jnp.max, then fp32 compares),
then stream_compact_indices (compaction.py:65-82).  One segment with 1-3
partial maxima per score, and ragged segments with per-segment thresholds;
and given masks with the per-head lists.  Also the many-query bound of bf16
queries over random shapes.  Deterministic (derandomize), no example
database.
"""

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st
from hypothesis.extra import numpy as hnp

from oracle import oc_oracle as O

pytestmark = pytest.mark.gpu

F32 = np.float32
POOL = [float(x) for x in (-np.inf, np.inf, np.nan, -0.0, 0.0, 1e-45, -1e-45, 1e-39, -1.5, 1.0,
                           np.nextafter(F32(1), F32(2)), np.nextafter(F32(1), F32(0)), 2.5, 7.0,
                           np.finfo(F32).max, -np.finfo(F32).max)]
ELEMS = st.one_of(st.sampled_from(POOL), st.floats(width=32, allow_nan=True, allow_infinity=True))
THRESH = st.one_of(st.sampled_from(POOL), st.floats(width=32, allow_nan=True, allow_infinity=True))
FUZZ = settings(derandomize=True, database=None, max_examples=60, deadline=None,
                suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])


def _dev():
    return torch.device("cuda:0")


@st.composite
def one_segment(draw):
    nb = draw(st.integers(1, 160))
    h = draw(st.integers(1, 8))
    parts = draw(st.integers(1, 3))
    tm = draw(hnp.arrays(F32, (parts, nb, h), elements=ELEMS))
    z = draw(hnp.arrays(F32, (nb, h), elements=ELEMS))
    return tm, z, draw(THRESH), draw(THRESH)


@given(one_segment())
@FUZZ
def test_fuzz_mask_compact(case):
    from orthocache_amd import _ops

    tm, z, tau, zmax = case
    parts, nb, h = tm.shape
    dev = _dev()
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=dev, tau_max=torch.from_numpy(tm).to(dev),
                          zeta=torch.from_numpy(z).to(dev), tau=tau, zeta_max=zmax, want_mask=True)
    torch.cuda.synchronize()
    exp = O.mask_from_scores(O.nanmax_axis0(tm), z, tau, zmax)
    order, n = O.stream_compact_indices(exp)
    np.testing.assert_array_equal(c.mask.cpu().numpy(), exp)
    np.testing.assert_array_equal(c.indices.cpu().numpy(), order)
    assert int(c.num_active[0]) == n


@st.composite
def segments(draw):
    lens = draw(st.lists(st.integers(1, 40), min_size=2, max_size=6))
    h = draw(st.integers(1, 4))
    nb = sum(lens)
    tm = draw(hnp.arrays(F32, (nb, h), elements=ELEMS))
    z = draw(hnp.arrays(F32, (nb, h), elements=ELEMS))
    taus = draw(hnp.arrays(F32, (len(lens),), elements=THRESH))
    zmaxs = draw(hnp.arrays(F32, (len(lens),), elements=THRESH))
    return lens, tm, z, taus, zmaxs


@given(segments())
@FUZZ
def test_fuzz_mask_compact_segments(case):
    from orthocache_amd import _ops

    lens, tm, z, taus, zmaxs = case
    nb, h = tm.shape
    dev = _dev()
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=dev, tau_max=torch.from_numpy(tm).to(dev),
                          zeta=torch.from_numpy(z).to(dev), tau=torch.from_numpy(taus).to(dev),
                          zeta_max=torch.from_numpy(zmaxs).to(dev), want_mask=True,
                          cu_blocks=torch.from_numpy(cu).to(dev), num_segments=len(lens))
    torch.cuda.synchronize()
    mask, idx, cnt = c.mask.cpu().numpy(), c.indices.cpu().numpy(), c.num_active.cpu().numpy()
    for s in range(len(lens)):
        lo, hi = cu[s], cu[s + 1]
        exp = O.mask_from_scores(tm[lo:hi], z[lo:hi], float(taus[s]), float(zmaxs[s]))
        order, n = O.stream_compact_indices(exp)
        np.testing.assert_array_equal(mask[lo:hi], exp)
        np.testing.assert_array_equal(idx[lo:hi], order)
        assert int(cnt[s]) == n


@st.composite
def given_masks(draw):
    nb = draw(st.integers(1, 600))
    h = draw(st.integers(1, 8))
    density = draw(st.sampled_from([0.0, 0.01, 0.1, 0.5, 1.0]))
    seed = draw(st.integers(0, 2**31 - 1))
    m = np.random.default_rng(seed).random((nb, h)) < density
    return m


@given(given_masks())
@FUZZ
def test_fuzz_given_mask_head_lists(m):
    """A given (block, head) mask: the unified active-first permutation and
    count (compaction.py:65-82) and every head's own list (the per-head
    compaction behind the predicated per-head attention, sparse_attention.py:5-64)."""
    from orthocache_amd import _ops

    nb, h = m.shape
    dev = _dev()
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=dev, mask_in=torch.from_numpy(m).to(dev),
                          want_head_lists=True)
    torch.cuda.synchronize()
    order, n = O.stream_compact_indices(m)
    np.testing.assert_array_equal(c.indices.cpu().numpy(), order)
    assert int(c.num_active[0]) == n
    hi, hn = c.head_indices.cpu().numpy(), c.head_num_active.cpu().numpy()
    for k in range(h):
        oh, nh = O.stream_compact_indices(m[:, k])
        np.testing.assert_array_equal(hi[k], oh)
        assert int(hn[0, k]) == nh


@st.composite
def bound_shapes(draw):
    d = draw(st.sampled_from([64, 128, 256]))
    hkv = draw(st.sampled_from([1, 2, 4]))
    group = draw(st.sampled_from([1, 2, 3, 4, 8]))
    sq = draw(st.integers(1, 96))
    nblk = draw(st.integers(1, 40))
    shift = draw(st.sampled_from([0.0, 0.5, -2.0]))
    seed = draw(st.integers(0, 2**31 - 1))
    return d, hkv, group, sq, nblk, shift, seed


@given(bound_shapes())
@settings(derandomize=True, database=None, max_examples=20, deadline=None,
          suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])
def test_fuzz_bf16_query_bounds(shape):
    """Many-query bounds of bf16 queries (the bf16 matrix-core kernel, k̄
    split into three bf16 terms) over random head dims, GQA groups, query
    counts and block counts: against the float64 oracle
    (spectral_energy.py:141-177) and against the fp32-MFMA kernel on the
    same values."""
    import orthocache_amd as oc

    d, hkv, group, sq, nblk, shift, seed = shape
    rng = np.random.default_rng(seed)
    dev = _dev()
    qd = torch.from_numpy(rng.standard_normal((sq, hkv * group, d)).astype(F32)).to(dev).to(torch.bfloat16)
    kd = torch.from_numpy((rng.standard_normal((nblk * 512, hkv, d)) + shift).astype(F32)).to(dev).to(torch.bfloat16)
    b = oc.compute_query_aware_bounds(qd, kd).float().cpu().numpy()
    b32 = oc.compute_query_aware_bounds(qd.float(), kd).float().cpu().numpy()
    np.testing.assert_allclose(b, b32, rtol=2e-6, atol=2e-6)
    q, keys = qd.float().cpu().numpy(), kd.float().cpu().numpy()
    np.testing.assert_allclose(b, O.query_aware_bounds(O.fold_gqa(q, hkv), keys), rtol=1e-5, atol=1e-5)
