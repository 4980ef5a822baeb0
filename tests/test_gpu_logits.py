"""GPU parity: attention logits formed in the scoring pass.

The scoring kernel can write q.k * log2(e)/sqrt(d) for every key row while it
streams the keys (at most 4 query rows per kv head); the decode attention then
reads those logits and the values instead of keys and values.  Checked here:
the logits against the float64 oracle (``block_logits``), the scores of the
same launch bit for bit against a launch without logits, and the attention
from logits against the oracle and against the key-reading attention.
Tolerances: logits 1e-5 of the largest |logit|; attention as in
test_gpu_attention.py (1e-4 fp32 inputs, 2e-3 bf16/fp16 inputs, fp32 out).
"""

import math

import numpy as np
import pytest
import torch

from oracle import oc_oracle as O

pytestmark = pytest.mark.gpu

LOG2E = 1.0 / math.log(2.0)


def np32(t):
    return t.detach().float().cpu().numpy()


def close(out, ref, rel):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), 1e-6)
    err = np.abs(out - ref).max() / scale
    assert err <= rel, f"max error {err:.3e} relative to scale (tolerance {rel})"


def make(dev, nb, sq, hq, hkv, d, dtype, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    q = torch.randn(sq, hq, d, generator=g, device=dev).to(dtype)
    k = (torch.randn(nb * 512, hkv, d, generator=g, device=dev) + 0.5).to(dtype)
    v = torch.randn(nb * 512, hkv, d, generator=g, device=dev).to(dtype)
    return q, k, v


CASES = [
    # (sq, hq, hkv, d, dtype): nq = sq * hq / hkv query rows per kv head
    (1, 32, 16, 256, torch.bfloat16),   # C2 shape (nq 2)
    (1, 32, 8, 128, torch.bfloat16),    # C3 shape (nq 4)
    (1, 1, 1, 128, torch.bfloat16),     # C1 shape (nq 1)
    (1, 6, 2, 64, torch.bfloat16),      # nq 3 (padded to 4)
    (2, 2, 2, 128, torch.float32),      # two query tokens, nq 2
    (1, 4, 4, 256, torch.float32),      # fp32 keys, 64 lanes per row
    (1, 8, 2, 128, torch.float16),      # fp16, nq 4
    (1, 2, 2, 512, torch.bfloat16),     # 64 lanes per row, bf16
]


@pytest.mark.parametrize("sq,hq,hkv,d,dtype", CASES)
def test_score_logits_vs_oracle(dev, sq, hq, hkv, d, dtype):
    from orthocache_amd import _ops

    nb = 3
    q, k, v = make(dev, nb, sq, hq, hkv, d, dtype, seed=d + hq + sq)
    nq = sq * hq // hkv
    with_lg = _ops.score(k, q, want_logits=True)
    plain = _ops.score(k, q)
    torch.cuda.synchronize()
    lg = np32(with_lg.logits)
    nqp = _ops.logits_nq_pad(nq)
    assert lg.shape == (nb, hkv, 512, nqp)
    ref = O.block_logits(np32(q), np32(k)) * LOG2E
    close(lg[..., :nq], ref, 1e-5)
    assert np.all(lg[..., nq:] == 0.0)
    # The scores of the launch that also writes logits are the same bits.
    assert torch.equal(with_lg.zeta, plain.zeta)
    assert torch.equal(with_lg.tau_max, plain.tau_max)


def test_score_logits_segments_and_pages(dev):
    from orthocache_amd import _ops

    # Three segments of 2, 1 and 3 blocks in a shuffled page pool.
    hkv, g, d = 4, 2, 128
    seg_blocks = [2, 1, 3]
    nb = sum(seg_blocks)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    pool = torch.randn(nb * 512, hkv, d, generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn(3, 1, hkv * g, d, generator=gen, device=dev).to(torch.bfloat16)
    pages = torch.tensor([4, 0, 5, 2, 1, 3], dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 2, 3, 6], dtype=torch.int32, device=dev)
    res = _ops.score(pool, q, cu_blocks=cu, num_segments=3, pages=pages, want_logits=True)
    torch.cuda.synchronize()
    lg = np32(res.logits)
    poolf, qf, pg = np32(pool), np32(q), pages.cpu().numpy()
    j = 0
    for s, n in enumerate(seg_blocks):
        keys = np.concatenate([poolf[pg[b] * 512:(pg[b] + 1) * 512] for b in range(j, j + n)])
        ref = O.block_logits(qf[s], keys) * LOG2E
        close(lg[j:j + n, ..., :g], ref, 1e-5)
        j += n


def test_logits_limits(dev):
    from orthocache_amd import _ops

    q, k, _ = make(dev, 1, 1, 10, 2, 128, torch.bfloat16, seed=1)  # nq 5
    with pytest.raises(ValueError):
        _ops.score(k, q, want_logits=True)


@pytest.mark.parametrize("sq,hq,hkv,d,dtype", CASES)
def test_attend_from_logits(dev, sq, hq, hkv, d, dtype):
    from orthocache_amd import _ops

    nb = 5
    q, k, v = make(dev, nb, sq, hq, hkv, d, dtype, seed=3 * d + hq)
    sc = _ops.score(k, q, want_logits=True)
    mask = torch.tensor([1, 0, 1, 1, 0], dtype=torch.bool, device=dev)
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=mask)
    out_lg = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32, logits=sc.logits)
    out_k = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    ref = O.attention_active_blocks(np32(q), np32(k), np32(v), [0, 2, 3])
    tol = 1e-4 if dtype == torch.float32 else 2e-3
    close(np32(out_lg), ref, tol)
    close(np32(out_lg), np32(out_k), 1e-5)


def test_attend_from_logits_per_head_and_empty(dev):
    from orthocache_amd import _ops

    nb, hkv = 4, 2
    q, k, v = make(dev, nb, 1, 4, hkv, 128, torch.bfloat16, seed=9)
    sc = _ops.score(k, q, want_logits=True)
    # head 0 keeps blocks 1 and 3; head 1 keeps nothing (gated kernel: zeros)
    m = torch.tensor([[0, 0], [1, 0], [0, 0], [1, 0]], dtype=torch.bool, device=dev)
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=m, want_indices=False,
                          want_head_lists=True)
    out = _ops.attend(q, k, v, c.head_indices, c.head_num_active, per_head=True, out_dtype=torch.float32,
                      logits=sc.logits)
    ref = O.attention_per_head_gated(np32(q), np32(k), np32(v), m.cpu().numpy())
    close(np32(out), ref, 2e-3)
    assert np.all(np32(out)[:, 2:] == 0)


def test_decode_layer_uses_logits_and_matches(dev):
    """The fused layer (scoring-pass logits for nq <= 4) against the three
    separate calls without logits: same mask and permutation bit for bit,
    attention within fp32 rounding."""
    from orthocache_amd import _ops, workloads

    nb, hkv, hq, d = 16, 4, 8, 256
    k = workloads.make_keys(nb, hkv, d, seed=31, device=dev, noise_blocks=2)
    v = workloads.make_values(nb * 512, hkv, d, seed=32, device=dev)
    q = workloads.make_queries((1, hq, d), d, seed=33, device=dev)
    assert _ops.layer_uses_logits(k.dtype, d, hq // hkv, q.dtype)
    sc = _ops.score(k, q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, evict=0.75)
    layer = _ops.DecodeLayer(q, k, v, tau, zmax, out_dtype=torch.float32)
    out = layer.run()
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, tau_max=sc.tau_max, zeta=sc.zeta,
                          tau=tau, zeta_max=zmax)
    ref = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(layer.indices, c.indices) and torch.equal(layer.num_active, c.num_active)
    close(np32(out), np32(ref), 1e-5)


@pytest.mark.parametrize("hkv,hq,d,qdt", [
    (4, 4, 256, torch.float16),    # fp16, one row at head_dim 256
    (4, 4, 256, torch.float32),    # fp32 queries over fp16 keys
    (2, 8, 128, torch.float32),    # fp32 queries, four rows at head_dim 128
])
def test_decode_layer_fp16_without_logits(dev, hkv, hq, d, qdt):
    """fp16 shapes whose layer reads the keys in the attention instead of
    scoring-pass logits: same mask and list as the separate calls, attention
    within fp32 rounding, and the float64 oracle within the decode tolerance."""
    from orthocache_amd import _ops, workloads

    nb = 10
    k = workloads.make_keys(nb, hkv, d, seed=41, device=dev, dtype=torch.float16, noise_blocks=2)
    v = workloads.make_values(nb * 512, hkv, d, seed=42, device=dev, dtype=torch.float16)
    q = workloads.make_queries((1, hq, d), d, seed=43, device=dev, dtype=qdt)
    assert not _ops.layer_uses_logits(k.dtype, d, hq // hkv, q.dtype)
    sc = _ops.score(k, q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max[0], sc.zeta, evict=0.6)
    layer = _ops.DecodeLayer(q, k, v, tau, zmax, out_dtype=torch.float32)
    out = layer.run()
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, tau_max=sc.tau_max, zeta=sc.zeta,
                          tau=tau, zeta_max=zmax)
    ref = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(layer.indices, c.indices) and torch.equal(layer.num_active, c.num_active)
    close(np32(out), np32(ref), 1e-5)
    n = int(c.num_active[0])
    act = layer.indices[:n].cpu().numpy()
    close(np32(out), O.attention_active_blocks(np32(q), np32(k), np32(v), act), 2e-3)
    fused = out.clone()
    score, compact, attend = layer.phases()
    assert compact is None
    score()
    attend()
    torch.cuda.synchronize()
    assert float((fused - layer.out).abs().max()) <= 1e-5 * float(fused.abs().max())


@pytest.mark.parametrize("qdt", [torch.float16, torch.float32])
def test_ragged_decode_layer_fp16(dev, qdt):
    """A ragged fp16 batch through the fused layer: with fp32 queries (four
    rows at head_dim 128) the layer skips scoring-pass logits and the ranges
    attention reads the keys; with fp16 queries it uses the logits.  Lists
    match the oracle's mask and compaction exactly, attention the float64
    oracle within the decode tolerance."""
    from orthocache_amd import _ops, varlen, workloads

    hkv, hq, d = 2, 8, 128
    lens = [3 * 512, 512, 4 * 512]
    cu = np.concatenate([[0], np.cumsum(lens)]) // 512
    nb = int(cu[-1])
    k = workloads.make_keys(nb, hkv, d, seed=61, device=dev, dtype=torch.float16, noise_blocks=2)
    v = workloads.make_values(nb * 512, hkv, d, seed=62, device=dev, dtype=torch.float16)
    q = workloads.make_queries((len(lens), 1, hq, d), d, seed=63, device=dev, dtype=qdt)
    assert _ops.layer_uses_logits(k.dtype, d, hq // hkv, q.dtype) == (qdt == torch.float16)
    cu_seqlens = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    tm, z = varlen.score_varlen(q, k, cu_seqlens)
    taus, zmaxs = [], []
    for s in range(len(lens)):
        t, zm = workloads.calibrate_unified(tm[cu[s]:cu[s + 1]], z[cu[s]:cu[s + 1]], 0.5)
        taus.append(t)
        zmaxs.append(zm)
    tau_t = torch.tensor(taus, dtype=torch.float32, device=dev)
    zmax_t = torch.tensor(zmaxs, dtype=torch.float32, device=dev)
    out, meta = varlen.orthocache_decode_varlen(q, k, v, cu_seqlens, tau_t, zmax_t, out_dtype=torch.float32)
    torch.cuda.synchronize()
    idx = np32(meta["indices"]).astype(np.int64)
    tmn, zn = np32(meta["tau_max"]), np32(meta["zeta"])
    for s in range(len(lens)):
        lo, hi = cu[s], cu[s + 1]
        mask = O.mask_from_scores(tmn[lo:hi], zn[lo:hi], taus[s], zmaxs[s])
        order, n = O.stream_compact_indices(mask)
        np.testing.assert_array_equal(idx[lo:hi], order)
        assert int(meta["num_active"][s]) == n
        ref = O.attention_active_blocks(np32(q[s]), np32(k[lo * 512:hi * 512]), np32(v[lo * 512:hi * 512]),
                                        order[:n])
        close(np32(out[s]), ref, 2e-3)


@pytest.mark.parametrize("nb,hkv,hq,d,keep", [
    (1, 1, 1, 128, "all"), (2, 16, 32, 256, "all"), (13, 16, 32, 256, "some"), (128, 16, 32, 256, "some"),
    (7, 8, 32, 128, "none"), (40, 2, 8, 64, "some"), (300, 4, 4, 128, "some")])
def test_streaming_attention_edges(dev, nb, hkv, hq, d, keep):
    """The streaming form (one partial per (head, split); used with logits on
    one segment) against the key-reading attention and the oracle: a single
    block, fewer chunks than splits, empty and full lists, long lists."""
    from orthocache_amd import _ops

    q, k, v = make(dev, nb, 1, hq, hkv, d, torch.bfloat16, seed=nb * 7 + hkv)
    rng = np.random.default_rng(nb)
    m_np = {"all": np.ones(nb, bool), "none": np.zeros(nb, bool), "some": rng.random(nb) < 0.3}[keep]
    mask = torch.from_numpy(m_np).to(dev)
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=mask)
    sc = _ops.score(k, q, want_logits=True)
    out_lg = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32, logits=sc.logits)
    out_k = _ops.attend(q, k, v, c.indices, c.num_active, out_dtype=torch.float32)
    torch.cuda.synchronize()
    blocks = [int(j) for j in np.nonzero(m_np)[0]]
    ref = O.attention_active_blocks(np32(q), np32(k), np32(v), blocks)
    if not blocks:
        assert np.all(np32(out_lg) == 0) and np.all(np32(out_k) == 0)
        return
    close(np32(out_lg), ref, 2e-3)
    close(np32(out_lg), np32(out_k), 1e-5)


@pytest.mark.parametrize("empty_head_all", [False, True])
def test_streaming_per_head_lists_and_uniform(dev, empty_head_all):
    """Per-head lists through the logits path, including a head that keeps
    nothing: zeros (gated kernel) or equal weights over every block (the
    predicated reference's all-masked softmax, uniform flag)."""
    from orthocache_amd import _ops

    nb, hkv, hq, d = 6, 3, 6, 128
    q, k, v = make(dev, nb, 1, hq, hkv, d, torch.bfloat16, seed=19)
    sc = _ops.score(k, q, want_logits=True)
    m = np.zeros((nb, hkv), bool)
    m[[0, 3, 4], 0] = True
    m[[5], 1] = True  # head 2 keeps nothing
    mask = torch.from_numpy(m).to(dev)
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=mask, want_indices=False,
                          want_head_lists=True, empty_head_all=empty_head_all)
    kw = dict(per_head=True, uniform=c.head_uniform if empty_head_all else None, out_dtype=torch.float32)
    out_lg = _ops.attend(q, k, v, c.head_indices, c.head_num_active, logits=sc.logits, **kw)
    out_k = _ops.attend(q, k, v, c.head_indices, c.head_num_active, **kw)
    torch.cuda.synchronize()
    if empty_head_all:
        ref = O.attention_per_head_predicated(np32(q), np32(k), np32(v), m)
    else:
        ref = O.attention_per_head_gated(np32(q), np32(k), np32(v), m)
    close(np32(out_lg), ref, 2e-3)
    close(np32(out_lg), np32(out_k), 1e-5)


def test_streaming_ragged_segments(dev):
    """Several segments of very different retained lengths (one empty) through
    the logits path, against the key-reading attention and the oracle."""
    from orthocache_amd import _ops

    hkv, hq, d = 4, 16, 128
    seg_blocks = [9, 1, 30, 4]
    keep = [[0, 3, 8], [], list(range(0, 30, 2)), [1, 2, 3]]
    nb = sum(seg_blocks)
    gen = torch.Generator(device=dev)
    gen.manual_seed(23)
    k = torch.randn(nb * 512, hkv, d, generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn(nb * 512, hkv, d, generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn(len(seg_blocks), 1, hq, d, generator=gen, device=dev).to(torch.bfloat16)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(seg_blocks)]), dtype=torch.int32, device=dev)
    m = np.zeros(nb, bool)
    off = 0
    for n, kb in zip(seg_blocks, keep):
        m[[off + j for j in kb]] = True
        off += n
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=torch.from_numpy(m).to(dev),
                          cu_blocks=cu, num_segments=len(seg_blocks))
    sc = _ops.score(k, q, cu_blocks=cu, num_segments=len(seg_blocks), want_logits=True)
    kw = dict(cu_blocks=cu, num_segments=len(seg_blocks), out_dtype=torch.float32)
    out_lg = _ops.attend(q, k, v, c.indices, c.num_active, logits=sc.logits, **kw)
    out_k = _ops.attend(q, k, v, c.indices, c.num_active, **kw)
    torch.cuda.synchronize()
    close(np32(out_lg), np32(out_k), 1e-5)
    off = 0
    qn, kn, vn = np32(q), np32(k), np32(v)
    for s, (n, kb) in enumerate(zip(seg_blocks, keep)):
        ks, vs = kn[off * 512:(off + n) * 512], vn[off * 512:(off + n) * 512]
        ref = O.attention_active_blocks(qn[s], ks, vs, kb)
        if kb:
            close(np32(out_lg)[s], ref, 2e-3)
        else:
            assert np.all(np32(out_lg)[s] == 0)
        off += n


def _rising_keys(dev, q, hkv, nblk, centers, seed):
    """Keys whose logits against the kv head's (shared) query direction sit
    around a per-block centre (log2 units) with a spread of +-3: the streaming
    softmax's reference point must move by less and by more than its 2^8
    headroom from block to block."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    sq, hq, d = q.shape[-3:]
    grp = hq // hkv
    qf = q.float().reshape(-1, hq, d)[0]
    k = torch.empty(nblk * 512, hkv, d, device=dev)
    for h in range(hkv):
        u = qf[h * grp:(h + 1) * grp].mean(0)
        scale = math.sqrt(d) / LOG2E / float(u.dot(u))
        t = torch.tensor(centers, device=dev, dtype=torch.float32).repeat_interleave(512)
        t = t + 3.0 * torch.randn(nblk * 512, generator=g, device=dev)
        k[:, h] = t[:, None] * scale * u[None, :] + 0.05 * torch.randn(nblk * 512, d, generator=g, device=dev)
    return k.to(q.dtype)


@pytest.mark.parametrize("form", ["split", "ranges"])
def test_streaming_lazy_rescale_rising_logits(dev, form):
    """Logit levels that climb block by block, in steps below and above the
    2^8 headroom of the lazy rescale (and one that falls back), through the
    scoring-pass logits and the streaming attention, against the oracle."""
    from orthocache_amd import _ops

    hkv, hq, d = 2, 8, 128
    centers = [0.0, 2.0, 4.0, 15.0, 16.0, 30.0, 5.0, 31.0, 45.0, 44.0]
    nblk = len(centers)
    gen = torch.Generator(device=dev)
    gen.manual_seed(41)
    nseg = 1 if form == "split" else 2
    q = (torch.randn(nseg, 1, hq, d, generator=gen, device=dev) * 0.2 + 1.0).to(torch.bfloat16)
    ks, vs = [], []
    for s in range(nseg):
        ks.append(_rising_keys(dev, q[s], hkv, nblk, centers, seed=42 + s))
        vs.append(torch.randn(nblk * 512, hkv, d, generator=gen, device=dev).to(torch.bfloat16))
    k, v = torch.cat(ks), torch.cat(vs)
    keep = [0, 1, 2, 3, 5, 6, 7, 8, 9]  # block 4 evicted
    m = np.zeros(nblk * nseg, bool)
    for s in range(nseg):
        m[[s * nblk + j for j in keep]] = True
    if form == "split":
        qq = q[0]
        c = _ops.mask_compact(num_blocks=nblk, num_kv_heads=hkv, device=dev, mask_in=torch.from_numpy(m).to(dev))
        sc = _ops.score(k, qq, want_logits=True)
        kw = dict(out_dtype=torch.float32)
    else:
        qq = q
        cu = torch.tensor([0, nblk, 2 * nblk], dtype=torch.int32, device=dev)
        c = _ops.mask_compact(num_blocks=nblk * nseg, num_kv_heads=hkv, device=dev, mask_in=torch.from_numpy(m).to(dev),
                              cu_blocks=cu, num_segments=nseg)
        sc = _ops.score(k, qq, cu_blocks=cu, num_segments=nseg, want_logits=True)
        kw = dict(cu_blocks=cu, num_segments=nseg, out_dtype=torch.float32)
    out = _ops.attend(qq, k, v, c.indices, c.num_active, logits=sc.logits, **kw)
    torch.cuda.synchronize()
    lg = np32(sc.logits)
    assert lg.max() - lg.min() > 60.0  # the designed spread of logit levels is present
    qn, kn, vn, on = np32(q), np32(k), np32(v), np32(out).reshape(nseg, 1, hq, d)
    for s in range(nseg):
        sl = slice(s * nblk * 512, (s + 1) * nblk * 512)
        ref = O.attention_active_blocks(qn[s], kn[sl], vn[sl], keep)
        close(on[s], ref, 2e-3)


def test_ranges_combine_many_partials(dev):
    """One list far longer than the other: with four query rows the ranges
    form cuts the 4808 chunks into 512 ranges of 10, so the long list is
    merged from 480 partials (one per workgroup piece) -- more than one batch
    of staged weights in the per-list combine.  Against the key-reading
    attention (a different partition) and the oracle."""
    from orthocache_amd import _ops

    hkv, hq, d = 1, 4, 128
    seg_blocks = [600, 2]
    nb = sum(seg_blocks)
    gen = torch.Generator(device=dev)
    gen.manual_seed(51)
    k = torch.randn(nb * 512, hkv, d, generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn(nb * 512, hkv, d, generator=gen, device=dev).to(torch.bfloat16)
    q = torch.randn(len(seg_blocks), 1, hq, d, generator=gen, device=dev).to(torch.bfloat16)
    cu = torch.tensor([0, 600, 602], dtype=torch.int32, device=dev)
    m = np.zeros(nb, bool)
    m[:600] = True
    m[601] = True
    c = _ops.mask_compact(num_blocks=nb, num_kv_heads=hkv, device=dev, mask_in=torch.from_numpy(m).to(dev),
                          cu_blocks=cu, num_segments=2)
    sc = _ops.score(k, q, cu_blocks=cu, num_segments=2, want_logits=True)
    kw = dict(cu_blocks=cu, num_segments=2, out_dtype=torch.float32)
    out_lg = _ops.attend(q, k, v, c.indices, c.num_active, logits=sc.logits, **kw)
    out_k = _ops.attend(q, k, v, c.indices, c.num_active, **kw)
    torch.cuda.synchronize()
    close(np32(out_lg), np32(out_k), 1e-5)
    qn, kn, vn = np32(q), np32(k), np32(v)
    close(np32(out_lg)[0], O.attention_active_blocks(qn[0], kn[:600 * 512], vn[:600 * 512], range(600)), 2e-3)
    close(np32(out_lg)[1], O.attention_active_blocks(qn[1], kn[600 * 512:], vn[600 * 512:], [1]), 2e-3)
