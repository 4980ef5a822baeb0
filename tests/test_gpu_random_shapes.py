"""GPU parity on seeded random shapes: the decode layer and the prefill layer.

Each case draws its shape from a fixed seed (key dtype, head_dim, kv heads,
GQA group, query tokens, query and output dtypes, block counts, ragged
segments, eviction), so the sweep reaches combinations that the hand-picked
cases of the other files do not: two-head scoring tiles with logits and odd
head counts, 16-bit outputs of the split-partial combine, several segments of
one to a dozen blocks, caches paged over a pool in random page order, every
block or no block kept.  Checked per case:

- the layer's scores (``tau_max``, ``zeta``) against the float64 oracle
  (``query_aware_bounds`` over the folded GQA queries, ``spectral_decay_ratio``),
  rtol/atol 1e-5 (prefill: the per-tile maxima);
- mask, active-first permutation and count bit for bit against the oracle's
  two-gate mask and compaction applied to the layer's own fp32 scores;
- the attention output against the float64 oracle over the retained blocks:
  1e-4 of the output scale for fp32 inputs and output, 2e-3 for 16-bit inputs
  with an fp32 output, 1e-2 with a 16-bit output (bf16 rounding of the result).
"""

import numpy as np
import pytest
import torch

from oracle import oc_oracle as O

pytestmark = pytest.mark.gpu

BLOCK = 512
DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def np32(t):
    return t.detach().float().cpu().numpy()


def close(out, ref, rel):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(np.abs(ref).max(), 1e-6)
    err = np.abs(out - ref).max() / scale
    assert err <= rel, f"max error {err:.3e} relative to scale (tolerance {rel})"


def tolerance(kv, out):
    if kv == "f32" and out == "f32":
        return 1e-4
    return 2e-3 if out == "f32" else 1e-2


def decode_case(i):
    r = np.random.default_rng(7000 + i)
    kv = str(r.choice(["bf16", "bf16", "f16", "f32"]))
    d = int(r.choice([32, 64, 128, 256] if kv == "f32" else [64, 128, 128, 256]))
    hkv = int(r.choice([1, 2, 3, 4, 8]))
    group = int(r.choice([1, 2, 4, 8]))
    sq = int(r.choice([1, 1, 1, 2, 3]))
    while sq * group > 16:
        sq -= 1
    qdt = "f32" if r.random() < 0.2 else kv
    out = "f32" if r.random() < 0.5 else kv
    nseg = 1 if r.random() < 0.6 else int(r.integers(2, 5))
    lens = [int(x) for x in r.integers(1, 13, size=nseg)]
    evict = float(r.choice([0.0, 0.3, 0.5, 0.75, 1.0]))
    paged = bool(r.random() < 0.3)
    return dict(kv=kv, d=d, hkv=hkv, group=group, sq=sq, qdt=qdt, out=out, lens=lens, evict=evict, paged=paged,
                seed=7000 + i)


def prefill_case(i):
    r = np.random.default_rng(9000 + i)
    kv = str(r.choice(["bf16", "f16"]))
    d = int(r.choice([64, 128]))
    hkv = int(r.choice([1, 2, 4]))
    group = int(r.choice([1, 2, 4]))
    sq = int(r.integers(17, 300))
    out = "f32" if r.random() < 0.4 else kv
    nb = int(r.integers(2, 17))
    evict = float(r.choice([0.25, 0.5, 0.75]))
    return dict(kv=kv, d=d, hkv=hkv, group=group, sq=sq, out=out, nb=nb, evict=evict, seed=9000 + i)


def case_id(c):
    lens = c.get("lens", [c.get("nb")])
    qdt = f"-q{c['qdt']}" if c.get("qdt", c["kv"]) != c["kv"] else ""
    return (f"{c['kv']}{qdt}-d{c['d']}-kv{c['hkv']}x{c['group']}-sq{c['sq']}-out{c['out']}-"
            f"nb{'+'.join(map(str, lens))}-ev{c['evict']}{'-paged' if c.get('paged') else ''}")


DECODE = [decode_case(i) for i in range(40)]
PREFILL = [prefill_case(i) for i in range(12)]


@pytest.mark.parametrize("c", DECODE, ids=[case_id(c) for c in DECODE])
def test_random_decode_layer(dev, c):
    from orthocache_amd import _ops, workloads

    print("case", case_id(c), "seed", c["seed"], flush=True)
    kv, d, hkv, group, sq = DT[c["kv"]], c["d"], c["hkv"], c["group"], c["sq"]
    lens = c["lens"]
    nseg, nb = len(lens), sum(lens)
    k = workloads.make_keys(nb, hkv, d, seed=c["seed"], device=dev, dtype=kv, noise_blocks=max(1, nb // 5))
    v = workloads.make_values(nb * BLOCK, hkv, d, seed=c["seed"] + 1, device=dev, dtype=kv)
    multi = nseg > 1
    qshape = (nseg, sq, hkv * group, d) if multi else (sq, hkv * group, d)
    q = workloads.make_queries(qshape, d, seed=c["seed"] + 2, device=dev, dtype=DT[c["qdt"]])
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    kw = dict(cu_blocks=torch.from_numpy(cu).to(dev), num_segments=nseg) if multi else {}
    kl, vl = k, v   # the logical caches the oracle reads
    if c["paged"]:
        # scatter the logical blocks over a larger pool of pages in random order;
        # the unused pages hold other values
        g = torch.Generator().manual_seed(c["seed"] + 3)
        npages = nb + 3
        pages = torch.randperm(npages, generator=g)[:nb].to(torch.int32)
        pool = lambda x: torch.randn((npages * BLOCK,) + tuple(x.shape[1:]), generator=g).to(x.dtype).to(dev)
        k, v = pool(kl), pool(vl)
        k.view(npages, BLOCK, hkv, d)[pages.long()] = kl.view(nb, BLOCK, hkv, d)
        v.view(npages, BLOCK, hkv, d)[pages.long()] = vl.view(nb, BLOCK, hkv, d)
        kw["pages"] = pages.to(dev)

    sc = _ops.score(k, q, **kw)
    taus, zmaxs = [], []
    for s in range(nseg):
        t, z = workloads.calibrate_unified(sc.tau_max[0][cu[s]:cu[s + 1]], sc.zeta[cu[s]:cu[s + 1]], c["evict"])
        taus.append(t)
        zmaxs.append(z)
    if multi:
        tau = torch.tensor(taus, dtype=torch.float32, device=dev)
        zmax = torch.tensor(zmaxs, dtype=torch.float32, device=dev)
    else:
        tau, zmax = taus[0], zmaxs[0]
    layer = _ops.DecodeLayer(q, k, v, tau, zmax, out_dtype=DT[c["out"]], **kw)
    out = layer.run()
    torch.cuda.synchronize()

    tm, zn = np32(layer.tau_max), np32(layer.zeta)
    idx = np32(layer.indices).astype(np.int64)
    qn, kn, vn = np32(q), np32(kl), np32(vl)
    for s in range(nseg):
        lo, hi = int(cu[s]), int(cu[s + 1])
        kseg, vseg = kn[lo * BLOCK:hi * BLOCK], vn[lo * BLOCK:hi * BLOCK]
        qs = qn[s] if multi else qn
        np.testing.assert_allclose(tm[lo:hi], O.query_aware_bounds(O.fold_gqa(qs, hkv), kseg).max(axis=0),
                                   rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(zn[lo:hi], O.spectral_decay_ratio(kseg), rtol=1e-5, atol=1e-6)
        mask = O.mask_from_scores(tm[lo:hi], zn[lo:hi], taus[s], zmaxs[s])
        order, n = O.stream_compact_indices(mask)
        assert int(layer.num_active[s]) == n
        np.testing.assert_array_equal(idx[lo:hi], order)
        ref = O.attention_active_blocks(qs, kseg, vseg, order[:n])
        got = np32(out[s] if multi else out)
        if n == 0:
            assert np.all(got == 0.0)
        else:
            close(got, ref, tolerance(c["kv"] if c["qdt"] == c["kv"] else "bf16", c["out"]))


@pytest.mark.parametrize("c", PREFILL, ids=[case_id(c) for c in PREFILL])
def test_random_prefill_layer(dev, c):
    from orthocache_amd import _ops, workloads

    print("case", case_id(c), "seed", c["seed"], flush=True)
    kv, d, hkv, group, sq, nb = DT[c["kv"]], c["d"], c["hkv"], c["group"], c["sq"], c["nb"]
    k = workloads.make_keys(nb, hkv, d, seed=c["seed"], device=dev, dtype=kv, noise_blocks=max(1, nb // 5))
    v = workloads.make_values(nb * BLOCK, hkv, d, seed=c["seed"] + 1, device=dev, dtype=kv)
    q = workloads.make_queries((sq, hkv * group, d), d, seed=c["seed"] + 2, device=dev, dtype=kv)
    sc = _ops.score(k, q)
    tau, zmax = workloads.calibrate_unified(sc.tau_max.amax(dim=0), sc.zeta, c["evict"])
    layer = _ops.PrefillLayer(q, k, v, tau, zmax, out_dtype=DT[c["out"]])
    out = layer.run()
    torch.cuda.synchronize()

    parts, zn = np32(layer.tau_max), np32(layer.zeta)
    qn, kn, vn = np32(q), np32(k), np32(v)
    qf = O.fold_gqa(qn, hkv)                                    # (sq*group, hkv, d), row t*group + g
    bounds = O.query_aware_bounds(qf, kn)                       # (sq*group, nb, hkv)
    tile = 64                                                   # query rows per bound tile
    assert parts.shape[0] == -(-qf.shape[0] // tile)
    for p in range(parts.shape[0]):
        seg = bounds[p * tile:(p + 1) * tile]
        if seg.shape[0]:
            np.testing.assert_allclose(parts[p], seg.max(axis=0), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(zn, O.spectral_decay_ratio(kn), rtol=1e-5, atol=1e-6)
    mask = O.mask_from_scores(O.nanmax_axis0(parts), zn, tau, zmax)
    order, n = O.stream_compact_indices(mask)
    assert int(layer.num_active[0]) == n
    np.testing.assert_array_equal(np32(layer.indices).astype(np.int64), order)
    pick = np.sort(np.random.default_rng(c["seed"]).choice(sq, min(sq, 24), replace=False))
    ref = O.attention_active_blocks(qn[pick], kn, vn, order[:n])
    close(np32(out)[pick], ref, tolerance(c["kv"], c["out"]))
