"""CPU tests of the host side: the C-ABI library surface and the scoring identity.

No GPU work is launched: the library is loaded, its exports are checked
against include/orthocache_hip.h, and argument validation is exercised on
NULL or malformed arguments (which fail before any device call).
"""

import ctypes as C
import os
import re

import numpy as np
import pytest
from scipy.linalg import hadamard

from oracle import oc_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "orthocache_hip.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:oc|orthocache)_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from orthocache_amd import _native as N

    if not N.LIB_PATH.exists():
        pytest.fail("liborthocache_hip.so is not built: run __graft_entry__.build()")
    return N.lib()


def test_library_exports_every_declared_symbol(lib):
    syms = _declared_symbols()
    assert len(syms) >= 14
    missing = [s for s in syms if not hasattr(lib, s)]
    assert missing == []


def test_binding_covers_header(lib):
    from orthocache_amd import _native as N

    assert set(N.EXPORTED_SYMBOLS) == set(_declared_symbols())


def test_abi_version(lib):
    assert lib.oc_abi_version() == 3


def test_struct_sizes_match_header_layout(lib):
    # Field counts mirror the C structs; a mismatch would shift every field.
    from orthocache_amd import _native as N

    text = open(HEADER).read()
    for cname, py in (("oc_fwht_args", N.FwhtArgs), ("oc_score_args", N.ScoreArgs),
                      ("oc_bound_args", N.BoundArgs), ("oc_compact_args", N.CompactArgs),
                      ("oc_attend_args", N.AttendArgs), ("oc_layer_args", N.LayerArgs),
                      ("oc_block_stats", N.BlockStats)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (cname, cname), text, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body)
        names = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            decl = re.sub(r"^(const\s+)?[a-z0-9_]+\s*\**\s*", "", decl)
            names += [n.strip().lstrip("*") for n in decl.split(",")]
        assert names == [f[0] for f in py._fields_], cname


def test_validation_errors_without_gpu(lib):
    from orthocache_amd import _native as N

    a = N.ScoreArgs()
    assert lib.oc_score_blocks(C.byref(a), None) == -1
    assert b"NULL" in lib.oc_last_error()
    a.keys = 16
    a.keys_dtype = 1
    a.head_dim = 96  # 96 bf16 = 12 lanes of 8: not a supported layout
    a.keys_tok_stride = 96
    a.keys_head_stride = 96
    a.num_kv_heads = 1
    assert lib.oc_score_blocks(C.byref(a), None) == -2
    assert b"head_dim" in lib.oc_last_error()
    c = N.CompactArgs()
    assert lib.oc_mask_compact(C.byref(c), None) == -1
    assert lib.oc_copy_blocks(16, 16, 16, 16, 1, 100, 0, None) == -1  # not a multiple of 16
    assert lib.oc_band_energy(16, 1, 1, 1, 10, 5, 16, None) == -1  # s0 > s1
    assert lib.oc_query_bound_tiles(2, 16) == 1
    assert lib.oc_query_bound_tiles(512, 1) == 8
    assert lib.oc_query_bound_tiles(65, 1) == 2


def test_cached_layer_rejects_null_stats(lib):
    from orthocache_amd import _native as N

    a = N.LayerArgs()
    assert lib.oc_decode_layer_cached(C.byref(a), None, None, 0, None) == -1
    st = N.BlockStats()
    assert lib.oc_decode_layer_cached(C.byref(a), C.byref(st), None, 0, None) == -1
    assert lib.oc_decode_layer_cached_workspace_size(C.byref(a)) == 0


def test_attend_workspace_rejects_bad_args(lib):
    from orthocache_amd import _native as N

    a = N.AttendArgs()
    assert lib.oc_attend_workspace_size(C.byref(a)) == 0
    assert lib.oc_attend(C.byref(a), None, 0, None) == -1


def _plan_args(sq, hq, hkv, d, dtype, block=512, nb=256, q_dtype=None):
    """AttendArgs with fake, aligned device addresses: oc_attend_plan only
    validates and sizes, it never dereferences them."""
    from orthocache_amd import _native as N

    a = N.AttendArgs()
    fake = 1 << 20
    a.q = a.k = a.v = a.out = a.indices = a.counts = fake
    a.q_dtype = dtype if q_dtype is None else q_dtype
    a.kv_dtype = a.out_dtype = dtype
    a.q_tok_stride, a.q_head_stride = hq * d, d
    a.k_tok_stride = a.v_tok_stride = hkv * d
    a.k_head_stride = a.v_head_stride = d
    a.out_tok_stride, a.out_head_stride = hq * d, d
    a.head_dim, a.num_kv_heads, a.group, a.sq = d, hkv, hq // hkv, sq
    a.block_size, a.total_blocks, a.num_segments = block, nb, 1
    return a


@pytest.mark.parametrize("sq,hq,hkv,d,dt,block,qdt,expect", [
    (512, 8, 8, 128, 1, 512, None, (1, 16)),   # C4: 16 (head, 256-row) tiles x 16 splits
    (512, 8, 8, 128, 2, 512, None, (1, 16)),   # fp16
    (512, 8, 8, 64, 1, 512, None, (1, 16)),
    (16, 32, 8, 128, 1, 512, None, (1, 16)),   # 4 x 16 = 64 rows per kv head, one query tile
    (32, 1, 1, 128, 1, 512, None, (1, 16)),    # threshold: 32 rows
    (31, 1, 1, 128, 1, 512, None, (0, 0)),     # below it: decode kernel
    (1, 32, 16, 256, 1, 512, None, (0, 0)),    # C2 decode
    (512, 8, 8, 256, 1, 512, None, (0, 0)),    # head_dim 256: decode kernel
    (512, 8, 8, 128, 0, 512, None, (0, 0)),    # fp32 K/V
    (512, 8, 8, 128, 1, 512, 0, (0, 0)),       # fp32 q with bf16 K/V
    (512, 8, 8, 128, 1, 100, None, (0, 0)),    # block not a multiple of 64
])
def test_attend_plan_routing(lib, sq, hq, hkv, d, dt, block, qdt, expect):
    a = _plan_args(sq, hq, hkv, d, dt, block=block, nb=256 if block == 512 else 6, q_dtype=qdt)
    kern, ns = C.c_int32(-1), C.c_int32(-1)
    assert lib.oc_attend_plan(C.byref(a), C.byref(kern), C.byref(ns)) == 0, lib.oc_last_error()
    assert (kern.value, ns.value) == expect


def test_attend_plan_split_is_bounded_by_tiles(lib):
    # 2 blocks x 8 tiles: at most 16 / 8 = 2 splits (about 8 tiles each).
    a = _plan_args(512, 8, 8, 128, 1, nb=2)
    kern, ns = C.c_int32(), C.c_int32()
    assert lib.oc_attend_plan(C.byref(a), C.byref(kern), C.byref(ns)) == 0
    assert (kern.value, ns.value) == (1, 2)
    assert lib.oc_attend_plan(None, C.byref(kern), C.byref(ns)) == -1


def _kernel_band_identity(block):
    """NumPy emulation of the scoring kernel's arithmetic for one (512, D) tile:
    bit-8 differences, a 4-point WHT over bits 6-7, and a centred low band."""
    x = block.reshape(8, 64, -1)          # x[k, l, d] = K[64k + l, d]
    d = x[:4] - x[4:]
    e_high = 0.5 * np.sum(d * d)
    u = x[:4] + x[4:]
    a0, a1, a2, a3 = u[0] + u[1], u[0] - u[1], u[2] + u[3], u[2] - u[3]
    # The kernel forms y1^2 + y3^2 as 2 a1^2 + 2 a3^2 (y1, y3 = a1 +- a3).
    y0, y2 = a0 + a2, a0 - a2
    e_mid = 0.125 * np.sum(2.0 * a1 * a1 + 2.0 * a3 * a3 + y2 * y2)
    e_low = 0.125 * np.sum((y0 - y0.mean(axis=0, keepdims=True)) ** 2)
    dc = y0.sum(axis=0) / np.sqrt(512)
    return dc, e_low, e_mid, e_high


@pytest.mark.parametrize("offset", [0.0, 5.0, 1e3])
def test_scoring_identity_matches_full_spectrum(offset):
    rng = np.random.default_rng(20)
    blk = rng.standard_normal((512, 24)) + offset * rng.standard_normal(24)
    dc, lo, mi, hi = _kernel_band_identity(blk)
    c = hadamard(512) @ blk / np.sqrt(512)
    np.testing.assert_allclose(dc, c[0], rtol=1e-12, atol=1e-9)
    np.testing.assert_allclose(lo, np.sum(c[1:64] ** 2), rtol=1e-9)
    np.testing.assert_allclose(mi, np.sum(c[64:256] ** 2), rtol=1e-9)
    np.testing.assert_allclose(hi, np.sum(c[256:] ** 2), rtol=1e-9)


def test_scoring_identity_fp32_cancellation_free():
    # A large block mean must not swamp the low band (the centred form keeps
    # it; E_0 - DC^2 in fp32 would lose it).
    rng = np.random.default_rng(21)
    blk = (rng.standard_normal((512, 64)) * 0.01 + 100.0).astype(np.float32)
    _, lo32, _, _ = _kernel_band_identity(blk.astype(np.float32))
    _, lo, _, _ = O.spectral_bands(blk.reshape(512, 1, 64).astype(np.float64))
    np.testing.assert_allclose(lo32, lo[0, 0], rtol=1e-4)


@pytest.mark.parametrize("kv", ["bf16", "f16"])
@pytest.mark.parametrize("qf32", [False, True])
@pytest.mark.parametrize("d,nq", [(64, 1), (128, 1), (128, 2), (128, 3), (128, 4), (256, 1), (256, 2),
                                  (256, 4), (512, 1), (128, 5)])
def test_layer_logits_choice_matches_library(lib, kv, qf32, d, nq):
    """_ops.layer_uses_logits restates the library's choice: the layer
    workspace exceeds the cached layer's (which never forms logits) by the
    logits buffer exactly when the scoring pass writes them."""
    import torch

    from orthocache_amd import _native as N, _ops

    kdt = torch.bfloat16 if kv == "bf16" else torch.float16
    qdt = torch.float32 if qf32 else kdt
    nb, hkv = 24, 2
    a = N.LayerArgs()
    a.q = 256; a.q_dtype = N.dtype_code(qdt); a.q_tok_stride = nq * hkv * d; a.q_head_stride = d
    a.k = 256; a.v = 256; a.kv_dtype = N.dtype_code(kdt)
    a.k_tok_stride = a.v_tok_stride = hkv * d; a.k_head_stride = a.v_head_stride = d
    a.head_dim = d; a.num_kv_heads = hkv; a.group = nq; a.sq = 1; a.total_blocks = nb; a.num_segments = 1
    a.out = 256; a.out_dtype = N.dtype_code(qdt); a.out_tok_stride = nq * hkv * d; a.out_head_stride = d
    full = int(lib.oc_decode_layer_workspace_size(C.byref(a)))
    cached = int(lib.oc_decode_layer_cached_workspace_size(C.byref(a)))
    assert full > 0 and cached > 0
    logit_bytes = -(-nb * hkv * 512 * _ops.logits_nq_pad(nq) * 4 // 256) * 256
    uses = _ops.layer_uses_logits(kdt, d, nq, qdt)
    assert full - cached == (logit_bytes if uses else 0)
    if kv == "bf16" and nq <= 4 and d <= 256:
        assert uses


def test_unaligned_workspace_rejected(lib):
    """A workspace that is not 256-byte aligned is refused before any launch
    (the kernels read it with 16-byte vector loads at 256-byte offsets)."""
    from orthocache_amd import _native as N

    a = _plan_args(1, 32, 16, 256, 1, nb=128)
    need = int(lib.oc_attend_workspace_size(C.byref(a)))
    assert need > 0
    base = 1 << 24
    assert lib.oc_attend(C.byref(a), base + 16, need + 256, None) == -1
    assert b"256-byte aligned" in lib.oc_last_error()
    la = N.LayerArgs()
    for f in ("q", "k", "v", "out"):
        setattr(la, f, 1 << 20)
    la.q_dtype = la.kv_dtype = la.out_dtype = 1
    la.q_tok_stride = la.out_tok_stride = 32 * 256
    la.q_head_stride = la.out_head_stride = la.k_head_stride = la.v_head_stride = 256
    la.k_tok_stride = la.v_tok_stride = 16 * 256
    la.head_dim, la.num_kv_heads, la.group, la.sq, la.total_blocks, la.num_segments = 256, 16, 2, 1, 128, 1
    need = int(lib.oc_decode_layer_workspace_size(C.byref(la)))
    assert need > 0
    assert lib.oc_decode_layer(C.byref(la), base + 128, need + 256, None) == -1
    assert b"256-byte aligned" in lib.oc_last_error()


def test_noalloc_rejects_layers_beyond_its_scratch(lib):
    """oc_decode_layer_noalloc refuses, before any launch or device call, a
    layer whose workspace exceeds the library's fixed scratch (here C2's shape
    at 512K tokens: 67 MB of scoring-pass logits alone)."""
    from orthocache_amd import _native as N

    la = N.LayerArgs()
    for f in ("q", "k", "v", "out"):
        setattr(la, f, 1 << 20)
    la.q_dtype = la.kv_dtype = la.out_dtype = 1
    la.q_tok_stride = la.out_tok_stride = 32 * 256
    la.q_head_stride = la.out_head_stride = la.k_head_stride = la.v_head_stride = 256
    la.k_tok_stride = la.v_tok_stride = 16 * 256
    la.head_dim, la.num_kv_heads, la.group, la.sq, la.num_segments = 256, 16, 2, 1, 1
    la.total_blocks = 1024
    need = int(lib.oc_decode_layer_workspace_size(C.byref(la)))
    assert need > N.NOALLOC_SCRATCH_BYTES
    assert lib.oc_decode_layer_noalloc(C.byref(la), None) == -4
    msg = lib.oc_last_error()
    assert b"scratch" in msg and str(need).encode() in msg
    # C2 at 64K tokens fits
    la.total_blocks = 128
    assert 0 < int(lib.oc_decode_layer_workspace_size(C.byref(la))) <= N.NOALLOC_SCRATCH_BYTES
    assert lib.oc_decode_layer_noalloc(None, None) == -1


@pytest.mark.parametrize("nb,hkv,evict,seed", [(128, 16, 0.9, 0), (128, 16, 0.5, 1), (16, 1, 0.5, 2), (40, 3, 0.75, 3)])
def test_calibrate_unified_thresholds_off_the_scores(nb, hkv, evict, seed):
    """calibrate_unified (host-side, CPU tensors here) places tau strictly
    between the K-th and (K+1)-th unified scores and zeta_max strictly between
    two zeta values: the mask keeps exactly K blocks and no score equals a
    threshold, so a restatement whose scores differ in the last bits keeps
    the same blocks."""
    import torch

    from orthocache_amd import workloads

    g = torch.Generator().manual_seed(seed)
    tm = torch.randn(nb, hkv, generator=g) * 3 + 40
    z = torch.rand(nb, hkv, generator=g) * 8
    tau, zmax = workloads.calibrate_unified(tm, z, evict)
    assert tau == float(np.float32(tau)) and zmax == float(np.float32(zmax))
    tmn, zn = tm.numpy(), z.numpy()
    assert not np.any(tmn == np.float32(tau)) and not np.any(zn == np.float32(zmax))
    mask = O.mask_from_scores(tmn, zn, tau, zmax)
    _, n = O.stream_compact_indices(mask)
    assert n == int(round(nb * (1 - evict)))
    # nudging every score by 4 ulps either way keeps the same mask
    for direction in (np.inf, -np.inf):
        nudged = tmn.copy()
        for _ in range(4):
            nudged = np.nextafter(nudged, np.float32(direction))
        np.testing.assert_array_equal(O.mask_from_scores(nudged, zn, tau, zmax), mask)


def test_partitioned_rejects_uneven_head_shards():
    """The head-sharding rule of partitioning.py:46-50 needs both head axes to
    split evenly; the check runs before anything touches a device."""
    import torch

    import orthocache_amd as oc

    q = torch.zeros(1, 4, 64)
    kv = torch.zeros(512, 2, 64)
    m = torch.ones(1, 2, dtype=torch.bool)
    with pytest.raises(ValueError, match="split evenly"):
        oc.orthocache_attention_partitioned(q, kv, kv, m, num_shards=3)
    with pytest.raises(ValueError, match=">= 1"):
        oc.orthocache_attention_partitioned(q, kv, kv, m, num_shards=0)


def test_custom_call_rejects_bad_descriptors(lib):
    """orthocache_compacted_attention checks its descriptor before any device
    call: a missing descriptor, negative sizes and a key count that is not
    num_blocks * block_size leave oc_last_error() set; no query rows is a
    no-op."""

    class Desc(C.Structure):
        _fields_ = [("seq_len_q", C.c_int32), ("seq_len_k", C.c_int32), ("head_dim", C.c_int32),
                    ("block_size", C.c_int32), ("num_blocks", C.c_int32)]

    def call(desc):
        ins = (C.c_void_p * 5)(16, 16, 16, 16, C.addressof(desc) if desc is not None else None)
        lib.orthocache_compacted_attention(C.c_void_p(16), ins)
        return lib.oc_last_error()

    assert b"descriptor" in call(None)
    assert b"num_blocks -1" in call(Desc(1, 512, 64, 512, -1))
    assert b"seq_len_k 500" in call(Desc(1, 500, 64, 512, 1))
    before = lib.oc_last_error()
    call(Desc(0, 512, 64, 512, 1))
    assert lib.oc_last_error() == before
