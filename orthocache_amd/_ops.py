"""Thin wrappers: torch tensors -> liborthocache_hip.so calls.

Every function launches HIP kernels on the tensors' device, on torch's
current stream, and returns device tensors.  No host synchronisation
happens here.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import _native as N
from ._native import BLOCK, check, dtype_code, lib, ptr, require_gpu, stream_ptr


def _kv_view(t: torch.Tensor, name: str) -> torch.Tensor:
    """(S, H, D) with unit dim stride and 16-byte aligned rows, else a copy."""
    if t.dim() != 3:
        raise ValueError(f"{name} must be (seq, heads, head_dim), got shape {tuple(t.shape)}")
    es = t.element_size()
    ok = (t.stride(2) == 1 and t.data_ptr() % 16 == 0 and (t.stride(0) * es) % 16 == 0
          and (t.stride(1) * es) % 16 == 0)
    return t if ok else t.contiguous()


def _q_view(t: torch.Tensor, kv_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Queries with unit dim stride and 16-byte aligned rows; with kv_dtype, in
    the kv dtype or fp32 (the attention kernel reads one of the two)."""
    if kv_dtype is not None and t.dtype not in (kv_dtype, torch.float32):
        t = t.float()
    es = t.element_size()
    ok = t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((t.stride(i) * es) % 16 == 0
                                                             for i in range(t.dim() - 1) if t.shape[i] > 1)
    return t if ok else t.clone(memory_format=torch.contiguous_format)


def kv_group(q_heads: int, kv_heads: int) -> int:
    if q_heads % kv_heads:
        raise ValueError(f"query heads ({q_heads}) must be a multiple of kv heads ({kv_heads})")
    return q_heads // kv_heads


# ------------------------------------------------------------------- FWHT
def fwht_rows(x: torch.Tensor, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """FWHT along dim -2 of a (batch, 512, ncols) tensor (columns contiguous)."""
    require_gpu(x)
    if x.dim() != 3 or x.shape[1] != BLOCK:
        raise ValueError("fwht_rows expects (batch, 512, ncols)")
    if x.stride(2) != 1:
        x = x.contiguous()
    y = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
    a = N.FwhtArgs(ptr(x), dtype_code(x.dtype), x.stride(0), x.stride(1),
                   ptr(y), dtype_code(y.dtype), y.stride(0), y.stride(1), x.shape[2], x.shape[0])
    check(lib().oc_fwht512(C.byref(a), stream_ptr(x.device)), "oc_fwht512")
    return y


def band_energy(spec: torch.Tensor, s0: int, s1: int) -> torch.Tensor:
    """sum_{s in [s0,s1)} sum_d spec[b, s, h, d]^2 for a (nb, 512, H, D) fp32 spectrum."""
    spec = spec.contiguous()
    nb, _, h, d = spec.shape
    out = torch.empty((nb, h), dtype=torch.float32, device=spec.device)
    check(lib().oc_band_energy(ptr(spec), nb, h, d, s0, s1, ptr(out), stream_ptr(spec.device)),
          "oc_band_energy")
    return out


def block_energy(keys: torch.Tensor, block_size: int) -> torch.Tensor:
    require_gpu(keys)
    keys = _kv_view(keys, "keys")
    s, h, d = keys.shape
    nb = s // block_size
    out = torch.empty((nb, h), dtype=torch.float32, device=keys.device)
    check(lib().oc_block_energy(ptr(keys), dtype_code(keys.dtype), keys.stride(0), keys.stride(1), d, h,
                                nb, block_size, ptr(out), stream_ptr(keys.device)), "oc_block_energy")
    return out


# ----------------------------------------------------------------- scores
@dataclass
class Scores:
    tau_max: torch.Tensor | None   # (P, nb, Hkv) partial maxima over query tiles
    zeta: torch.Tensor | None      # (nb, Hkv)
    dc: torch.Tensor | None = None
    e_low: torch.Tensor | None = None
    e_mid: torch.Tensor | None = None
    e_high: torch.Tensor | None = None
    e_ac: torch.Tensor | None = None
    bounds: torch.Tensor | None = None  # (Sq*G, nb, Hkv)
    logits: torch.Tensor | None = None  # (nb, Hkv, 512, nq_pad): q.k * log2(e)/sqrt(d)
    mask: torch.Tensor | None = None    # (nb, Hkv) bool: the two-gate mask


INLINE_QUERY_LIMIT = 16
LOGITS_QUERY_LIMIT = 4  # query rows per kv head for scoring-pass logits


def logits_nq_pad(nq: int) -> int:
    """Query slots per key row in the scoring-pass logits (1, 2 or 4)."""
    return 1 if nq <= 1 else (2 if nq <= 2 else 4)


MASK_LIST_MAX_BLOCKS = 2048  # blocks of one segment whose attention can take a mask


def layer_uses_keep(num_blocks: int, single_segment: bool) -> bool:
    """Whether oc_decode_layer has its scoring pass write the two-gate mask
    and the attention derive the list from it (the library's
    layer_uses_keep): one segment of 1..2048 blocks."""
    return single_segment and 1 <= num_blocks <= MASK_LIST_MAX_BLOCKS


def _set_thresholds(a, tau, zeta_max, device):
    """tau / zeta_max (Python floats, rounded to fp32, or per-segment device
    tensors) into an argument struct; returns tensors to keep alive."""
    keep = []
    if isinstance(tau, torch.Tensor):
        t = tau.to(device=device, dtype=torch.float32).contiguous()
        a.tau_arr = ptr(t); keep.append(t)
    else:
        a.tau = float(tau)
    if isinstance(zeta_max, torch.Tensor):
        z = zeta_max.to(device=device, dtype=torch.float32).contiguous()
        a.zeta_max_arr = ptr(z); keep.append(z)
    else:
        a.zeta_max = float(zeta_max)
    return keep


def layer_uses_logits(kv_dtype: torch.dtype, head_dim: int, nq: int,
                      q_dtype: torch.dtype = torch.bfloat16) -> bool:
    """Whether oc_decode_layer forms the logits in its scoring pass (the
    library's layer_uses_logits): 1..4 query rows per kv head and at most 64
    lanes of 16 bytes per key row, except fp16 keys with one row at head_dim
    256 or with fp32 queries and 3-4 rows at head_dim 128, where the layer is
    faster with the attention reading the keys."""
    if kv_dtype == torch.float16 and ((head_dim == 256 and nq == 1) or
                                      (q_dtype == torch.float32 and head_dim == 128 and nq > 2)):
        return False
    lanes = head_dim * torch.empty((), dtype=kv_dtype).element_size() // 16
    return 1 <= nq <= LOGITS_QUERY_LIMIT and lanes <= 64


def score(keys: torch.Tensor, q: torch.Tensor | None = None, *, want_bands: bool = False,
          want_bounds: bool = False, want_zeta: bool = True, cu_blocks: torch.Tensor | None = None,
          num_segments: int = 1, pages: torch.Tensor | None = None, want_logits: bool = False,
          gate=None) -> Scores:
    """One pass over the keys: zeta, bands and (with q) the query-aware bound.

    keys: (S, Hkv, D), S a multiple of 512.  q: (Sq, Hq, D) for one segment or
    (B, Sq, Hq, D) with cu_blocks for several.  Small query counts get their
    maximum bound inline; large ones (or want_bounds) go through the tiled
    bound kernel.  want_logits (at most 4 query rows per kv head): also the
    attention logits of every key row, formed in the same pass.  gate =
    (tau, zeta_max): also the two-gate mask from the same scores (inline
    bound only).
    """
    require_gpu(keys, q, cu_blocks)
    keys = _kv_view(keys, "keys")
    s, hkv, d = keys.shape
    if s % BLOCK:
        raise ValueError(f"seq_len {s} is not a multiple of the block size {BLOCK}")
    nb = s // BLOCK
    pages = _pages_view(pages, keys)
    if pages is not None:
        nb = pages.shape[0]  # logical blocks; keys is the page pool
    dev = keys.device
    f32 = dict(dtype=torch.float32, device=dev)
    tiles = (nb, hkv)
    zeta = torch.empty(tiles, **f32) if want_zeta else None
    res = Scores(tau_max=None, zeta=zeta)
    sq = group = 0
    q_ok = q is not None
    if q_ok:
        q = _q_view(q, keys.dtype)
        if cu_blocks is None:
            if q.dim() != 3:
                raise ValueError("q must be (seq_q, heads, head_dim)")
            sq, hq, qd = q.shape
            qseg = 0
        else:
            if q.dim() != 4:
                raise ValueError("with cu_blocks, q must be (segments, seq_q, heads, head_dim)")
            _, sq, hq, qd = q.shape
            qseg = q.stride(0)
        if qd != d:
            raise ValueError(f"q head_dim {qd} != keys head_dim {d}")
        group = kv_group(hq, hkv)
    nq = sq * group
    inline = q_ok and not want_bounds and nq <= INLINE_QUERY_LIMIT
    need_dc = want_bands or (q_ok and not inline)
    if want_bands or need_dc:
        res.dc = torch.empty((nb, hkv, d), **f32)
        res.e_ac = torch.empty(tiles, **f32)
    if want_bands:
        res.e_low = torch.empty(tiles, **f32)
        res.e_mid = torch.empty(tiles, **f32)
        res.e_high = torch.empty(tiles, **f32)
    if inline:
        res.tau_max = torch.empty((1,) + tiles, **f32)
    if want_logits:
        if not (inline and 1 <= nq <= LOGITS_QUERY_LIMIT):
            raise ValueError(f"logits need 1..{LOGITS_QUERY_LIMIT} query rows per kv head, got {nq}")
        res.logits = torch.empty((nb, hkv, BLOCK, logits_nq_pad(nq)), **f32)
    if gate is not None and not inline:
        raise ValueError("the two-gate mask from the scoring pass needs the inline bound (at most 16 query rows)")
    a = N.ScoreArgs()
    a.keys = ptr(keys); a.keys_dtype = dtype_code(keys.dtype)
    a.keys_tok_stride = keys.stride(0); a.keys_head_stride = keys.stride(1)
    a.head_dim = d; a.num_kv_heads = hkv; a.total_blocks = nb
    a.cu_blocks = ptr(cu_blocks); a.num_segments = num_segments
    a.pages = ptr(pages)
    a.num_pages = s // BLOCK
    if inline:
        a.q = ptr(q); a.q_dtype = dtype_code(q.dtype)
        a.q_seg_stride = q.stride(0) if cu_blocks is not None else 0
        a.q_tok_stride = q.stride(-3); a.q_head_stride = q.stride(-2)
        a.sq = sq; a.group = group
        a.tau_max = ptr(res.tau_max)
    a.zeta = ptr(res.zeta); a.dc = ptr(res.dc); a.e_low = ptr(res.e_low); a.e_mid = ptr(res.e_mid)
    a.e_high = ptr(res.e_high); a.e_ac = ptr(res.e_ac)
    a.logits = ptr(res.logits)
    alive = []
    if gate is not None:
        res.mask = torch.empty(tiles, dtype=torch.uint8, device=dev)
        a.mask = ptr(res.mask)
        alive = _set_thresholds(a, gate[0], gate[1], dev)
    check(lib().oc_score_blocks(C.byref(a), stream_ptr(dev)), "oc_score_blocks")
    del alive
    if res.mask is not None:
        res.mask = res.mask.view(torch.bool)
    if q_ok and not inline:
        if cu_blocks is not None:
            raise ValueError("many-query bounds need a single segment")
        ntiles = int(lib().oc_query_bound_tiles(sq, group))
        res.tau_max = torch.empty((ntiles,) + tiles, **f32)
        if want_bounds:
            res.bounds = torch.empty((nq, nb, hkv), **f32)
        b = N.BoundArgs(ptr(res.dc), ptr(res.e_ac), ptr(q), dtype_code(q.dtype), q.stride(0), q.stride(1),
                        sq, group, d, hkv, nb, ptr(res.bounds), ptr(res.tau_max))
        check(lib().oc_query_bounds(C.byref(b), stream_ptr(dev)), "oc_query_bounds")
    return res


def _pages_view(pages, pool: torch.Tensor, block_size: int = BLOCK):
    """Validate a page list (int32, one physical page of ``pool`` per logical
    block) or pass None through."""
    if pages is None:
        return None
    if not isinstance(pages, torch.Tensor) or pages.dim() != 1 or pages.dtype != torch.int32:
        raise ValueError("pages must be a 1-D int32 tensor (one physical page per logical block)")
    if pages.device != pool.device:
        raise ValueError("pages must be on the keys' device")
    if pool.shape[0] % block_size:
        raise ValueError(f"the page pool's token count {pool.shape[0]} is not a multiple of {block_size}")
    return pages.contiguous()


# ------------------------------------------------------ mask + compaction
@dataclass
class Compacted:
    mask: torch.Tensor | None          # (nb, Hkv) bool
    active: torch.Tensor | None        # (nb,) bool
    indices: torch.Tensor | None       # (nb,) int32 permutation
    num_active: torch.Tensor | None    # (segments,) int32
    head_indices: torch.Tensor | None = None     # (Hkv, nb) int32
    head_num_active: torch.Tensor | None = None  # (segments, Hkv) int32
    head_uniform: torch.Tensor | None = None     # (segments, Hkv) int32


def mask_compact(*, num_blocks: int, num_kv_heads: int, device: torch.device,
                 tau_max: torch.Tensor | None = None, zeta: torch.Tensor | None = None,
                 tau=None, zeta_max=None, mask_in: torch.Tensor | None = None,
                 want_mask: bool = False, want_active: bool = False, want_indices: bool = True,
                 want_head_lists: bool = False, empty_head_all: bool = False,
                 cu_blocks: torch.Tensor | None = None, num_segments: int = 1) -> Compacted:
    """Two-gate mask (or a given mask) -> masks, permutation and counts, on device.

    tau / zeta_max: Python floats (rounded to fp32 as JAX does) or per-segment
    fp32 device tensors.  A gate whose input is None is off.
    """
    nb, hkv = num_blocks, num_kv_heads
    a = N.CompactArgs()
    if mask_in is not None:
        if mask_in.dtype != torch.bool:
            mask_in = mask_in != 0
        m = mask_in.contiguous().view(torch.uint8)
        if m.dim() == 1:
            heads_in = 1
        elif m.dim() == 2 and m.shape[1] in (1, hkv):
            heads_in = m.shape[1]
        else:
            raise ValueError(f"block_mask must be (num_blocks,) or (num_blocks, {hkv}), got {tuple(m.shape)}")
        if m.shape[0] != nb:
            raise ValueError(f"block_mask has {m.shape[0]} blocks, expected {nb}")
        a.mask_in = ptr(m); a.mask_in_heads = heads_in
    else:
        if tau_max is None:
            raise ValueError("need scores or a mask")
        tau_max = tau_max.contiguous()
        a.tau_max = ptr(tau_max); a.tau_parts = tau_max.shape[0] if tau_max.dim() == 3 else 1
        if zeta is not None:
            zeta = zeta.contiguous()
            a.zeta = ptr(zeta)
        if isinstance(tau, torch.Tensor):
            tau = tau.to(device=device, dtype=torch.float32).contiguous()
            a.tau_arr = ptr(tau)
        else:
            a.tau = float(tau)
        if zeta is not None:
            if isinstance(zeta_max, torch.Tensor):
                zeta_max = zeta_max.to(device=device, dtype=torch.float32).contiguous()
                a.zeta_max_arr = ptr(zeta_max)
            else:
                a.zeta_max = float(zeta_max)
    a.cu_blocks = ptr(cu_blocks); a.num_segments = num_segments
    a.num_kv_heads = hkv; a.total_blocks = nb
    u8 = dict(dtype=torch.uint8, device=device)
    i32 = dict(dtype=torch.int32, device=device)
    res = Compacted(None, None, None, None)
    if want_mask:
        res.mask = torch.empty((nb, hkv), **u8)
        a.mask_out = ptr(res.mask)
    if want_active:
        res.active = torch.empty((nb,), **u8)
        a.active_out = ptr(res.active)
    if want_indices:
        res.indices = torch.empty((nb,), **i32)
        res.num_active = torch.empty((num_segments,), **i32)
        a.indices = ptr(res.indices); a.num_active = ptr(res.num_active)
    if want_head_lists:
        res.head_indices = torch.empty((hkv, nb), **i32)
        res.head_num_active = torch.empty((num_segments, hkv), **i32)
        res.head_uniform = torch.empty((num_segments, hkv), **i32)
        a.head_indices = ptr(res.head_indices); a.head_num_active = ptr(res.head_num_active)
        a.head_uniform = ptr(res.head_uniform); a.empty_head_all = 1 if empty_head_all else 0
    check(lib().oc_mask_compact(C.byref(a), stream_ptr(device)), "oc_mask_compact")
    if res.mask is not None:
        res.mask = res.mask.view(torch.bool)
    if res.active is not None:
        res.active = res.active.view(torch.bool)
    return res


def copy_blocks(src: torch.Tensor, dst: torch.Tensor, indices: torch.Tensor, num_active: torch.Tensor,
                num_blocks: int, scatter: bool) -> None:
    block_bytes = src.numel() * src.element_size() // max(1, src.shape[0])
    check(lib().oc_copy_blocks(ptr(src), ptr(dst), ptr(indices), ptr(num_active), num_blocks, block_bytes,
                               1 if scatter else 0, stream_ptr(src.device)), "oc_copy_blocks")


# --------------------------------------------------------------- attention
def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, indices: torch.Tensor, counts: torch.Tensor, *,
           block_size: int = BLOCK, per_head: bool = False, uniform: torch.Tensor | None = None,
           out_dtype: torch.dtype | None = None, cu_blocks: torch.Tensor | None = None,
           num_segments: int = 1, out: torch.Tensor | None = None, pages: torch.Tensor | None = None,
           logits: torch.Tensor | None = None, mask: torch.Tensor | None = None,
           indices_out: torch.Tensor | None = None, num_active_out: torch.Tensor | None = None) -> torch.Tensor:
    """Attention over the listed blocks.  q: (Sq, Hq, D) (or (B, Sq, Hq, D) with
    cu_blocks); k, v: (S, Hkv, D).  Returns q-shaped output in out_dtype.
    logits: the ``score(..., want_logits=True)`` logits of the same q and keys;
    the keys are then not read.  mask: a (nb, Hkv) block mask of one segment
    instead of indices/counts (pass None for those); the kernel takes the
    blocks any head keeps and writes the active-first permutation and the
    count into indices_out / num_active_out when given."""
    a, out, q = _attend_args(q, k, v, indices, counts, block_size=block_size, per_head=per_head, uniform=uniform,
                             out_dtype=out_dtype, cu_blocks=cu_blocks, num_segments=num_segments, out=out,
                             pages=pages)
    if mask is not None:
        if mask.dim() != 2 or mask.shape != (a.total_blocks, a.num_kv_heads):
            raise ValueError(f"mask must be (num_blocks, kv_heads) = ({a.total_blocks}, {a.num_kv_heads})")
        mask = (mask if mask.dtype == torch.bool else mask != 0).contiguous().view(torch.uint8)
        if indices_out is None:
            indices_out = torch.empty((a.total_blocks,), dtype=torch.int32, device=q.device)
        if num_active_out is None:
            num_active_out = torch.empty((1,), dtype=torch.int32, device=q.device)
        a.mask = ptr(mask); a.indices_out = ptr(indices_out); a.num_active_out = ptr(num_active_out)
    if logits is not None:
        if logits.dtype != torch.float32 or not logits.is_contiguous() or logits.shape[:3] != (a.total_blocks, a.num_kv_heads, BLOCK):
            raise ValueError("logits must be the contiguous fp32 (blocks, kv_heads, 512, nq_pad) output of score()")
        a.logits = ptr(logits)
    L = lib()
    ws_bytes = int(L.oc_attend_workspace_size(C.byref(a)))
    if ws_bytes == 0 and a.total_blocks > 0:
        # Size query failed validation: surface the message.
        check(L.oc_attend(C.byref(a), None, 0, stream_ptr(q.device)), "oc_attend")
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
    check(L.oc_attend(C.byref(a), ptr(ws), ws_bytes, stream_ptr(q.device)), "oc_attend")
    return out


def attend_plan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, indices: torch.Tensor, counts: torch.Tensor,
                **kw) -> tuple[str, int]:
    """Kernel family ``attend`` would use for these arguments ("decode" or
    "prefill_mfma") and the prefill split count (0 for decode)."""
    a, _, _ = _attend_args(q, k, v, indices, counts, **kw)
    kern, nsplit = C.c_int32(), C.c_int32()
    check(lib().oc_attend_plan(C.byref(a), C.byref(kern), C.byref(nsplit)), "oc_attend_plan")
    return ("prefill_mfma" if kern.value == 1 else "decode"), int(nsplit.value)


def _attend_args(q, k, v, indices, counts, *, block_size: int = BLOCK, per_head: bool = False,
                 uniform=None, out_dtype=None, cu_blocks=None, num_segments: int = 1, out=None, pages=None):
    require_gpu(q, k, v, indices, counts)
    if indices is None and counts is None:
        pass  # a block mask replaces the list (attend(..., mask=...))
    elif indices is None or counts is None:
        raise ValueError("indices and counts go together")
    out_dtype = out_dtype or q.dtype
    k = _kv_view(k, "keys")
    v = _kv_view(v, "values")
    q = _q_view(q, k.dtype)
    s, hkv, d = k.shape
    if v.shape != k.shape:
        raise ValueError(f"values shape {tuple(v.shape)} != keys shape {tuple(k.shape)}")
    if s % block_size:
        raise ValueError(f"seq_len {s} is not a multiple of block_size {block_size}")
    if q.shape[-1] != d:
        raise ValueError(f"q head_dim {q.shape[-1]} != keys head_dim {d}")
    group = kv_group(q.shape[-2], hkv)
    sq = q.shape[-3]
    if out is None:
        out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
    a = N.AttendArgs()
    a.q = ptr(q); a.q_dtype = dtype_code(q.dtype)
    a.q_seg_stride = q.stride(0) if q.dim() == 4 else 0
    a.q_tok_stride = q.stride(-3); a.q_head_stride = q.stride(-2)
    a.k = ptr(k); a.v = ptr(v); a.kv_dtype = dtype_code(k.dtype)
    if v.dtype != k.dtype:
        raise ValueError("keys and values must share a dtype")
    a.k_tok_stride = k.stride(0); a.k_head_stride = k.stride(1)
    a.v_tok_stride = v.stride(0); a.v_head_stride = v.stride(1)
    a.head_dim = d; a.num_kv_heads = hkv; a.group = group; a.sq = sq
    a.block_size = block_size; a.total_blocks = s // block_size
    pages = _pages_view(pages, k, block_size)
    if pages is not None:
        a.total_blocks = pages.shape[0]
        a.pages = ptr(pages)
        a.num_pages = s // block_size
    a.cu_blocks = ptr(cu_blocks); a.num_segments = num_segments
    a.indices = ptr(indices); a.counts = ptr(counts); a.per_head = 1 if per_head else 0
    a.uniform = ptr(uniform)
    a.out = ptr(out); a.out_dtype = dtype_code(out.dtype)
    a.out_seg_stride = out.stride(0) if out.dim() == 4 else 0
    a.out_tok_stride = out.stride(-3); a.out_head_stride = out.stride(-2)
    return a, out, q


# ------------------------------------------------------------- one layer
class DecodeLayer:
    """Pre-bound score -> compact -> attend for fixed shapes (reusable workspace).

    keys/values (S, Hkv, D) packed over segments; q (B, Sq, Hq, D) when
    cu_blocks is given, else (Sq, Hq, D).  Call ``run()`` to launch the three
    kernels on the current stream.
    """

    def __init__(self, q, k, v, tau, zeta_max, *, cu_blocks=None, num_segments=1, out=None,
                 out_dtype=None, keep_scores=True, pages=None):
        require_gpu(q, k, v, cu_blocks, pages)
        self.k = _kv_view(k, "keys")
        self.v = _kv_view(v, "values")
        self.q = _q_view(q, self.k.dtype)
        s, hkv, d = self.k.shape
        if s % BLOCK:
            raise ValueError(f"seq_len {s} is not a multiple of {BLOCK}")
        nb = s // BLOCK
        self.pages = _pages_view(pages, self.k)
        if self.pages is not None:
            nb = self.pages.shape[0]
        dev = self.k.device
        self.device = dev
        group = kv_group(self.q.shape[-2], hkv)
        self.out = out if out is not None else torch.empty(self.q.shape, dtype=out_dtype or q.dtype, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.tau_max = torch.empty((nb, hkv), **f32) if keep_scores else None
        self.zeta = torch.empty((nb, hkv), **f32) if keep_scores else None
        self.indices = torch.empty((nb,), dtype=torch.int32, device=dev)
        self.num_active = torch.empty((num_segments,), dtype=torch.int32, device=dev)
        a = N.LayerArgs()
        q_ = self.q
        a.q = ptr(q_); a.q_dtype = dtype_code(q_.dtype)
        a.q_seg_stride = q_.stride(0) if q_.dim() == 4 else 0
        a.q_tok_stride = q_.stride(-3); a.q_head_stride = q_.stride(-2)
        a.k = ptr(self.k); a.v = ptr(self.v); a.kv_dtype = dtype_code(self.k.dtype)
        a.k_tok_stride = self.k.stride(0); a.k_head_stride = self.k.stride(1)
        a.v_tok_stride = self.v.stride(0); a.v_head_stride = self.v.stride(1)
        a.head_dim = d; a.num_kv_heads = hkv; a.group = group; a.sq = q_.shape[-3]
        a.total_blocks = nb; a.cu_blocks = ptr(cu_blocks); a.num_segments = num_segments
        a.pages = ptr(self.pages)
        a.num_pages = s // BLOCK
        self._tau_t = self._zmax_t = None
        if isinstance(tau, torch.Tensor):
            self._tau_t = tau.to(device=dev, dtype=torch.float32).contiguous()
            a.tau_arr = ptr(self._tau_t)
        else:
            a.tau = float(tau)
        if isinstance(zeta_max, torch.Tensor):
            self._zmax_t = zeta_max.to(device=dev, dtype=torch.float32).contiguous()
            a.zeta_max_arr = ptr(self._zmax_t)
        else:
            a.zeta_max = float(zeta_max)
        a.out = ptr(self.out); a.out_dtype = dtype_code(self.out.dtype)
        o = self.out
        a.out_seg_stride = o.stride(0) if o.dim() == 4 else 0
        a.out_tok_stride = o.stride(-3); a.out_head_stride = o.stride(-2)
        a.tau_max = ptr(self.tau_max); a.zeta = ptr(self.zeta)
        a.indices = ptr(self.indices); a.num_active = ptr(self.num_active)
        self.cu_blocks = cu_blocks
        self.args = a
        L = lib()
        ws = int(L.oc_decode_layer_workspace_size(C.byref(a)))
        if ws == 0:
            check(L.oc_decode_layer(C.byref(a), None, 0, 0), "oc_decode_layer")
        self.workspace = torch.empty((ws,), dtype=torch.uint8, device=dev)
        self._ws_ptr = ptr(self.workspace)
        self._ws_bytes = ws
        self._fn = L.oc_decode_layer
        self._argp = C.byref(a)

    def run(self, stream: int | None = None) -> torch.Tensor:
        s = stream_ptr(self.device) if stream is None else stream
        check(self._fn(self._argp, self._ws_ptr, self._ws_bytes, s), "oc_decode_layer")
        return self.out

    def capture(self) -> "torch.cuda.CUDAGraph":
        """A HIP graph of one run(): ``replay()`` launches the whole layer with
        one host call (for launch-bound decode loops).  The graph holds only
        the layer's kernels (no memset or copy nodes) and the bound buffers:
        update q, the caches and thresholds in place between replays."""
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self.run()  # first launch outside the capture
        torch.cuda.current_stream(self.device).wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.run()
        return g

    def phases(self):
        """Callables (score, compact, attend) launching the layer's phases one
        at a time on the current stream, with the kernels run() uses (for
        per-kernel timing).  compact is None when the layer has no compaction
        launch (one segment: the scoring pass writes the mask and the
        attention derives the list from it)."""
        a = self.args
        L = lib()
        sa = N.ScoreArgs()
        sa.keys = a.k; sa.keys_dtype = a.kv_dtype; sa.keys_tok_stride = a.k_tok_stride
        sa.keys_head_stride = a.k_head_stride; sa.head_dim = a.head_dim; sa.num_kv_heads = a.num_kv_heads
        sa.total_blocks = a.total_blocks; sa.cu_blocks = a.cu_blocks; sa.num_segments = a.num_segments
        sa.q = a.q; sa.q_dtype = a.q_dtype; sa.q_seg_stride = a.q_seg_stride; sa.q_tok_stride = a.q_tok_stride
        sa.q_head_stride = a.q_head_stride; sa.sq = a.sq; sa.group = a.group
        sa.tau_max = a.tau_max; sa.zeta = a.zeta; sa.pages = a.pages; sa.num_pages = a.num_pages
        ca = N.CompactArgs()
        ca.tau_max = a.tau_max; ca.tau_parts = 1; ca.zeta = a.zeta
        ca.tau_arr = a.tau_arr; ca.tau = a.tau; ca.zeta_max_arr = a.zeta_max_arr; ca.zeta_max = a.zeta_max
        ca.cu_blocks = a.cu_blocks; ca.num_segments = a.num_segments
        ca.num_kv_heads = a.num_kv_heads; ca.total_blocks = a.total_blocks
        ca.indices = a.indices; ca.num_active = a.num_active
        ta = N.AttendArgs()
        for f in ("q", "q_dtype", "q_seg_stride", "q_tok_stride", "q_head_stride", "k", "v", "kv_dtype",
                  "k_tok_stride", "k_head_stride", "v_tok_stride", "v_head_stride", "head_dim", "num_kv_heads",
                  "group", "sq", "total_blocks", "cu_blocks", "num_segments", "out", "out_dtype",
                  "out_seg_stride", "out_tok_stride", "out_head_stride", "pages", "num_pages"):
            setattr(ta, f, getattr(a, f))
        ta.block_size = BLOCK; ta.indices = a.indices; ta.counts = a.num_active
        # The fused layer forms the attention logits in its scoring pass when
        # it can; the phases do the same, so each phase times the layer's kernel.
        self._phase_logits = None
        if layer_uses_logits(self.k.dtype, a.head_dim, a.sq * a.group, self.q.dtype):
            self._phase_logits = torch.empty((a.total_blocks, a.num_kv_heads, BLOCK, logits_nq_pad(a.sq * a.group)),
                                             dtype=torch.float32, device=self.device)
            sa.logits = ptr(self._phase_logits)
            ta.logits = ptr(self._phase_logits)
        keep = layer_uses_keep(a.total_blocks, self.cu_blocks is None)
        if keep:
            self._phase_keep = torch.empty((a.total_blocks, a.num_kv_heads), dtype=torch.uint8, device=self.device)
            sa.mask = ptr(self._phase_keep)
            sa.tau_arr = a.tau_arr; sa.tau = a.tau; sa.zeta_max_arr = a.zeta_max_arr; sa.zeta_max = a.zeta_max
            ta.mask = ptr(self._phase_keep)
            ta.indices = None; ta.counts = None
            ta.indices_out = a.indices; ta.num_active_out = a.num_active
        ws = int(L.oc_attend_workspace_size(C.byref(ta)))
        self._phase_ws = torch.empty((max(ws, 1),), dtype=torch.uint8, device=self.device)
        self._phase_args = (sa, ca, ta)
        dev = self.device
        wsp = ptr(self._phase_ws)

        def score():
            check(L.oc_score_blocks(C.byref(sa), stream_ptr(dev)), "oc_score_blocks")

        def compact():
            check(L.oc_mask_compact(C.byref(ca), stream_ptr(dev)), "oc_mask_compact")

        def attend():
            check(L.oc_attend(C.byref(ta), wsp, ws, stream_ptr(dev)), "oc_attend")

        return score, (None if keep else compact), attend


class PrefillLayer:
    """Pre-bound score -> query bounds -> compact -> attend for one chunk of
    many queries on one segment (chunked prefill), fixed shapes and buffers.

    q (Sq, Hq, D); keys/values (S, Hkv, D).  The bound of every query goes
    through the tiled bound kernel; with bf16/fp16 inputs and head_dim 64 or
    128 the attention runs on the matrix-core prefill kernels.  ``run()``
    launches the four calls on the current stream without host
    synchronisation; ``phases()`` returns them one at a time.
    """

    def __init__(self, q, k, v, tau, zeta_max, *, out=None, out_dtype=None):
        require_gpu(q, k, v)
        self.k = _kv_view(k, "keys")
        self.v = _kv_view(v, "values")
        self.q = _q_view(q, self.k.dtype)
        if self.q.dim() != 3:
            raise ValueError("q must be (seq_q, heads, head_dim)")
        s, hkv, d = self.k.shape
        if s % BLOCK:
            raise ValueError(f"seq_len {s} is not a multiple of {BLOCK}")
        nb = s // BLOCK
        sq, hq, qd = self.q.shape
        if qd != d:
            raise ValueError(f"q head_dim {qd} != keys head_dim {d}")
        group = kv_group(hq, hkv)
        dev = self.k.device
        self.device = dev
        L = lib()
        f32 = dict(dtype=torch.float32, device=dev)
        self.zeta = torch.empty((nb, hkv), **f32)
        self.dc = torch.empty((nb, hkv, d), **f32)
        self.e_ac = torch.empty((nb, hkv), **f32)
        ntiles = int(L.oc_query_bound_tiles(sq, group))
        self.tau_max = torch.empty((ntiles, nb, hkv), **f32)
        self.indices = torch.empty((nb,), dtype=torch.int32, device=dev)
        self.num_active = torch.empty((1,), dtype=torch.int32, device=dev)
        self.out = out if out is not None else torch.empty(self.q.shape, dtype=out_dtype or q.dtype, device=dev)

        sa = N.ScoreArgs()
        sa.keys = ptr(self.k); sa.keys_dtype = dtype_code(self.k.dtype)
        sa.keys_tok_stride = self.k.stride(0); sa.keys_head_stride = self.k.stride(1)
        sa.head_dim = d; sa.num_kv_heads = hkv; sa.total_blocks = nb; sa.num_segments = 1
        sa.zeta = ptr(self.zeta); sa.dc = ptr(self.dc); sa.e_ac = ptr(self.e_ac)
        ba = N.BoundArgs(ptr(self.dc), ptr(self.e_ac), ptr(self.q), dtype_code(self.q.dtype), self.q.stride(0),
                         self.q.stride(1), sq, group, d, hkv, nb, None, ptr(self.tau_max))
        ca = N.CompactArgs()
        ca.tau_max = ptr(self.tau_max); ca.tau_parts = ntiles; ca.zeta = ptr(self.zeta)
        ca.tau = float(tau); ca.zeta_max = float(zeta_max)
        ca.num_segments = 1; ca.num_kv_heads = hkv; ca.total_blocks = nb
        ca.indices = ptr(self.indices); ca.num_active = ptr(self.num_active)
        ta, _, _ = _attend_args(self.q, self.k, self.v, self.indices, self.num_active, out=self.out)
        ws = int(L.oc_attend_workspace_size(C.byref(ta)))
        if ws == 0:
            check(L.oc_attend(C.byref(ta), None, 0, stream_ptr(dev)), "oc_attend")
        self.workspace = torch.empty((ws,), dtype=torch.uint8, device=dev)
        self.args = (sa, ba, ca, ta)
        wsp = ptr(self.workspace)

        def score():
            check(L.oc_score_blocks(C.byref(sa), stream_ptr(dev)), "oc_score_blocks")

        def bounds():
            check(L.oc_query_bounds(C.byref(ba), stream_ptr(dev)), "oc_query_bounds")

        def compact():
            check(L.oc_mask_compact(C.byref(ca), stream_ptr(dev)), "oc_mask_compact")

        def attend():
            check(L.oc_attend(C.byref(ta), wsp, ws, stream_ptr(dev)), "oc_attend")

        self._phases = (score, bounds, compact, attend)

    def run(self) -> torch.Tensor:
        for f in self._phases:
            f()
        return self.out

    def phases(self):
        return self._phases
