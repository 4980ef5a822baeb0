"""Synthetic workloads of the benchmark configurations, generated on the GPU.

Seeded torch generators on the device; nothing is read from disk.
  c1: single-head decode, 1 query / 1 kv head, d=128, 8K tokens (16 blocks)
  c2: global-attention decode layer, 32 q / 16 kv heads, d=256, 64K tokens
  c3: ragged decode batch, 32 sequences of 4K-32K tokens, 32 q / 8 kv heads, d=128
  c4: chunked prefill, 512 queries x 128K keys, 8 heads, d=128
  c5: 60-layer scoring sweep (50 x 1K-token sliding + 10 x 64K global), 16 kv heads, d=256
Keys are N(0,1) plus a per-(block, head, dim) mean offset with std 0.5; a
fraction of blocks get an alternating-sign +-1 pattern added along the token
axis (the configs' "high-sequency noise"; in the natural Hadamard order it
lands on coefficient 1).  Queries are N(0,1)/sqrt(d).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from ._native import BLOCK


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def make_keys(nb: int, hkv: int, d: int, *, seed: int, device, dtype=torch.bfloat16, offset_std: float = 0.5,
              noise_frac: float = 0.1, noise_blocks: int | None = None, scale: float = 1.0) -> torch.Tensor:
    """(nb*512, hkv, d) keys: scale*N(0,1) + block offsets, some blocks noise-injected."""
    g = _gen(seed, device)
    k = torch.randn((nb, BLOCK, hkv, d), generator=g, device=device, dtype=torch.float32) * scale
    k += torch.randn((nb, 1, hkv, d), generator=g, device=device, dtype=torch.float32) * offset_std
    n_noise = noise_blocks if noise_blocks is not None else int(round(noise_frac * nb))
    if n_noise > 0:
        perm = torch.randperm(nb, generator=g, device=device)[:n_noise]
        sign = torch.ones(BLOCK, device=device)
        sign[1::2] = -1.0
        k[perm] += sign.reshape(1, BLOCK, 1, 1)
    return k.reshape(nb * BLOCK, hkv, d).to(dtype)


def make_values(s: int, hkv: int, d: int, *, seed: int, device, dtype=torch.bfloat16) -> torch.Tensor:
    g = _gen(seed, device)
    return torch.randn((s, hkv, d), generator=g, device=device, dtype=torch.float32).to(dtype)


def make_queries(shape, d: int, *, seed: int, device, dtype=torch.bfloat16) -> torch.Tensor:
    g = _gen(seed, device)
    return (torch.randn(tuple(shape), generator=g, device=device, dtype=torch.float32) / math.sqrt(d)).to(dtype)


def _f32(x: float) -> float:
    return float(torch.tensor(x, dtype=torch.float32))


def _between(lo: float, hi: float) -> float:
    """An fp32 threshold t with lo < t <= hi for fp32 values lo < hi: their
    midpoint rounded to fp32, or hi when no fp32 value lies strictly between."""
    t = _f32((lo + hi) / 2.0)
    return t if lo < t <= hi else hi


def calibrate_unified(tau_max: torch.Tensor, zeta: torch.Tensor, evict: float, zeta_quantile: float = 0.95):
    """(tau, zeta_max) so that the unified two-gate mask keeps round(nb*(1-evict)) blocks.

    zeta_max lies at the given quantile of zeta over (block, head), halfway
    between the two neighbouring fp32 values there; a block's unified score is
    the max tau_max over the heads that pass the zeta gate; tau lies halfway
    between the K-th and (K+1)-th largest unified scores, so the fp32 compare
    keeps exactly the top K when those differ, and no score sits on the
    threshold (a restatement that rounds a score differently in its last bits
    keeps the same blocks).  Host-synchronising; done once, outside any timed
    region.
    """
    nb = tau_max.shape[0]
    zs = torch.sort(zeta.flatten().float()).values
    i = min(int(zeta_quantile * (zs.numel() - 1)), zs.numel() - 1)
    j = i
    while j + 1 < zs.numel() and float(zs[j + 1]) == float(zs[i]):
        j += 1
    zmax = float(zs[i]) if j + 1 >= zs.numel() else _between(float(zs[i]), float(zs[j + 1]))
    ok = zeta <= zmax
    u = torch.where(ok, tau_max, torch.full_like(tau_max, -math.inf)).amax(dim=-1)
    keep = int(round(nb * (1.0 - evict)))
    if keep <= 0:
        return math.inf, zmax
    vals = torch.sort(u, descending=True).values.tolist()
    kth = vals[min(keep, nb) - 1]
    if keep >= nb or vals[keep] == -math.inf or vals[keep] == kth:
        return kth, zmax
    return _between(vals[keep], kth), zmax


def percentile(x: torch.Tensor, q: float) -> float:
    """numpy-style linear-interpolation percentile (q in [0, 100])."""
    return float(torch.quantile(x.flatten().double(), q / 100.0).item())


@dataclass
class Workload:
    name: str
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    tau: object = None
    zeta_max: object = None
    cu_seqlens: torch.Tensor | None = None
    meta: dict = field(default_factory=dict)


def c1(device, seed: int = 1) -> Workload:
    d, hkv, nb = 128, 1, 16
    k = make_keys(nb, hkv, d, seed=seed, device=device, noise_blocks=4)
    v = make_values(nb * BLOCK, hkv, d, seed=seed + 1, device=device)
    q = make_queries((1, 1, d), d, seed=seed + 2, device=device)
    return Workload("c1_decode_1x1_d128_8k", q, k, v, meta={"tau_pct": 50, "zeta_pct": 75})


def c2(device, seed: int = 2, seq: int = 65536) -> Workload:
    d, hkv, hq = 256, 16, 32
    nb = seq // BLOCK
    k = make_keys(nb, hkv, d, seed=seed, device=device, noise_frac=0.1)
    v = make_values(nb * BLOCK, hkv, d, seed=seed + 1, device=device)
    q = make_queries((1, hq, d), d, seed=seed + 2, device=device)
    return Workload(f"c2_gemma_global_decode_32q16kv_d256_{seq // 1024}k", q, k, v)


def c3(device, seed: int = 3, batch: int = 32, lo: int = 4096, hi: int = 32768) -> Workload:
    d, hkv, hq = 128, 8, 32
    g = torch.Generator()
    g.manual_seed(seed)
    lens = (torch.randint(lo // BLOCK, hi // BLOCK + 1, (batch,), generator=g) * BLOCK).tolist()
    evict = (0.30 + 0.65 * torch.rand((batch,), generator=g)).tolist()
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    nb = cu[-1] // BLOCK
    k = make_keys(nb, hkv, d, seed=seed + 1, device=device, noise_frac=0.1)
    v = make_values(nb * BLOCK, hkv, d, seed=seed + 2, device=device)
    q = make_queries((batch, 1, hq, d), d, seed=seed + 3, device=device)
    return Workload("c3_ragged_b32_32q8kv_d128", q, k, v,
                    cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=device),
                    meta={"lens": lens, "evict": evict})


def c4(device, seed: int = 4, queries: int = 512, seq: int = 131072) -> Workload:
    d, hkv, hq = 128, 8, 8
    nb = seq // BLOCK
    k = make_keys(nb, hkv, d, seed=seed, device=device, noise_frac=0.1)
    v = make_values(nb * BLOCK, hkv, d, seed=seed + 1, device=device)
    q = make_queries((queries, hq, d), d, seed=seed + 2, device=device)
    return Workload("c4_prefill_512x128k_8h_d128", q, k, v, meta={"evict": 0.75})


def c5(device, seed: int = 5, sliding_layers: int = 50, global_layers: int = 10, window: int = 1024,
       global_len: int = 65536) -> Workload:
    d, hkv, hq = 256, 16, 32
    g = torch.Generator()
    g.manual_seed(seed)
    lens = [window] * sliding_layers + [global_len] * global_layers
    var = (0.5 + 1.5 * torch.rand((len(lens),), generator=g)).tolist()
    parts = []
    cu = [0]
    for i, (n, vv) in enumerate(zip(lens, var)):
        parts.append(make_keys(n // BLOCK, hkv, d, seed=seed * 1000 + i, device=device, noise_frac=0.1,
                               scale=math.sqrt(vv)))
        cu.append(cu[-1] + n)
    k = torch.cat(parts, dim=0)
    del parts
    q = make_queries((len(lens), 1, hq, d), d, seed=seed + 7, device=device)
    return Workload("c5_sweep_60layers_16kv_d256", q, k, None,
                    cu_seqlens=torch.tensor(cu, dtype=torch.int32, device=device),
                    meta={"lens": lens, "var": var, "evict": 0.9})
