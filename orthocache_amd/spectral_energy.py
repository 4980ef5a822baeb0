"""Spectral block scoring on the GPU (reference: src/orthocache/spectral_energy.py).

Every function keeps the reference's name, arguments and output shapes.
Scores are computed in fp32 from one pass over the keys by the fused HIP
scoring kernel; the reference instead materialises the full 512-point
spectrum once per call (and twice in compute_multiband_mask).

Deviations, all documented: outputs are float32 whatever the key dtype (the
reference computes in the key dtype; its parity target is the fp32 path), and
q may carry G x the kv heads (GQA), in which case query head h*G+g scores
against kv head h and bounds are returned in the folded (Sq*G, nb, Hkv)
layout.
"""

from __future__ import annotations

import torch

from . import _ops
from ._native import BLOCK, require_gpu

# spectral_energy.py:15-18 - natural-index band boundaries.
BAND_DC = 0
BAND_LOW = (1, 64)
BAND_MID = (64, 256)
BAND_HIGH = (256, 512)

ZETA_EPS = 1e-6


def _check_keys(keys: torch.Tensor, block_size: int) -> None:
    require_gpu(keys)
    if keys.dim() != 3:
        raise ValueError(f"keys must be (seq_len, num_heads, head_dim), got {tuple(keys.shape)}")
    if block_size != BLOCK:
        raise ValueError(f"the FWHT scoring path needs block_size == 512, got {block_size}")
    if keys.shape[0] % block_size:
        raise ValueError(f"seq_len {keys.shape[0]} is not a multiple of block_size {block_size}")


def _is_default(band_low, band_mid, band_high) -> bool:
    return tuple(band_low) == BAND_LOW and tuple(band_mid) == BAND_MID and tuple(band_high) == BAND_HIGH


def compute_block_energy_jax(keys: torch.Tensor, block_size: int = 512) -> torch.Tensor:
    """Sum of squared keys per (block, head): ``spectral_energy.py:21-35``."""
    require_gpu(keys)
    if keys.dim() != 3:
        raise ValueError("keys must be (seq_len, num_heads, head_dim)")
    if keys.shape[0] % block_size:
        raise ValueError(f"seq_len {keys.shape[0]} is not a multiple of block_size {block_size}")
    return _ops.block_energy(keys, block_size)


def _run_fwht_on_blocks(keys: torch.Tensor, block_size: int = 512) -> torch.Tensor:
    """(S, H, D) -> WHT coefficients (nb, 512, H, D) fp32: ``spectral_energy.py:38-66``."""
    _check_keys(keys, block_size)
    s, h, d = keys.shape
    nb = s // block_size
    x = keys.reshape(nb, block_size, h * d)
    return _ops.fwht_rows(x, out_dtype=torch.float32).reshape(nb, block_size, h, d)


def compute_spectral_bands(keys: torch.Tensor, block_size: int = 512, band_low: tuple = BAND_LOW,
                           band_mid: tuple = BAND_MID, band_high: tuple = BAND_HIGH):
    """(dc (nb,H,D), low (nb,H), mid (nb,H), high (nb,H)): ``spectral_energy.py:69-106``."""
    _check_keys(keys, block_size)
    if _is_default(band_low, band_mid, band_high):
        sc = _ops.score(keys, want_bands=True, want_zeta=False)
        return sc.dc, sc.e_low, sc.e_mid, sc.e_high
    spec = _run_fwht_on_blocks(keys, block_size)
    dc = spec[:, BAND_DC].contiguous()
    return (dc, _ops.band_energy(spec, *band_low), _ops.band_energy(spec, *band_mid),
            _ops.band_energy(spec, *band_high))


def compute_spectral_decay_ratio(keys: torch.Tensor, block_size: int = 512, band_low: tuple = BAND_LOW,
                                 band_high: tuple = BAND_HIGH) -> torch.Tensor:
    """zeta = E_high / (E_low + 1e-6), (nb, H): ``spectral_energy.py:109-138``."""
    _check_keys(keys, block_size)
    if tuple(band_low) == BAND_LOW and tuple(band_high) == BAND_HIGH:
        return _ops.score(keys, want_zeta=True).zeta
    _, lo, _, hi = compute_spectral_bands(keys, block_size, band_low, (band_low[1], band_high[0]), band_high)
    return hi / (lo + ZETA_EPS)


def compute_query_aware_bounds(q: torch.Tensor, keys: torch.Tensor, block_size: int = 512) -> torch.Tensor:
    """Logit upper bounds (Sq, nb, H): ``spectral_energy.py:141-177``.

    tau_j(q) = q.kbar/sqrt(d) + ||q|| sqrt(E_AC)/sqrt(d).  With GQA
    (q heads = G x kv heads) the result is (Sq*G, nb, Hkv), query row t*G+g.
    """
    _check_keys(keys, block_size)
    require_gpu(q)
    if q.dim() != 3:
        raise ValueError("q must be (seq_len_q, num_heads, head_dim)")
    return _ops.score(keys, q, want_bounds=True, want_zeta=False).bounds


def _tau_max(q: torch.Tensor, keys: torch.Tensor, want_zeta: bool):
    sc = _ops.score(keys, q, want_zeta=want_zeta)
    return sc


def compute_query_aware_mask(q: torch.Tensor, keys: torch.Tensor, tau: float, block_size: int = 512) -> torch.Tensor:
    """max over queries of the bound >= tau, (nb, H) bool: ``spectral_energy.py:180-196``."""
    _check_keys(keys, block_size)
    require_gpu(q)
    sc = _tau_max(q, keys, want_zeta=False)
    nb, h = keys.shape[0] // block_size, keys.shape[1]
    return _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=keys.device, tau_max=sc.tau_max,
                             tau=tau, want_mask=True, want_indices=False).mask


def compute_multiband_mask(q: torch.Tensor, keys: torch.Tensor, tau: float, zeta_max: float,
                           block_size: int = 512) -> torch.Tensor:
    """Two-gate mask (bound >= tau) & (zeta <= zeta_max), (nb, H) bool:
    ``spectral_energy.py:199-234``.  One scoring pass serves both gates."""
    _check_keys(keys, block_size)
    require_gpu(q)
    sc = _tau_max(q, keys, want_zeta=True)
    nb, h = keys.shape[0] // block_size, keys.shape[1]
    return _ops.mask_compact(num_blocks=nb, num_kv_heads=h, device=keys.device, tau_max=sc.tau_max,
                             zeta=sc.zeta, tau=tau, zeta_max=zeta_max, want_mask=True,
                             want_indices=False).mask


def generate_threshold_mask(energies: torch.Tensor, epsilon: float) -> torch.Tensor:
    """energies >= epsilon: ``spectral_energy.py:237-239``."""
    return energies >= epsilon
