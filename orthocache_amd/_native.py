"""ctypes binding of liborthocache_hip.so (declared in include/orthocache_hip.h).

The library is built in-tree by ``orthocache_amd._build`` (or
``__graft_entry__.build()``).  There is no fallback: if the library is
missing or a call fails, this module raises.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "liborthocache_hip.so"

OC_F32, OC_BF16, OC_F16 = 0, 1, 2
BLOCK = 512

_DTYPE_CODES = {torch.float32: OC_F32, torch.bfloat16: OC_BF16, torch.float16: OC_F16}

_vp = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float


class FwhtArgs(C.Structure):
    _fields_ = [("x", _vp), ("x_dtype", _i32), ("x_batch_stride", _i64), ("x_row_stride", _i64),
                ("y", _vp), ("y_dtype", _i32), ("y_batch_stride", _i64), ("y_row_stride", _i64),
                ("n_cols", _i64), ("n_batch", _i64)]


class ScoreArgs(C.Structure):
    _fields_ = [("keys", _vp), ("keys_dtype", _i32), ("keys_tok_stride", _i64), ("keys_head_stride", _i64),
                ("head_dim", _i32), ("num_kv_heads", _i32), ("total_blocks", _i32),
                ("cu_blocks", _vp), ("num_segments", _i32),
                ("q", _vp), ("q_dtype", _i32), ("q_seg_stride", _i64), ("q_tok_stride", _i64),
                ("q_head_stride", _i64), ("sq", _i32), ("group", _i32),
                ("tau_max", _vp), ("zeta", _vp), ("dc", _vp), ("e_low", _vp), ("e_mid", _vp),
                ("e_high", _vp), ("e_ac", _vp), ("pages", _vp), ("num_pages", _i32), ("logits", _vp),
                ("mask", _vp), ("tau_arr", _vp), ("tau", _f32), ("zeta_max_arr", _vp), ("zeta_max", _f32)]


class BoundArgs(C.Structure):
    _fields_ = [("dc", _vp), ("e_ac", _vp), ("q", _vp), ("q_dtype", _i32),
                ("q_tok_stride", _i64), ("q_head_stride", _i64),
                ("sq", _i32), ("group", _i32), ("head_dim", _i32), ("num_kv_heads", _i32),
                ("num_blocks", _i32), ("bounds", _vp), ("tau_part", _vp)]


class CompactArgs(C.Structure):
    _fields_ = [("tau_max", _vp), ("tau_parts", _i32), ("zeta", _vp), ("mask_in", _vp),
                ("mask_in_heads", _i32), ("tau_arr", _vp), ("tau", _f32), ("zeta_max_arr", _vp),
                ("zeta_max", _f32), ("cu_blocks", _vp), ("num_segments", _i32),
                ("num_kv_heads", _i32), ("total_blocks", _i32),
                ("mask_out", _vp), ("active_out", _vp), ("indices", _vp), ("num_active", _vp),
                ("head_indices", _vp), ("head_num_active", _vp), ("head_uniform", _vp),
                ("empty_head_all", _i32)]


class AttendArgs(C.Structure):
    _fields_ = [("q", _vp), ("q_dtype", _i32), ("q_seg_stride", _i64), ("q_tok_stride", _i64),
                ("q_head_stride", _i64),
                ("k", _vp), ("v", _vp), ("kv_dtype", _i32),
                ("k_tok_stride", _i64), ("k_head_stride", _i64), ("v_tok_stride", _i64),
                ("v_head_stride", _i64),
                ("head_dim", _i32), ("num_kv_heads", _i32), ("group", _i32), ("sq", _i32),
                ("block_size", _i32), ("total_blocks", _i32),
                ("cu_blocks", _vp), ("num_segments", _i32),
                ("indices", _vp), ("counts", _vp), ("per_head", _i32), ("uniform", _vp),
                ("out", _vp), ("out_dtype", _i32),
                ("out_seg_stride", _i64), ("out_tok_stride", _i64), ("out_head_stride", _i64), ("pages", _vp), ("num_pages", _i32),
                ("logits", _vp), ("mask", _vp), ("indices_out", _vp), ("num_active_out", _vp)]


class LayerArgs(C.Structure):
    _fields_ = [("q", _vp), ("q_dtype", _i32), ("q_seg_stride", _i64), ("q_tok_stride", _i64),
                ("q_head_stride", _i64),
                ("k", _vp), ("v", _vp), ("kv_dtype", _i32),
                ("k_tok_stride", _i64), ("k_head_stride", _i64), ("v_tok_stride", _i64),
                ("v_head_stride", _i64),
                ("head_dim", _i32), ("num_kv_heads", _i32), ("group", _i32), ("sq", _i32),
                ("total_blocks", _i32), ("cu_blocks", _vp), ("num_segments", _i32),
                ("tau_arr", _vp), ("tau", _f32), ("zeta_max_arr", _vp), ("zeta_max", _f32),
                ("out", _vp), ("out_dtype", _i32),
                ("out_seg_stride", _i64), ("out_tok_stride", _i64), ("out_head_stride", _i64),
                ("tau_max", _vp), ("zeta", _vp), ("mask", _vp), ("indices", _vp), ("num_active", _vp), ("pages", _vp), ("num_pages", _i32)]


class BlockStats(C.Structure):
    _fields_ = [("dc", _vp), ("e_ac", _vp), ("zeta", _vp)]


EXPORTED_SYMBOLS = (
    "oc_last_error", "oc_abi_version", "oc_fwht512", "oc_band_energy", "oc_block_energy",
    "oc_score_blocks", "oc_query_bounds", "oc_query_bound_tiles", "oc_mask_compact",
    "oc_copy_blocks", "oc_attend_workspace_size", "oc_attend", "oc_attend_plan",
    "oc_decode_layer_workspace_size", "oc_decode_layer",
    "oc_decode_layer_cached_workspace_size", "oc_decode_layer_cached", "oc_decode_layer_noalloc",
    "orthocache_compacted_attention",
)

NOALLOC_SCRATCH_BYTES = 32 << 20  # OC_NOALLOC_SCRATCH_BYTES

_lib = None


def lib() -> C.CDLL:
    """Load the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build the HIP extension first "
            "(python -m orthocache_amd._build, or __graft_entry__.build())")
    L = C.CDLL(str(LIB_PATH))
    L.oc_last_error.restype = C.c_char_p
    L.oc_abi_version.restype = C.c_int
    for name, argt in (
        ("oc_fwht512", [C.POINTER(FwhtArgs), _vp]),
        ("oc_band_energy", [_vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp]),
        ("oc_block_energy", [_vp, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _vp, _vp]),
        ("oc_score_blocks", [C.POINTER(ScoreArgs), _vp]),
        ("oc_query_bounds", [C.POINTER(BoundArgs), _vp]),
        ("oc_mask_compact", [C.POINTER(CompactArgs), _vp]),
        ("oc_copy_blocks", [_vp, _vp, _vp, _vp, _i32, _i64, _i32, _vp]),
        ("oc_attend", [C.POINTER(AttendArgs), _vp, C.c_size_t, _vp]),
        ("oc_attend_plan", [C.POINTER(AttendArgs), C.POINTER(_i32), C.POINTER(_i32)]),
        ("oc_decode_layer", [C.POINTER(LayerArgs), _vp, C.c_size_t, _vp]),
        ("oc_decode_layer_noalloc", [C.POINTER(LayerArgs), _vp]),
    ):
        f = getattr(L, name)
        f.argtypes = argt
        f.restype = C.c_int
    L.oc_query_bound_tiles.argtypes = [_i32, _i32]
    L.oc_query_bound_tiles.restype = _i32
    L.oc_attend_workspace_size.argtypes = [C.POINTER(AttendArgs)]
    L.oc_attend_workspace_size.restype = C.c_size_t
    L.oc_decode_layer_workspace_size.argtypes = [C.POINTER(LayerArgs)]
    L.oc_decode_layer_workspace_size.restype = C.c_size_t
    L.oc_decode_layer_cached_workspace_size.argtypes = [C.POINTER(LayerArgs)]
    L.oc_decode_layer_cached_workspace_size.restype = C.c_size_t
    L.oc_decode_layer_cached.argtypes = [C.POINTER(LayerArgs), C.POINTER(BlockStats), _vp, C.c_size_t, _vp]
    L.oc_decode_layer_cached.restype = C.c_int
    L.orthocache_compacted_attention.argtypes = [_vp, C.POINTER(_vp)]
    L.orthocache_compacted_attention.restype = None
    _lib = L
    return L


class OrthoCacheError(RuntimeError):
    pass


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().oc_last_error().decode(errors="replace")
        if rc in (-1,):
            raise ValueError(f"{what}: {msg}")
        raise OrthoCacheError(f"{what} failed ({rc}): {msg}")


# ------------------------------------------------------------------ helpers
def dtype_code(t: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[t]
    except KeyError:
        raise ValueError(f"unsupported dtype {t} (float32, bfloat16, float16)") from None


def ptr(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ValueError("orthocache_amd runs on the GPU: tensors must be on a cuda (ROCm) device")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError("all tensors must be on the same device")
    if dev is None:
        raise ValueError("no tensor given")
    return dev


def aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0
