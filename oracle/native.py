"""ctypes wrappers for oracle/_build/liboc_port.so and oracle/_ref (TEST INFRASTRUCTURE)."""

from __future__ import annotations

import ctypes as C

import numpy as np

from .build import PORT_LIB, REF_LIB

_port = None
_ref = None


def port():
    global _port
    if _port is None:
        if not PORT_LIB.exists():
            raise RuntimeError(f"{PORT_LIB} missing: run oracle/build.py")
        L = C.CDLL(str(PORT_LIB))
        L.oc_port_threads.restype = C.c_int
        L.oc_port_score.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]
        L.oc_port_compact.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_float, C.c_float, C.c_void_p,
                                      C.c_void_p]
        L.oc_port_compact.restype = C.c_int
        L.oc_port_attend.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int,
                                     C.c_void_p, C.c_int, C.c_void_p]
        _port = L
    return _port


def _p(a):
    return a.ctypes.data if a is not None else None


def port_score(keys_bf16: np.ndarray, qf: np.ndarray | None):
    """keys_bf16: uint16 (S, H, D); qf: fp32 folded queries (nq, H, D)."""
    s, h, d = keys_bf16.shape
    nb = s // 512
    keys_bf16 = np.ascontiguousarray(keys_bf16, dtype=np.uint16)
    tm = np.empty((nb, h), np.float32)
    z = np.empty((nb, h), np.float32)
    nq = 0
    if qf is not None:
        qf = np.ascontiguousarray(qf, dtype=np.float32)
        nq = qf.shape[0]
    port().oc_port_score(_p(keys_bf16), nb, h, d, _p(qf), nq, _p(tm) if nq else None, _p(z))
    return (tm if nq else None), z


def port_compact(tau_max, zeta, tau, zeta_max):
    nb, h = tau_max.shape
    tau_max = np.ascontiguousarray(tau_max, np.float32)
    zeta = np.ascontiguousarray(zeta, np.float32)
    mask = np.empty((nb, h), np.uint8)
    idx = np.empty((nb,), np.int32)
    n = port().oc_port_compact(_p(tau_max), _p(zeta), nb, h, tau, zeta_max, _p(mask), _p(idx))
    return mask.astype(bool), idx, int(n)


def port_attend(q, k_bf16, v_bf16, indices, num_active):
    sq, hq, d = q.shape
    hkv = k_bf16.shape[1]
    q = np.ascontiguousarray(q, np.float32)
    k_bf16 = np.ascontiguousarray(k_bf16, np.uint16)
    v_bf16 = np.ascontiguousarray(v_bf16, np.uint16)
    idx = np.ascontiguousarray(indices, np.int32)
    out = np.empty((sq, hq, d), np.float32)
    port().oc_port_attend(_p(q), _p(k_bf16), _p(v_bf16), sq, hq, hkv, d, _p(idx), int(num_active), _p(out))
    return out


def ref_available() -> bool:
    return REF_LIB.exists()


class _Desc(C.Structure):
    # notebooks/phase_d_kaggle.py:211-217
    _fields_ = [("seq_len_q", C.c_int32), ("seq_len_k", C.c_int32), ("head_dim", C.c_int32),
                ("block_size", C.c_int32), ("num_blocks", C.c_int32)]


def ref_compacted_attention(q, keys, values, block_mask, block_size=512):
    """The reference's own C++ CPU attention (single head, fp32):
    inputs q (Sq, D), keys/values (Sk, D), block_mask int32 (nb,)."""
    global _ref
    if _ref is None:
        _ref = C.CDLL(str(REF_LIB))
        _ref.orthocache_compacted_attention.argtypes = [C.c_void_p, C.c_void_p]
        _ref.orthocache_compacted_attention.restype = None
    q = np.ascontiguousarray(q, np.float32)
    keys = np.ascontiguousarray(keys, np.float32)
    values = np.ascontiguousarray(values, np.float32)
    m = np.ascontiguousarray(block_mask, np.int32)
    sq, d = q.shape
    sk = keys.shape[0]
    desc = _Desc(sq, sk, d, block_size, sk // block_size)
    out = np.zeros((sq, d), np.float32)
    ins = (C.c_void_p * 5)(q.ctypes.data, keys.ctypes.data, values.ctypes.data, m.ctypes.data,
                           C.addressof(desc))
    _ref.orthocache_compacted_attention(out.ctypes.data, ins)
    return out
