"""fwht_512 on the GPU (reference: src/orthocache/fwht.py:4-65)."""

from __future__ import annotations

import torch

from . import _ops
from ._native import require_gpu

_FLOATS = (torch.float32, torch.bfloat16, torch.float16)


def fwht_512(x: torch.Tensor) -> torch.Tensor:
    """512-row fast Walsh-Hadamard transform along axis 0, normalised by 1/sqrt(512).

    Same contract as the reference (``fwht.py:4-65``): input (512, d) or
    (512,), output in natural (Hadamard) order with the input's shape.  The
    arithmetic is fp32 for every input type; a bf16/fp16 input is rounded to
    its dtype once at the end (the reference keeps the input dtype, so its
    bf16 path rounds after every stage).  Integer inputs give float32.
    """
    require_gpu(x)
    if x.dim() not in (1, 2) or x.shape[0] != 512:
        raise ValueError(f"fwht_512 expects shape (512,) or (512, d), got {tuple(x.shape)}")
    out_dtype = x.dtype if x.dtype in _FLOATS else torch.float32
    if x.dtype not in _FLOATS:
        x = x.to(torch.float32)
    one_d = x.dim() == 1
    x2 = x.reshape(512, -1)
    y = _ops.fwht_rows(x2.unsqueeze(0), out_dtype=out_dtype)[0]
    return y.reshape(512) if one_d else y
