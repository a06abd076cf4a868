"""LayerNorm drop-in: kernel_fn(x, weight, bias, eps=1e-5).

Mirrors reference.py:20-23 (F.layer_norm over the last dim) and kernels/layernorm.py:65-70.
weight / bias may be None (identity scale / zero shift, as F.layer_norm allows). Runs
ak_layernorm (rows.hip).
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import device_guard, match_dtype, rows_view

KERNEL_TYPE = "layernorm"


def kernel_fn(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
              eps: float = 1e-5) -> torch.Tensor:
    _lib.require_gpu("layernorm", x, weight, bias)
    code = _lib.dtype_code(x, "layernorm")
    x2 = rows_view(x)
    rows, cols = x2.shape
    w = match_dtype(weight, x.dtype)
    b = match_dtype(bias, x.dtype)
    w = None if w is None else w.contiguous().view(-1)
    b = None if b is None else b.contiguous().view(-1)
    for name, t in (("weight", w), ("bias", b)):
        if t is not None and t.numel() != cols:
            raise ValueError(f"layernorm: {name} has {t.numel()} elements, x rows have {cols}")
    y = torch.empty_like(x2)
    with device_guard(x):
        st = _lib.load().ak_layernorm(code, x2.data_ptr(), _lib.ptr(w), _lib.ptr(b), y.data_ptr(),
                                      rows, cols, float(eps), _lib.stream_of(x))
    _lib.check(st, "ak_layernorm", shape=tuple(x.shape), dtype=x.dtype)
    return y.view(x.shape)
