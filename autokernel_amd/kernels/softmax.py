"""Softmax drop-in: kernel_fn(x, dim=-1).

Mirrors reference.py:15-17 (F.softmax) and kernels/softmax.py:57. Any rank; a dim other than the
last is moved last around the kernel call. Runs ak_softmax (rows.hip).
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import device_guard, rows_view

KERNEL_TYPE = "softmax"


def kernel_fn(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    _lib.require_gpu("softmax", x)
    code = _lib.dtype_code(x, "softmax")
    if x.dim() == 0:
        return kernel_fn(x.reshape(1)).reshape(())
    d = dim % x.dim()
    xm = x if d == x.dim() - 1 else x.movedim(d, -1)
    x2 = rows_view(xm)
    rows, cols = x2.shape
    y = torch.empty_like(x2)
    with device_guard(x):
        st = _lib.load().ak_softmax(code, x2.data_ptr(), y.data_ptr(), rows, cols, _lib.stream_of(x))
    _lib.check(st, "ak_softmax", shape=tuple(x.shape), dtype=x.dtype)
    y = y.view(xm.shape)
    return y if d == x.dim() - 1 else y.movedim(-1, d)
