"""Reduction drop-in: kernel_fn(x, dim=-1) (sum) and reduce_max(x, dim=-1).

Mirrors reference.py:72-78 (x.sum(dim), x.max(dim).values) and kernels/reduce.py:51, which
handles any dim. x is viewed as [outer, reduce, inner] and reduced in place of dim, with no
permute copy. Sum accumulates in fp32 in a fixed order (bitwise deterministic) and rounds once;
max is exact and propagates NaN. Runs ak_reduce_sum / ak_reduce_max (rows.hip).
"""
from __future__ import annotations

import math

import torch

from .. import _lib
from ._common import device_guard

KERNEL_TYPE = "reduce"


def _reduce(x: torch.Tensor, dim: int, is_max: bool) -> torch.Tensor:
    op = "reduce_max" if is_max else "reduce_sum"
    _lib.require_gpu(op, x)
    code = _lib.dtype_code(x, op)
    if x.dim() == 0:
        return x.clone()
    d = dim % x.dim()
    outer = math.prod(x.shape[:d])
    red = x.shape[d]
    inner = math.prod(x.shape[d + 1:])
    if is_max and red == 0:
        raise ValueError("reduce_max: cannot reduce an empty dimension")
    xc = x.contiguous()
    out_shape = x.shape[:d] + x.shape[d + 1:]
    y = torch.empty(out_shape, device=x.device, dtype=x.dtype)
    fn = _lib.load().ak_reduce_max if is_max else _lib.load().ak_reduce_sum
    with device_guard(x):
        st = fn(code, xc.data_ptr(), y.data_ptr(), outer, red, inner, _lib.stream_of(x))
    _lib.check(st, "ak_" + op, shape=tuple(x.shape), dim=dim, dtype=x.dtype)
    return y


def kernel_fn(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    return _reduce(x, dim, False)


def reduce_max(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    return _reduce(x, dim, True)
