"""RMSNorm drop-in: kernel_fn(x, weight, eps=1e-6).

Mirrors reference.py:26-29 (rmsnorm_ref) and the slot kernels/rmsnorm.py:45: x of any rank,
normalised over the last dim, output of x's shape and dtype. Runs ak_rmsnorm (rows.hip).
A weight of another dtype is cast to x's dtype first (as the reference starters do,
kernels/cuda/rmsnorm.py:176-180).
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import device_guard, match_dtype, rows_view

KERNEL_TYPE = "rmsnorm"


def kernel_fn(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    _lib.require_gpu("rmsnorm", x, weight)
    code = _lib.dtype_code(x, "rmsnorm")
    x2 = rows_view(x)
    rows, cols = x2.shape
    w = match_dtype(weight, x.dtype).contiguous().view(-1)
    if w.numel() != cols:
        raise ValueError(f"rmsnorm: weight has {w.numel()} elements, x rows have {cols}")
    y = torch.empty_like(x2)
    with device_guard(x):
        st = _lib.load().ak_rmsnorm(code, x2.data_ptr(), w.data_ptr(), y.data_ptr(), rows, cols,
                                    float(eps), _lib.stream_of(x))
    _lib.check(st, "ak_rmsnorm", shape=tuple(x.shape), dtype=x.dtype)
    return y.view(x.shape)


def rms_norm_rsqrt(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """A LLaMA block's RMSNorm module (models/llama_7b.py:28-30): x * rsqrt(mean(x^2) + eps) * w,
    each op rounded to x's dtype. Runs ak_rmsnorm_rsqrt."""
    _lib.require_gpu("rms_norm_rsqrt", x, weight)
    code = _lib.dtype_code(x, "rms_norm_rsqrt")
    x2 = rows_view(x)
    rows, cols = x2.shape
    w = match_dtype(weight, x.dtype).contiguous().view(-1)
    y = torch.empty_like(x2)
    with device_guard(x):
        st = _lib.load().ak_rmsnorm_rsqrt(code, x2.data_ptr(), w.data_ptr(), y.data_ptr(), rows, cols,
                                          float(eps), _lib.stream_of(x))
    _lib.check(st, "ak_rmsnorm_rsqrt", shape=tuple(x.shape), dtype=x.dtype)
    return y.view(x.shape)
