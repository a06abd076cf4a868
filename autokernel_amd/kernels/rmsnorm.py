"""RMSNorm drop-in: kernel_fn(x, weight, eps=1e-6).

Mirrors reference.py:26-29 (rmsnorm_ref) and the slot kernels/rmsnorm.py:45: x of any rank,
normalised over the last dim, output of x's shape and dtype. Runs ak_rmsnorm (rows.hip).
A weight of another dtype is cast to x's dtype first (as the reference starters do,
kernels/cuda/rmsnorm.py:176-180). kernel_fn is kernels/host.py's rmsnorm.
"""
from __future__ import annotations

import torch

from . import _ops
from ._common import match_dtype, require_gpu, rows_view
from .host import rmsnorm as kernel_fn  # noqa: F401

KERNEL_TYPE = "rmsnorm"


def rms_norm_rsqrt(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """A LLaMA block's RMSNorm module (models/llama_7b.py:28-30): x * rsqrt(mean(x^2) + eps) * w,
    each op rounded to x's dtype. Runs ak_rmsnorm_rsqrt."""
    require_gpu("rms_norm_rsqrt", x, weight)
    x2 = rows_view(x)
    w = match_dtype(weight, x.dtype).contiguous().view(-1)
    if w.numel() != x2.shape[1]:
        raise ValueError(f"rms_norm_rsqrt: weight has {w.numel()} elements, x rows have {x2.shape[1]}")
    y = torch.empty_like(x2)
    _ops.rmsnorm_rsqrt(y, x2, w, eps)
    return y.view(x.shape)
