"""Rotary-embedding drop-in: kernel_fn(x, cos, sin).

Mirrors reference.py:63-69 (interleaved pairs, cos / sin of shape [..., D/2] broadcast against
x[..., ::2]) and kernels/rotary_embedding.py:75. The table row of each x row is found from the
broadcast pattern without copying for the two layouts models use:
  * cos [S, D/2] (or with leading 1s) against x [..., S, D]        -> row r uses r % S
  * cos [S, 1, D/2] (or [1, S, 1, D/2]) against x [..., S, H, D]    -> row r uses (r // H) % S
Other broadcasts are expanded to one table row per x row. Mixed dtypes follow torch type
promotion (all operands are cast to the promoted dtype, which is exact). Runs ak_rope (rope.hip).
kernel_fn is kernels/host.py's rotary_embedding.
"""
from __future__ import annotations

import torch

from . import _ops
from ._common import require_gpu
from .host import rotary_embedding as kernel_fn  # noqa: F401

KERNEL_TYPE = "rotary_embedding"


def apply_fp32_tables(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """A LLaMA block's RoPE (models/llama_7b.py:40-48) on x [B, T, H, D]: fp32 tables [>= T, D/2],
    fp32 arithmetic, one rounding to x's dtype. x may be a column slice of a wider projection
    output (head and dim contiguous, any token stride). Returns a dense [B, T, H, D] tensor.
    Runs ak_rope_f32_tables."""
    require_gpu("rope_fp32_tables", x, cos, sin)
    B, T, H, D = x.shape
    if not (x.stride(3) == 1 and x.stride(2) == D and x.stride(0) == T * x.stride(1)):
        x = x.contiguous()
    c = cos[:T].float().contiguous()
    s = sin[:T].float().contiguous()
    y = torch.empty((B, T, H, D), device=x.device, dtype=x.dtype)
    _ops.rope_f32_tables(y, x, c, s, B * T * H, D, T, H, x.stride(1))
    return y
