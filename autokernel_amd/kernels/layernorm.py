"""LayerNorm drop-in: kernel_fn(x, weight, bias, eps=1e-5).

Mirrors reference.py:20-23 (F.layer_norm over the last dim) and kernels/layernorm.py:65-70.
weight / bias may be None (identity scale / zero shift, as F.layer_norm allows). Runs
ak_layernorm (rows.hip). The function is kernels/host.py's layernorm.
"""
from __future__ import annotations

from .host import layernorm as kernel_fn  # noqa: F401

KERNEL_TYPE = "layernorm"
