"""Reduction drop-in: kernel_fn(x, dim=-1) (sum) and reduce_max(x, dim=-1).

Mirrors reference.py:72-78 (x.sum(dim), x.max(dim).values) and kernels/reduce.py:51, which
handles any dim. x is viewed as [outer, reduce, inner] and reduced in place of dim, with no
permute copy. Sum accumulates in fp32 in a fixed order (bitwise deterministic) and rounds once;
max is exact and propagates NaN. Runs ak_reduce_sum / ak_reduce_max (rows.hip). The functions
are kernels/host.py's reduce and reduce_max.
"""
from __future__ import annotations

from .host import reduce as kernel_fn  # noqa: F401
from .host import reduce_max  # noqa: F401

KERNEL_TYPE = "reduce"
