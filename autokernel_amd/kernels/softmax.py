"""Softmax drop-in: kernel_fn(x, dim=-1).

Mirrors reference.py:15-17 (F.softmax) and kernels/softmax.py:57. Any rank; a dim other than the
last is moved last around the kernel call. Runs ak_softmax (rows.hip). The function is
kernels/host.py's softmax.
"""
from __future__ import annotations

from .host import softmax as kernel_fn  # noqa: F401

KERNEL_TYPE = "softmax"
