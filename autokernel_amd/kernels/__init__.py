"""The nine AutoKernel ops as drop-in kernel_fn modules backed by libak355 (gfx950 HIP).

Each module exposes KERNEL_TYPE and kernel_fn with the signature of the matching reference.py
function, like the reference's kernels/*.py slot modules. The kernel_fns themselves live in
kernels/host.py (the shape layer shared with the HuggingFace Kernels export), bound here to the
ctypes-backed ops of kernels/_ops.py.
"""
from __future__ import annotations

from . import _ops, host

host.bind(_ops)

from . import (cross_entropy, flash_attention, fused_mlp, layernorm, matmul, reduce, rmsnorm,  # noqa: E402
               rotary_embedding, softmax)

MODULES = {m.KERNEL_TYPE: m for m in (matmul, softmax, layernorm, rmsnorm, flash_attention,
                                      fused_mlp, cross_entropy, rotary_embedding, reduce)}
KERNELS = {name: m.kernel_fn for name, m in MODULES.items()}


def get(kernel_type: str):
    """kernel_fn for a KERNEL_TYPE name (bench.py KERNEL_CONFIGS keys)."""
    try:
        return KERNELS[kernel_type]
    except KeyError:
        raise KeyError(f"unknown kernel type {kernel_type!r}; known: {sorted(KERNELS)}") from None
