"""Helpers shared by the kernel_fn modules: GPU check and row flattening."""
from __future__ import annotations

import torch


def rows_view(x: torch.Tensor) -> torch.Tensor:
    """[..., N] -> contiguous [rows, N] (a view when x is already contiguous)."""
    if x.dim() == 0:
        x = x.reshape(1, 1)
    elif x.dim() == 1:
        x = x.reshape(1, -1)
    x = x.contiguous()
    return x.view(-1, x.shape[-1])


def match_dtype(t: torch.Tensor | None, dtype: torch.dtype) -> torch.Tensor | None:
    if t is None or t.dtype == dtype:
        return t
    return t.to(dtype)


def require_gpu(op: str, *tensors: torch.Tensor | None) -> None:
    """RuntimeError for a CPU tensor: the library has no CPU path."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{op}: expected GPU tensors, got a tensor on {t.device} "
                               "(autokernel_amd has no CPU path)")
