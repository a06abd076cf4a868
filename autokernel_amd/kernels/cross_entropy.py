"""Cross-entropy drop-in: kernel_fn(logits, targets).

Mirrors reference.py:58-60 (F.cross_entropy on logits.view(-1, V), targets.view(-1): mean over
rows, ignore_index -100) and kernels/cross_entropy.py:70. Returns a 0-dim tensor of the logits'
dtype, as the reference does. A target outside [0, V) other than -100 gives NaN (torch raises a
device-side assert instead). Runs ak_cross_entropy (rows.hip) with a per-row fp32 workspace.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import device_guard

KERNEL_TYPE = "cross_entropy"
IGNORE_INDEX = -100


def kernel_fn(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    _lib.require_gpu("cross_entropy", logits, targets)
    code = _lib.dtype_code(logits, "cross_entropy")
    v = logits.shape[-1]
    x2 = logits.contiguous().view(-1, v)
    t = targets.reshape(-1)
    if t.dtype != torch.int64:
        t = t.to(torch.int64)
    t = t.contiguous()
    if t.numel() != x2.shape[0]:
        raise ValueError(f"cross_entropy: {x2.shape[0]} rows of logits but {t.numel()} targets")
    rows = x2.shape[0]
    loss = torch.empty(max(rows, 1), device=logits.device, dtype=torch.float32)
    out = torch.empty((), device=logits.device, dtype=logits.dtype)
    with device_guard(logits):
        st = _lib.load().ak_cross_entropy(code, x2.data_ptr(), t.data_ptr(), loss.data_ptr(),
                                          out.data_ptr(), rows, v, IGNORE_INDEX,
                                          _lib.stream_of(logits))
    _lib.check(st, "ak_cross_entropy", shape=tuple(logits.shape), dtype=logits.dtype)
    return out
