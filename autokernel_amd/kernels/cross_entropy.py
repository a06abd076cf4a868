"""Cross-entropy drop-in: kernel_fn(logits, targets).

Mirrors reference.py:58-60 (F.cross_entropy on logits.view(-1, V), targets.view(-1): mean over
rows, ignore_index -100) and kernels/cross_entropy.py:70. Returns a 0-dim tensor of the logits'
dtype, as the reference does. A target outside [0, V) other than -100 gives NaN (torch raises a
device-side assert instead). Runs ak_cross_entropy (rows.hip) with a per-row fp32 workspace. The
function is kernels/host.py's cross_entropy.
"""
from __future__ import annotations

from .host import IGNORE_INDEX  # noqa: F401
from .host import cross_entropy as kernel_fn  # noqa: F401

KERNEL_TYPE = "cross_entropy"
