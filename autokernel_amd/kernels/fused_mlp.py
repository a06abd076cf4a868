"""Fused SwiGLU MLP drop-in: kernel_fn(x, w_gate, w_up, w_down, activation="silu").

Mirrors reference.py:45-55 and kernels/fused_mlp.py:102: weights in nn.Linear layout
(w_gate, w_up [hidden, dim], w_down [dim, hidden]); activation "silu", "gelu" (exact erf) or
"relu2", any other string leaves the gate unactivated, as the reference does. The gate and up
projections, the activation and their product run in one dual-GEMM kernel (ak_mlp_gate_up);
the down projection is ak_gemm reading w_down in place. kernel_fn is kernels/host.py's fused_mlp.
"""
from __future__ import annotations

import torch

from . import _ops
from .host import ACT_NONE, ACTIVATIONS
from .host import fused_mlp as kernel_fn  # noqa: F401

KERNEL_TYPE = "fused_mlp"


def gate_up(x2: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, activation: str = "silu") -> torch.Tensor:
    """h = act(x2 @ w_gate.T) * (x2 @ w_up.T) for 2-D x2 [M, D] in one ak_mlp_gate_up launch, with
    the reference's roundings of gate, up, the activation and the product (reference.py:47-54)."""
    M, D = x2.shape
    H = w_gate.shape[0]
    if w_gate.shape != (H, D) or w_up.shape != (H, D):
        raise ValueError(f"fused_mlp: weight shapes {tuple(w_gate.shape)}, {tuple(w_up.shape)} do not fit x [*, {D}]")
    h = torch.empty((M, H), device=x2.device, dtype=x2.dtype)
    _ops.mlp_gate_up(h, x2.contiguous(), w_gate.contiguous(), w_up.contiguous(), ACTIVATIONS.get(activation, ACT_NONE))
    return h
