"""Fused SwiGLU MLP drop-in: kernel_fn(x, w_gate, w_up, w_down, activation="silu").

Mirrors reference.py:45-55 and kernels/fused_mlp.py:102: weights in nn.Linear layout
(w_gate, w_up [hidden, dim], w_down [dim, hidden]); activation "silu", "gelu" (exact erf) or
"relu2", any other string leaves the gate unactivated, as the reference does. The gate and up
projections, the activation and their product run in one dual-GEMM kernel (ak_mlp_gate_up);
the down projection is ak_gemm reading w_down in place.
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import device_guard
from .matmul import gemm

KERNEL_TYPE = "fused_mlp"


def gate_up(x2: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, activation: str = "silu") -> torch.Tensor:
    """h = act(x2 @ w_gate.T) * (x2 @ w_up.T) for 2-D x2 [M, D] in one ak_mlp_gate_up launch, with
    the reference's roundings of gate, up, the activation and the product (reference.py:47-54)."""
    code = _lib.dtype_code(x2, "fused_mlp")
    M, D = x2.shape
    H = w_gate.shape[0]
    if w_gate.shape != (H, D) or w_up.shape != (H, D):
        raise ValueError(f"fused_mlp: weight shapes {tuple(w_gate.shape)}, {tuple(w_up.shape)} do not fit x [*, {D}]")
    wg, wu = w_gate.contiguous(), w_up.contiguous()
    act = _lib.ACTIVATIONS.get(activation, _lib.ACT_NONE)
    h = torch.empty((M, H), device=x2.device, dtype=x2.dtype)
    with device_guard(x2):
        st = _lib.load().ak_mlp_gate_up(code, x2.data_ptr(), wg.data_ptr(), wu.data_ptr(),
                                        h.data_ptr(), M, H, D, act, _lib.stream_of(x2))
    _lib.check(st, "ak_mlp_gate_up", M=M, H=H, D=D, dtype=x2.dtype)
    return h


def kernel_fn(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
              activation: str = "silu") -> torch.Tensor:
    _lib.require_gpu("fused_mlp", x, w_gate, w_up, w_down)
    _lib.dtype_code(x, "fused_mlp")
    for name, w in (("w_gate", w_gate), ("w_up", w_up), ("w_down", w_down)):
        if w.dtype != x.dtype:
            raise ValueError(f"fused_mlp: {name} dtype {w.dtype} != x dtype {x.dtype}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    D = x2.shape[1]
    H = w_gate.shape[0]
    if w_gate.shape != (H, D) or w_up.shape != (H, D) or w_down.shape[1] != H:
        raise ValueError(f"fused_mlp: weight shapes {tuple(w_gate.shape)}, {tuple(w_up.shape)}, "
                         f"{tuple(w_down.shape)} do not fit x [*, {D}]")
    h = gate_up(x2, w_gate, w_up, activation)
    out = gemm(h, w_down.t())
    return out.view(*lead, w_down.shape[0])
