"""Flash-attention drop-in: kernel_fn(Q, K, V, causal=True, sm_scale=None).

Mirrors reference.py:32-42 and kernels/flash_attention.py:130: Q, K, V [batch, heads, seq, D]
(3-D [heads, seq, D] also accepted), default scale D**-0.5, causal mask j > i (top-left aligned).
K / V may carry fewer heads than Q when the head count divides (grouped-query attention; one KV
head broadcasts, as the reference's matmul does). Strided views with a contiguous last dim are
read in place, so [B, S, H, D] tensors need no transpose copy. f16 / bf16 with D 64 or 128 run
the MFMA kernels, and so do f16 / bf16 heads narrower than 128 (16, 32, 96, ...), zero-padded to
64 or 128: zero columns add nothing to Q K^T, the padded output columns are dropped, and the scale
stays D**-0.5 of the true D. fp32, and f16 / bf16 heads wider than 128, run the general kernel, which
keeps the reference's roundings step by step. Runs ak_flash_attn_fwd (attention.hip).
kernel_fn is kernels/host.py's flash_attention; attention() is the 4-D form the model plug-in
uses, which can also write into a strided output view.
"""
from __future__ import annotations

import torch

from . import _ops
from .host import flash_attention as kernel_fn  # noqa: F401

KERNEL_TYPE = "flash_attention"


def _prep(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def attention(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, causal: bool = True,
              sm_scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """4-D entry point: Q [B, Hq, Sq, D], K / V [B, Hkv, Sk, D]; out may be a strided view."""
    B, Hq, Sq, D = Q.shape
    Bk, Hkv, Sk, Dk = K.shape
    if V.shape != K.shape or Dk != D or Bk != B:
        raise ValueError(f"flash_attention: shapes Q{tuple(Q.shape)} K{tuple(K.shape)} V{tuple(V.shape)}")
    if Hkv == 0 or Hq % Hkv:
        raise ValueError(f"flash_attention: {Hq} query heads not a multiple of {Hkv} KV heads")
    if not (Q.dtype == K.dtype == V.dtype):
        raise ValueError("flash_attention: Q, K, V dtypes differ")
    if Q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError(f"flash_attention: dtype {Q.dtype} unsupported (float16, bfloat16, float32)")
    if not 1 <= D <= 256:
        raise ValueError(f"flash_attention: head_dim {D} unsupported (1 .. 256)")
    if sm_scale is None:
        sm_scale = D ** -0.5
    if Q.dtype != torch.float32 and D < 128 and D != 64:
        Dp = 64 if D < 64 else 128
        padded = [torch.nn.functional.pad(t, (0, Dp - D)) for t in (Q, K, V)]
        res = attention(*padded, causal, sm_scale)[..., :D]
        if out is None:
            return res.contiguous()
        out.copy_(res)
        return out
    Q, K, V = _prep(Q), _prep(K), _prep(V)
    O = out if out is not None else torch.empty((B, Hq, Sq, D), device=Q.device, dtype=Q.dtype)
    if Sk == 0:
        raise ValueError("flash_attention: empty key sequence")
    _ops.flash_attn_fwd(O, Q, K, V, bool(causal), float(sm_scale))
    return O
