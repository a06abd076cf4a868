"""PyTorch-CPU restatement of the reference's reference.py (test infrastructure only).

Each function follows the reference function cited beside it op for op: every intermediate is a
tensor of the input's dtype, so the rounding points (and f16 overflow to inf) are the
reference's. Inputs are moved to the CPU; results come back on the CPU.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def _cpu(*ts):
    return [t.detach().cpu() if isinstance(t, torch.Tensor) else t for t in ts]


def _mm(a, b):
    """torch.matmul with the reference's arithmetic: exact products summed in fp32 or wider, one
    rounding to the input dtype. f16 / bf16 operands are multiplied in fp32 and rounded (what the
    GPU BLAS path computes; CPU f16 GEMM is much slower); fp32 operands are multiplied in fp64 and
    rounded once, i.e. the correctly rounded product, so the oracle's own summation error does not
    eat into the 1e-4 fp32 tolerance."""
    if a.dtype in (torch.float16, torch.bfloat16) and b.dtype == a.dtype:
        return torch.matmul(a.float(), b.float()).to(a.dtype)
    if a.dtype == torch.float32 and b.dtype == torch.float32:
        return torch.matmul(a.double(), b.double()).float()
    return torch.matmul(a, b)


def matmul_ref(A, B):
    """reference.py:10-12 -- torch.matmul(A, B)."""
    A, B = _cpu(A, B)
    return _mm(A, B)


def softmax_ref(x, dim=-1):
    """reference.py:15-17 -- F.softmax(x, dim)."""
    (x,) = _cpu(x)
    return F.softmax(x, dim=dim)


def layernorm_ref(x, weight, bias, eps=1e-5):
    """reference.py:20-23 -- F.layer_norm over the last dim."""
    x, weight, bias = _cpu(x, weight, bias)
    return F.layer_norm(x, x.shape[-1:], weight, bias, eps)


def rmsnorm_ref(x, weight, eps=1e-6):
    """reference.py:26-29 -- rms = sqrt(mean(x**2, -1) + eps); (x / rms) * weight."""
    x, weight = _cpu(x, weight)
    sq = x ** 2
    rms = torch.sqrt(torch.mean(sq, dim=-1, keepdim=True) + eps)
    return (x / rms) * weight


def flash_attention_ref(Q, K, V, causal=True, sm_scale=None):
    """reference.py:32-42 -- (Q K^T) * scale, triu(…, 1) mask to -inf, softmax, @ V."""
    Q, K, V = _cpu(Q, K, V)
    if sm_scale is None:
        sm_scale = Q.shape[-1] ** -0.5
    scores = _mm(Q, K.transpose(-2, -1)) * sm_scale
    if causal:
        sq, sk = Q.shape[-2], K.shape[-2]
        upper = torch.triu(torch.ones(sq, sk, dtype=torch.bool), diagonal=1)
        scores = scores.masked_fill(upper, float("-inf"))
    return _mm(F.softmax(scores, dim=-1), V)


def fused_mlp_ref(x, w_gate, w_up, w_down, activation="silu"):
    """reference.py:45-55 -- act(x @ w_gate.T) * (x @ w_up.T) @ w_down.T, each step materialised."""
    x, w_gate, w_up, w_down = _cpu(x, w_gate, w_up, w_down)
    g = _mm(x, w_gate.T)
    u = _mm(x, w_up.T)
    if activation == "silu":
        g = F.silu(g)
    elif activation == "gelu":
        g = F.gelu(g)
    elif activation == "relu2":
        g = F.relu(g) ** 2
    return _mm(g * u, w_down.T)


def cross_entropy_ref(logits, targets, ignore_index=-100):
    """reference.py:58-60 -- F.cross_entropy(logits.view(-1, V), targets.view(-1)).

    For f16 / bf16 this spells out the arithmetic of the GPU run the reference harness makes:
    log_softmax stored in the logits' dtype, -logp[target] summed in fp32 over the rows whose
    target is not ignore_index, divided by their count, rounded once. (PyTorch's CPU kernel sums
    the half values in half and overflows once the sum passes 65504, e.g. 8192 rows of ~10.8.)
    """
    logits, targets = _cpu(logits, targets)
    x = logits.view(-1, logits.size(-1))
    t = targets.view(-1)
    if x.dtype not in (torch.float16, torch.bfloat16):
        return F.cross_entropy(x, t, ignore_index=ignore_index)
    lp = F.log_softmax(x, dim=-1)
    keep = t != ignore_index
    picked = -lp.gather(1, t.clamp_min(0).unsqueeze(1)).squeeze(1).float()
    return (picked[keep].sum() / keep.sum()).to(x.dtype)


def rotary_embedding_ref(x, cos, sin):
    """reference.py:63-69 -- interleaved pairs rotated, each product / sum rounded."""
    x, cos, sin = _cpu(x, cos, sin)
    even, odd = x[..., 0::2], x[..., 1::2]
    out_even = even * cos - odd * sin
    out_odd = even * sin + odd * cos
    return torch.stack((out_even, out_odd), dim=-1).flatten(-2)


def reduce_sum_ref(x, dim=-1):
    """reference.py:72-74 -- x.sum(dim)."""
    (x,) = _cpu(x)
    return x.sum(dim=dim)


def reduce_max_ref(x, dim=-1):
    """reference.py:76-78 -- x.max(dim).values."""
    (x,) = _cpu(x)
    return x.max(dim=dim).values


REFERENCE = {
    "matmul": lambda i: matmul_ref(i["A"], i["B"]),
    "softmax": lambda i: softmax_ref(i["x"]),
    "layernorm": lambda i: layernorm_ref(i["x"], i["weight"], i["bias"]),
    "rmsnorm": lambda i: rmsnorm_ref(i["x"], i["weight"]),
    "flash_attention": lambda i: flash_attention_ref(i["Q"], i["K"], i["V"]),
    "fused_mlp": lambda i: fused_mlp_ref(i["x"], i["w_gate"], i["w_up"], i["w_down"]),
    "cross_entropy": lambda i: cross_entropy_ref(i["logits"], i["targets"]),
    "rotary_embedding": lambda i: rotary_embedding_ref(i["x"], i["cos"], i["sin"]),
    "reduce": lambda i: reduce_sum_ref(i["x"]),
}
"""Keyword-dict wrappers in the style of the reference harness's _ref_* (bench.py:284-318)."""
