"""Stock PyTorch implementations of the nine ops: the comparison baseline of the harness.

These are reference.py's definitions (reference.py:10-78) written against torch, so that the
harness can check a kernel_fn on the GPU against stock PyTorch-ROCm and time that stock path for
"speedup_vs_pytorch", as the reference harness does with reference.py (bench.py:284-318,
:1060-1061). They are never called by a kernel_fn: the product path is libak355 only.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def matmul(A, B):
    return torch.matmul(A, B)


def softmax(x, dim=-1):
    return F.softmax(x, dim=dim)


def layernorm(x, weight, bias, eps=1e-5):
    return F.layer_norm(x, x.shape[-1:], weight, bias, eps)


def rmsnorm(x, weight, eps=1e-6):
    return (x / torch.sqrt(torch.mean(x ** 2, dim=-1, keepdim=True) + eps)) * weight


def flash_attention(Q, K, V, causal=True, sm_scale=None):
    if sm_scale is None:
        sm_scale = Q.shape[-1] ** -0.5
    s = torch.matmul(Q, K.transpose(-2, -1).contiguous()) * sm_scale
    if causal:
        mask = torch.triu(torch.ones(Q.shape[-2], K.shape[-2], device=Q.device, dtype=torch.bool), 1)
        s = s.masked_fill(mask, float("-inf"))
    return torch.matmul(F.softmax(s, dim=-1), V)


def fused_mlp(x, w_gate, w_up, w_down, activation="silu"):
    g = x @ w_gate.T
    u = x @ w_up.T
    if activation == "silu":
        g = F.silu(g)
    elif activation == "gelu":
        g = F.gelu(g)
    elif activation == "relu2":
        g = F.relu(g) ** 2
    return (g * u) @ w_down.T


def cross_entropy(logits, targets):
    return F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1))


def rotary_embedding(x, cos, sin):
    e, o = x[..., 0::2], x[..., 1::2]
    return torch.stack((e * cos - o * sin, e * sin + o * cos), dim=-1).flatten(-2)


def reduce_sum(x, dim=-1):
    return x.sum(dim=dim)


def reduce_max(x, dim=-1):
    return x.max(dim=dim).values


def _mm_checked(a, b):
    """a @ b; for fp32 the correctly rounded product (fp64 accumulation, one rounding to fp32)."""
    if a.dtype == torch.float32:
        return torch.matmul(a.double(), b.double()).float()
    return torch.matmul(a, b)


def fused_mlp_checked(x, w_gate, w_up, w_down, activation="silu"):
    """fused_mlp with every matrix product correctly rounded for fp32 (as _mm_checked)."""
    g = _mm_checked(x, w_gate.T)
    u = _mm_checked(x, w_up.T)
    if activation == "silu":
        g = F.silu(g)
    elif activation == "gelu":
        g = F.gelu(g)
    elif activation == "relu2":
        g = F.relu(g) ** 2
    return _mm_checked(g * u, w_down.T)


# keyword-dict wrappers keyed like the op table
BASELINE = {
    "matmul": lambda i: matmul(i["A"], i["B"]),
    "softmax": lambda i: softmax(i["x"]),
    "layernorm": lambda i: layernorm(i["x"], i["weight"], i["bias"]),
    "rmsnorm": lambda i: rmsnorm(i["x"], i["weight"]),
    "flash_attention": lambda i: flash_attention(i["Q"], i["K"], i["V"]),
    "fused_mlp": lambda i: fused_mlp(i["x"], i["w_gate"], i["w_up"], i["w_down"]),
    "cross_entropy": lambda i: cross_entropy(i["logits"], i["targets"]),
    "rotary_embedding": lambda i: rotary_embedding(i["x"], i["cos"], i["sin"]),
    "reduce": lambda i: reduce_sum(i["x"]),
}

# Correctness references of the harness: BASELINE, except that fp32 matrix products are checked
# against the correctly rounded product. Two fp32 summation orders over K = 8192 of N(0, 1) terms
# differ by ~1e-3, above the op table's fp32 tolerance (1e-4), so stock fp32 torch.matmul cannot
# referee a fp32 GEMM at that tolerance; it stays the timing baseline.
CHECK = dict(BASELINE)
CHECK["matmul"] = lambda i: _mm_checked(i["A"], i["B"])
CHECK["fused_mlp"] = lambda i: fused_mlp_checked(i["x"], i["w_gate"], i["w_up"], i["w_down"])
