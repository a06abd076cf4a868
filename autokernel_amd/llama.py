"""LLaMA-shaped decoder for the end-to-end check (the reference's models/llama_7b.py architecture).

Architecture (models/llama_7b.py:22-209): token embedding; per block RMSNorm
x * rsqrt(mean(x^2) + eps) * w, grouped-query attention (wq / wk / wv / wo without bias, RoPE on
q and k in fp32 with interleaved pairs, KV heads repeated, causal SDPA), residual, RMSNorm,
SwiGLU feed-forward w2(silu(w1 x) * w3 x), residual; final RMSNorm and output projection.
Module and attribute names match the reference so module-swapping plug-ins apply to both.

This is stock PyTorch: it is the baseline the plug-in (autokernel_amd.verify) replaces piece by
piece. LlamaModel7B: dim 4096, 32 layers, 32 heads, 8 KV heads, FFN 11008, vocab 32000.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps) * self.weight


def rope_tables(head_dim: int, n_pos: int, theta: float = 10000.0, device=None):
    """cos, sin [n_pos, head_dim / 2] in fp32 for positions 0..n_pos-1."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    ang = torch.outer(torch.arange(n_pos, dtype=torch.float32, device=device), inv)
    return ang.cos(), ang.sin()


def apply_rotary_emb(xq: torch.Tensor, xk: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
    """Rotate interleaved pairs of q, k [B, T, H, D] by position in fp32, cast back.

    Same arithmetic as the reference's complex multiply (models/llama_7b.py:40-48):
    (a + ib)(c + is) = (ac - bs) + i(as + bc), computed in fp32, then cast to the input dtype.
    """
    T = xq.shape[1]
    c = cos[:T].view(1, T, 1, -1)
    s = sin[:T].view(1, T, 1, -1)

    def rot(x):
        xf = x.float()
        a, b = xf[..., 0::2], xf[..., 1::2]
        return torch.stack((a * c - b * s, a * s + b * c), dim=-1).flatten(-2).type_as(x)

    return rot(xq), rot(xk)


class Attention(nn.Module):
    def __init__(self, dim: int, n_heads: int, n_kv_heads: int):
        super().__init__()
        self.n_heads = n_heads
        self.n_kv_heads = n_kv_heads
        self.head_dim = dim // n_heads
        self.n_rep = n_heads // n_kv_heads
        self.wq = nn.Linear(dim, n_heads * self.head_dim, bias=False)
        self.wk = nn.Linear(dim, n_kv_heads * self.head_dim, bias=False)
        self.wv = nn.Linear(dim, n_kv_heads * self.head_dim, bias=False)
        self.wo = nn.Linear(n_heads * self.head_dim, dim, bias=False)

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        B, T, _ = x.shape
        q = self.wq(x).view(B, T, self.n_heads, self.head_dim)
        k = self.wk(x).view(B, T, self.n_kv_heads, self.head_dim)
        v = self.wv(x).view(B, T, self.n_kv_heads, self.head_dim)
        q, k = apply_rotary_emb(q, k, cos, sin)
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        if self.n_rep > 1:
            k = k.repeat_interleave(self.n_rep, dim=1)
            v = v.repeat_interleave(self.n_rep, dim=1)
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.wo(y.transpose(1, 2).contiguous().view(B, T, -1))


class FeedForward(nn.Module):
    def __init__(self, dim: int, hidden_dim: int):
        super().__init__()
        self.w1 = nn.Linear(dim, hidden_dim, bias=False)  # gate
        self.w2 = nn.Linear(hidden_dim, dim, bias=False)  # down
        self.w3 = nn.Linear(dim, hidden_dim, bias=False)  # up

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class TransformerBlock(nn.Module):
    def __init__(self, dim: int, n_heads: int, n_kv_heads: int, hidden_dim: int):
        super().__init__()
        self.attention = Attention(dim, n_heads, n_kv_heads)
        self.feed_forward = FeedForward(dim, hidden_dim)
        self.attention_norm = RMSNorm(dim)
        self.ffn_norm = RMSNorm(dim)

    def forward(self, x, cos, sin):
        x = x + self.attention(self.attention_norm(x), cos, sin)
        return x + self.feed_forward(self.ffn_norm(x))


class LlamaModel(nn.Module):
    """Compact LLaMA (dim 768, 12 layers, 12 heads / 4 KV heads, FFN 2048)."""

    def __init__(self, vocab_size=32000, dim=768, n_layers=12, n_heads=12, n_kv_heads=4,
                 hidden_dim=2048, max_seq_len=2048):
        super().__init__()
        self.tok_embeddings = nn.Embedding(vocab_size, dim)
        self.layers = nn.ModuleList(TransformerBlock(dim, n_heads, n_kv_heads, hidden_dim) for _ in range(n_layers))
        self.norm = RMSNorm(dim)
        self.output = nn.Linear(dim, vocab_size, bias=False)
        cos, sin = rope_tables(dim // n_heads, max_seq_len * 2)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        h = self.tok_embeddings(input_ids)
        for layer in self.layers:
            h = layer(h, self.rope_cos, self.rope_sin)
        return self.output(self.norm(h))


class LlamaModel7B(LlamaModel):
    """LLaMA-7B shape: dim 4096, 32 layers, 32 heads / 8 KV heads, FFN 11008, vocab 32000."""

    def __init__(self, vocab_size=32000, dim=4096, n_layers=32, n_heads=32, n_kv_heads=8,
                 hidden_dim=11008, max_seq_len=4096):
        super().__init__(vocab_size, dim, n_layers, n_heads, n_kv_heads, hidden_dim, max_seq_len)


@torch.no_grad()
def init_weights(model: nn.Module, std: float = 0.02, seed: int = 0) -> nn.Module:
    """Random init: every Linear / Embedding weight ~ N(0, std), norm weights 1 (seeded)."""
    g = torch.Generator(device=next(model.parameters()).device)
    g.manual_seed(seed)
    for m in model.modules():
        if isinstance(m, (nn.Linear, nn.Embedding)):
            m.weight.normal_(0.0, std, generator=g)
        elif isinstance(m, RMSNorm):
            m.weight.fill_(1.0)
    return model


def build(name: str = "7b", dtype=torch.float16, device="cuda", seed: int = 0, n_layers: int | None = None):
    """Construct a model directly on `device` in `dtype` with the seeded N(0, 0.02) init."""
    cls = LlamaModel7B if name == "7b" else LlamaModel
    kw = {} if n_layers is None else {"n_layers": n_layers}
    with torch.device(device):
        model = cls(**kw).to(dtype)
    return init_weights(model, seed=seed).eval()
