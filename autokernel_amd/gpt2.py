"""GPT-2 (small by default) for the plug-in check: the reference's models/gpt2.py architecture.

Architecture (models/gpt2.py:18-141): token and position embeddings; per block a pre-LayerNorm
causal self-attention with one fused c_attn projection (3 x n_embd outputs, biased), scores
(q k^T) / sqrt(head_dim) masked by a lower-triangular `bias` buffer, an explicit softmax and
att @ v, then c_proj; a pre-LayerNorm MLP c_fc -> exact-erf GELU -> c_proj; final ln_f and an
lm_head whose weight is the token embedding's. Module and attribute names follow the reference
(transformer.{wte, wpe, h, ln_f}, attn.c_attn, n_head, n_embd, the `bias` mask), so the same
module-swapping plug-in applies to both.

This is stock PyTorch: the baseline autokernel_amd.verify replaces piece by piece. GPT2():
vocab 50257, block 1024, 12 layers, 12 heads, n_embd 768 (124 M parameters).
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F


class CausalSelfAttention(nn.Module):
    def __init__(self, n_embd: int, n_head: int, block_size: int):
        super().__init__()
        if n_embd % n_head:
            raise ValueError(f"n_embd {n_embd} is not a multiple of n_head {n_head}")
        self.n_head, self.n_embd, self.head_dim = n_head, n_embd, n_embd // n_head
        self.c_attn = nn.Linear(n_embd, 3 * n_embd)
        self.c_proj = nn.Linear(n_embd, n_embd)
        mask = torch.ones(block_size, block_size).tril()
        self.register_buffer("bias", mask.view(1, 1, block_size, block_size))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, T, C = x.shape
        heads = [t.view(B, T, self.n_head, self.head_dim).transpose(1, 2) for t in self.c_attn(x).split(C, dim=2)]
        q, k, v = heads
        scores = (q @ k.transpose(-2, -1)) * (1.0 / math.sqrt(self.head_dim))
        scores = scores.masked_fill(self.bias[:, :, :T, :T] == 0, float("-inf"))
        y = F.softmax(scores, dim=-1) @ v
        return self.c_proj(y.transpose(1, 2).contiguous().view(B, T, C))


class MLP(nn.Module):
    def __init__(self, n_embd: int):
        super().__init__()
        self.c_fc = nn.Linear(n_embd, 4 * n_embd)
        self.gelu = nn.GELU()
        self.c_proj = nn.Linear(4 * n_embd, n_embd)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.c_proj(self.gelu(self.c_fc(x)))


class Block(nn.Module):
    def __init__(self, n_embd: int, n_head: int, block_size: int):
        super().__init__()
        self.ln_1 = nn.LayerNorm(n_embd)
        self.attn = CausalSelfAttention(n_embd, n_head, block_size)
        self.ln_2 = nn.LayerNorm(n_embd)
        self.mlp = MLP(n_embd)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.attn(self.ln_1(x))
        return x + self.mlp(self.ln_2(x))


class GPT2(nn.Module):
    def __init__(self, vocab_size: int = 50257, block_size: int = 1024, n_layer: int = 12, n_head: int = 12,
                 n_embd: int = 768):
        super().__init__()
        self.block_size = block_size
        self.transformer = nn.ModuleDict(dict(
            wte=nn.Embedding(vocab_size, n_embd),
            wpe=nn.Embedding(block_size, n_embd),
            h=nn.ModuleList(Block(n_embd, n_head, block_size) for _ in range(n_layer)),
            ln_f=nn.LayerNorm(n_embd),
        ))
        self.lm_head = nn.Linear(n_embd, vocab_size, bias=False)
        self.transformer.wte.weight = self.lm_head.weight  # tied

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        T = input_ids.shape[1]
        if T > self.block_size:
            raise ValueError(f"sequence length {T} exceeds block_size {self.block_size}")
        pos = torch.arange(T, device=input_ids.device)
        x = self.transformer.wte(input_ids) + self.transformer.wpe(pos)
        for block in self.transformer.h:
            x = block(x)
        return self.lm_head(self.transformer.ln_f(x))


@torch.no_grad()
def init_weights(model: nn.Module, std: float = 0.02, seed: int = 0) -> nn.Module:
    """Seeded random init: Linear / Embedding weights and Linear biases ~ N(0, std), LayerNorm
    weights 1 + N(0, std) and biases N(0, std) (so every affine path is exercised)."""
    g = torch.Generator(device=next(model.parameters()).device)
    g.manual_seed(seed)
    for m in model.modules():
        if isinstance(m, (nn.Linear, nn.Embedding)):
            m.weight.normal_(0.0, std, generator=g)
            if getattr(m, "bias", None) is not None:
                m.bias.normal_(0.0, std, generator=g)
        elif isinstance(m, nn.LayerNorm):
            m.weight.normal_(1.0, std, generator=g)
            m.bias.normal_(0.0, std, generator=g)
    return model


def build(dtype=torch.float16, device="cuda", seed: int = 0, **kw) -> GPT2:
    """GPT2(**kw) on `device` in `dtype` with the seeded init (the causal mask stays exact ones)."""
    with torch.device(device):
        model = GPT2(**kw).to(dtype)
    return init_weights(model, seed=seed).eval()
