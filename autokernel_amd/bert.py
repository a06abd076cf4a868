"""BERT-base for the plug-in check: the reference's models/bert_base.py architecture.

Architecture (models/bert_base.py:16-114): word, position and token-type embeddings summed and
layer-normalised; per layer a bidirectional self-attention (query / key / value / out_proj
Linears, num_heads, F.scaled_dot_product_attention without a causal mask), then a post-LayerNorm
residual norm1(x + attention(x)), a GELU MLP (dense1 -> exact-erf GELU -> dense2) and
norm2(x + mlp(x)); the output is the pooled first token, tanh(pooler(x[:, 0])). Module and
attribute names follow the reference, so the same module-swapping plug-in applies to both.

This is stock PyTorch: the baseline autokernel_amd.verify replaces piece by piece. BertModel():
vocab 30522, hidden 768, 12 layers, 12 heads, intermediate 3072, 512 positions (110 M parameters).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


class BertSelfAttention(nn.Module):
    def __init__(self, hidden_size: int, num_heads: int):
        super().__init__()
        if hidden_size % num_heads:
            raise ValueError(f"hidden_size {hidden_size} is not a multiple of num_heads {num_heads}")
        self.num_heads, self.head_dim = num_heads, hidden_size // num_heads
        self.query = nn.Linear(hidden_size, hidden_size)
        self.key = nn.Linear(hidden_size, hidden_size)
        self.value = nn.Linear(hidden_size, hidden_size)
        self.out_proj = nn.Linear(hidden_size, hidden_size)

    def forward(self, x: torch.Tensor, attention_mask: torch.Tensor | None = None) -> torch.Tensor:
        B, T, C = x.shape

        def heads(lin):
            return lin(x).view(B, T, self.num_heads, self.head_dim).transpose(1, 2)
        y = F.scaled_dot_product_attention(heads(self.query), heads(self.key), heads(self.value),
                                           attn_mask=attention_mask)
        return self.out_proj(y.transpose(1, 2).contiguous().view(B, T, C))


class BertMLP(nn.Module):
    def __init__(self, hidden_size: int, intermediate_size: int):
        super().__init__()
        self.dense1 = nn.Linear(hidden_size, intermediate_size)
        self.dense2 = nn.Linear(intermediate_size, hidden_size)
        self.gelu = nn.GELU()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.dense2(self.gelu(self.dense1(x)))


class BertLayer(nn.Module):
    def __init__(self, hidden_size: int, num_heads: int, intermediate_size: int):
        super().__init__()
        self.attention = BertSelfAttention(hidden_size, num_heads)
        self.norm1 = nn.LayerNorm(hidden_size)
        self.mlp = BertMLP(hidden_size, intermediate_size)
        self.norm2 = nn.LayerNorm(hidden_size)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.norm1(x + self.attention(x))
        return self.norm2(x + self.mlp(x))


class BertModel(nn.Module):
    def __init__(self, vocab_size: int = 30522, hidden_size: int = 768, num_layers: int = 12, num_heads: int = 12,
                 intermediate_size: int = 3072, max_seq_len: int = 512):
        super().__init__()
        self.word_embeddings = nn.Embedding(vocab_size, hidden_size)
        self.position_embeddings = nn.Embedding(max_seq_len, hidden_size)
        self.token_type_embeddings = nn.Embedding(2, hidden_size)
        self.embed_norm = nn.LayerNorm(hidden_size)
        self.layers = nn.ModuleList(BertLayer(hidden_size, num_heads, intermediate_size) for _ in range(num_layers))
        self.pooler = nn.Linear(hidden_size, hidden_size)

    def encode(self, input_ids: torch.Tensor) -> torch.Tensor:
        """The last layer's hidden states [B, T, hidden]."""
        T = input_ids.shape[1]
        pos = torch.arange(T, device=input_ids.device).unsqueeze(0)
        x = (self.word_embeddings(input_ids) + self.position_embeddings(pos)
             + self.token_type_embeddings(torch.zeros_like(input_ids)))
        x = self.embed_norm(x)
        for layer in self.layers:
            x = layer(x)
        return x

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return torch.tanh(self.pooler(self.encode(input_ids)[:, 0]))


@torch.no_grad()
def init_weights(model: nn.Module, std: float = 0.02, seed: int = 0) -> nn.Module:
    """Seeded random init: Linear / Embedding weights and Linear biases ~ N(0, std), LayerNorm
    weights 1 + N(0, std) and biases N(0, std)."""
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


def build(dtype=torch.float16, device="cuda", seed: int = 0, **kw) -> BertModel:
    with torch.device(device):
        model = BertModel(**kw).to(dtype)
    return init_weights(model, seed=seed).eval()
