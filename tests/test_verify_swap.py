"""Module swapping of the plug-in verifier on a tiny LLaMA (CPU: structure only, no forward)."""
from __future__ import annotations

import torch.nn as nn

from autokernel_amd import llama, verify


def tiny():
    return llama.LlamaModel(vocab_size=100, dim=128, n_layers=2, n_heads=2, n_kv_heads=1, hidden_dim=256, max_seq_len=16)


def test_all_strategies_apply_and_restore():
    m = tiny()
    before = {n: type(x) for n, x in m.named_modules()}
    ctx = verify.OptimizedModelContext(m, verify.ALL_KERNELS)
    with ctx as pm:
        assert ctx.applied == {"attention": 2, "fused_mlp": 2, "matmul": 1, "rmsnorm": 5, "residual_block": 2}
        assert isinstance(pm.layers[0], verify.ResidualBlockWrapper)
        assert isinstance(pm.layers[0].original.attention, verify.AttentionWrapper)
        assert isinstance(pm.layers[1].original.feed_forward, verify.FeedForwardWrapper)
        assert isinstance(pm.output, verify.LinearWrapper)
        assert isinstance(pm.norm, verify.RMSNormWrapper)
    assert {n: type(x) for n, x in m.named_modules()} == before


def test_residual_blocks_need_swapped_branches():
    """The residual fusion engages only where both branches are libak355 wrappers with GEMMs."""
    for kinds, blocks in ((("matmul", "fused_mlp", "rotary_embedding"), 2), (("matmul", "fused_mlp"), 0),
                          (("fused_mlp", "flash_attention"), 0), (("matmul", "flash_attention"), 0)):
        m = tiny()
        ctx = verify.OptimizedModelContext(m, kinds)
        with ctx:
            assert ctx.applied.get("residual_block", 0) == blocks, kinds


def test_matmul_only_swaps_every_linear():
    m = tiny()
    ctx = verify.OptimizedModelContext(m, ["matmul"])
    with ctx:
        assert ctx.applied == {"matmul": 2 * 7 + 1}
        assert all(not isinstance(x, nn.Linear) or n.endswith(".original") for n, x in m.named_modules())


def test_unknown_strategy_rejected():
    import pytest
    with pytest.raises(ValueError):
        verify.OptimizedModelContext(tiny(), ["conv2d"])


def test_compare_outputs_rules():
    import torch
    a = torch.randn(4, 8)
    assert verify.compare_outputs(a, a.clone(), torch.float32)["correctness"] == "PASS"
    b = a.clone()
    b[0, 0] = float("nan")
    assert verify.compare_outputs(a, b, torch.float32)["correctness"] == "FAIL"
    assert verify.compare_outputs(b, b.clone(), torch.float32)["correctness"] == "PASS"  # NaN in both
    assert verify.compare_outputs(a, a + 1, torch.float32, 1e-2, 1e-2)["correctness"] == "FAIL"


class _EncoderAttention(nn.Module):
    """BERT-shaped self-attention (separate query / key / value / out_proj, no mask by default)."""

    def __init__(self, dim, heads):
        super().__init__()
        self.num_heads, self.head_dim = heads, dim // heads
        self.query, self.key, self.value, self.out_proj = (nn.Linear(dim, dim) for _ in range(4))
        self.dropout = nn.Dropout(0.0)

    def forward(self, x, attention_mask=None):
        import torch.nn.functional as F
        B, T, C = x.shape
        q, k, v = (lin(x).view(B, T, self.num_heads, self.head_dim).transpose(1, 2)
                   for lin in (self.query, self.key, self.value))
        y = F.scaled_dot_product_attention(q, k, v, attn_mask=attention_mask)
        return self.dropout(self.out_proj(y.transpose(1, 2).reshape(B, T, C)))


class _EncoderLayer(nn.Module):
    """Post-LayerNorm encoder layer (x = norm(x + sublayer(x))): no pre-norm residual fusion applies."""

    def __init__(self, dim, heads):
        super().__init__()
        self.attention, self.norm1 = _EncoderAttention(dim, heads), nn.LayerNorm(dim)
        self.mlp = nn.Sequential(nn.Linear(dim, 4 * dim), nn.GELU(), nn.Linear(4 * dim, dim))
        self.norm2 = nn.LayerNorm(dim)

    def forward(self, x):
        x = self.norm1(x + self.attention(x))
        return self.norm2(x + self.mlp(x))


def test_encoder_attention_strategy_applies_and_restores():
    m = nn.Sequential(_EncoderLayer(64, 4), _EncoderLayer(64, 4))
    before = {n: type(x) for n, x in m.named_modules()}
    ctx = verify.OptimizedModelContext(m, verify.ALL_KERNELS)
    with ctx:
        assert ctx.applied == {"attention": 2, "matmul": 4, "layernorm": 4}, ctx.applied
        assert isinstance(m[0].attention, verify.EncoderAttentionWrapper)
        assert isinstance(m[1].mlp[0], verify.LinearWrapper)
    assert {n: type(x) for n, x in m.named_modules()} == before


class _Gpt2Attention(nn.Module):
    """GPT-2-shaped causal attention: fused c_attn, explicit tril mask buffer, materialised scores."""

    def __init__(self, dim, heads, block, causal=True):
        super().__init__()
        self.n_head, self.n_embd = heads, dim
        self.c_attn, self.c_proj = nn.Linear(dim, 3 * dim), nn.Linear(dim, dim)
        self.attn_dropout, self.resid_dropout = nn.Dropout(0.0), nn.Dropout(0.0)
        import torch
        m = torch.ones(block, block)
        self.register_buffer("bias", (m.tril() if causal else m).view(1, 1, block, block))

    def forward(self, x):
        import math
        import torch
        B, T, C = x.shape
        q, k, v = (t.view(B, T, self.n_head, C // self.n_head).transpose(1, 2) for t in self.c_attn(x).split(C, 2))
        att = (q @ k.transpose(-2, -1).contiguous()) * (1.0 / math.sqrt(C // self.n_head))
        att = att.masked_fill(self.bias[:, :, :T, :T] == 0, float("-inf"))
        att = self.attn_dropout(torch.softmax(att.float(), dim=-1).to(x.dtype))
        return self.resid_dropout(self.c_proj((att @ v).transpose(1, 2).reshape(B, T, C)))


def test_fused_qkv_causal_attention_strategy():
    m = nn.ModuleList([_Gpt2Attention(64, 4, 32), _Gpt2Attention(64, 4, 32, causal=False)])
    before = {n: type(x) for n, x in m.named_modules()}
    ctx = verify.OptimizedModelContext(m, verify.ALL_KERNELS)
    with ctx:
        assert isinstance(m[0], verify.FusedQKVAttentionWrapper)
        assert not isinstance(m[1], verify.FusedQKVAttentionWrapper), "a non-causal mask must not be swapped"
        assert ctx.applied == {"attention": 1, "matmul": 2}, ctx.applied
    assert {n: type(x) for n, x in m.named_modules()} == before
