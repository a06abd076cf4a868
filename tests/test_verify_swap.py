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


# ------------------------------------------------------------------ external kernel modules
FAKE_LN = '''
import torch
KERNEL_TYPE = "layernorm"
CALLS = []
def kernel_fn(x, weight, bias, eps=1e-5):
    CALLS.append(tuple(x.shape))
    return torch.nn.functional.layer_norm(x, x.shape[-1:], weight, bias, eps)
'''
FAKE_MM = '''
import torch
KERNEL_TYPE = "matmul"
def kernel_fn(A, B):
    assert B.is_contiguous()          # the reference hands over weight.t().contiguous()
    return A @ B
'''
FAKE_RMS_NO_EPS = '''
import torch
def kernel_fn(x, weight):             # no eps parameter: the wrapper's TypeError fallback
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * weight
'''


def _write(d, name, text):
    p = d / name
    p.write_text(text)
    return str(p)


def test_discovery_by_file_name(tmp_path):
    for n in ("kernel_flash_attention_1_optimized.py", "kernel_matmul_12_optimized.py",
              "kernel_layernorm_3_optimized.py", "notes.py", "kernel_x_optimized.py"):
        _write(tmp_path, n, "def kernel_fn(*a):\n    return None\n")
    found = verify.discover_optimized_kernels(str(tmp_path))
    got = [(r.kernel_type, r.rank, r.speedup) for r in found]
    assert got == [("flash_attention", 1, 0.0), ("layernorm", 3, 0.0), ("matmul", 12, 0.0)]


def test_discovery_from_orchestration_state(tmp_path):
    import json
    _write(tmp_path, "kernel_matmul_1_optimized.py", FAKE_MM)
    _write(tmp_path, "op7_optimized.py", FAKE_LN)
    _write(tmp_path, "kernel_rmsnorm_2_optimized.py", FAKE_RMS_NO_EPS)
    state = {"kernels": [
        {"op_type": "matmul", "rank": 1, "speedup": 1.8},                       # conventional name
        {"type": "layernorm", "rank": 4, "best_speedup": 1.2, "file": "k/op7.py"},  # from "file"
        {"op_type": "rmsnorm", "rank": 2, "speedup": 0.9},                      # no speedup: dropped
        {"op_type": "softmax", "rank": 3, "speedup": 2.0},                      # file missing: dropped
    ]}
    (tmp_path / "orchestration_state.json").write_text(json.dumps(state))
    found = verify.discover_optimized_kernels(str(tmp_path))
    assert [(r.kernel_type, r.rank, r.speedup) for r in found] == [("matmul", 1, 1.8), ("layernorm", 4, 1.2)]
    assert found[1].optimized_path.endswith("op7_optimized.py")


def test_external_modules_swap_and_restore(tmp_path):
    """External kernel_fns replace nn.Linear / nn.LayerNorm / RMSNorm modules with the reference's
    call conventions; the forward equals stock; everything is restored on exit."""
    import torch
    ln = _write(tmp_path, "kernel_layernorm_1_optimized.py", FAKE_LN)
    mm = _write(tmp_path, "kernel_matmul_2_optimized.py", FAKE_MM)
    rms = _write(tmp_path, "kernel_rmsnorm_3_optimized.py", FAKE_RMS_NO_EPS)
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(16, 32), nn.LayerNorm(32), nn.Linear(32, 8, bias=False),
                          llama.RMSNorm(8)).eval()
    x = torch.randn(3, 5, 16)
    with torch.no_grad():
        ref = model(x)
    before = {n: type(m) for n, m in model.named_modules()}
    reps = [verify.replacement_from_module(p) for p in (ln, mm)] + verify.discover_optimized_kernels(str(tmp_path))[2:]
    ctx = verify.OptimizedModelContext(model, reps)
    with ctx as m, torch.no_grad():
        assert ctx.applied == {"matmul": 2, "layernorm": 1, "rmsnorm": 1}
        assert isinstance(m[0], verify.ModuleLinearWrapper) and isinstance(m[1], verify.ModuleLayerNormWrapper)
        assert isinstance(m[3], verify.ModuleRMSNormWrapper)
        out = m(x)
        calls = ctx.external["layernorm"].module_fn.__globals__["CALLS"]
        assert calls == [(15, 32)]  # called on the [rows, cols] view
    torch.testing.assert_close(out, ref, atol=1e-5, rtol=1e-5)
    assert {n: type(m) for n, m in model.named_modules()} == before


def test_external_module_notes_and_precedence(tmp_path):
    """Unsupported external types are noted and skipped; an external matmul wins over the
    libak355 matmul strategy; a module without kernel_fn is noted at load."""
    mm = _write(tmp_path, "kernel_matmul_1_optimized.py", FAKE_MM)
    bad = _write(tmp_path, "kernel_layernorm_1_optimized.py", "KERNEL_TYPE = 'layernorm'\n")
    sm = verify.KernelReplacement("softmax", 1, 2.0, mm)
    m = tiny()
    ctx = verify.OptimizedModelContext(m, ["matmul", "rmsnorm", verify.replacement_from_module(mm), sm,
                                           verify.KernelReplacement("layernorm", 1, 0.0, bad)])
    with ctx:
        assert ctx.applied["matmul"] == 2 * 7 + 1 and ctx.applied["rmsnorm"] == 5
        assert all(isinstance(w, verify.ModuleLinearWrapper) for n, w in m.named_modules() if n == "output")
    assert any("softmax" in n for n in ctx.notes)
    assert any("no kernel_fn" in n for n in ctx.notes)


def test_gpt2_and_bert_strategies_apply_and_restore():
    """The reference's GPT-2 and BERT architectures (small instances, CPU, no forward): the
    attention strategies, every remaining Linear and every LayerNorm are swapped and restored."""
    from autokernel_amd import bert, gpt2
    for model, attn in ((gpt2.GPT2(vocab_size=64, block_size=32, n_layer=2, n_head=2, n_embd=64),
                         verify.FusedQKVAttentionWrapper),
                        (bert.BertModel(vocab_size=64, hidden_size=64, num_layers=2, num_heads=2,
                                        intermediate_size=128, max_seq_len=32), verify.EncoderAttentionWrapper)):
        before = {n: type(x) for n, x in model.named_modules()}
        ctx = verify.OptimizedModelContext(model, verify.ALL_KERNELS)
        with ctx as m:
            assert ctx.applied == {"attention": 2, "gelu_mlp": 2, "matmul": 1, "layernorm": 5,
                                   "residual_block": 2}, (type(model), ctx.applied)
            assert sum(isinstance(x, attn) for x in m.modules()) == 2
        assert {n: type(x) for n, x in model.named_modules()} == before


def test_fused_qkv_weight_follows_weight_updates():
    """The fused [wq; wk; wv] copy is rebuilt when a source weight changes in place or is replaced."""
    import torch
    m = tiny()
    with verify.OptimizedModelContext(m, verify.ALL_KERNELS) as pm:
        wrap = pm.layers[0].original.attention
        att = wrap.original
        w0 = wrap.w_qkv
        assert torch.equal(w0, torch.cat([att.wq.weight, att.wk.weight, att.wv.weight]))
        assert wrap.w_qkv is w0                      # unchanged weights: no rebuild
        with torch.no_grad():
            att.wk.weight.add_(1.0)                  # in-place update
        w1 = wrap.w_qkv
        assert w1 is not w0 and torch.equal(w1[att.wq.weight.shape[0]:][:att.wk.weight.shape[0]], att.wk.weight)
        att.wv.weight = torch.nn.Parameter(torch.zeros_like(att.wv.weight))   # replaced
        assert torch.count_nonzero(wrap.w_qkv[-att.wv.weight.shape[0]:]) == 0


def test_encoder_fused_qkv_follows_parameter_updates():
    """BERT-style attention's concatenated [query; key; value] weight and bias are rebuilt when a
    source weight or bias changes in place or is replaced, and reused otherwise."""
    import torch
    from autokernel_amd import bert
    model = bert.BertModel(vocab_size=64, hidden_size=64, num_layers=1, num_heads=2, intermediate_size=128,
                           max_seq_len=32)
    with verify.OptimizedModelContext(model, verify.ALL_KERNELS) as m:
        wrap = next(x for x in m.modules() if isinstance(x, verify.EncoderAttentionWrapper))
        att = wrap.original
        assert wrap.fused_qkv
        w0, b0 = wrap._qkv_params()
        assert torch.equal(w0, torch.cat([att.query.weight, att.key.weight, att.value.weight]))
        assert torch.equal(b0, torch.cat([att.query.bias, att.key.bias, att.value.bias]))
        assert wrap._qkv_params()[0] is w0                 # unchanged parameters: no rebuild
        with torch.no_grad():
            att.key.bias.add_(1.0)                         # in-place update of a bias
        w1, b1 = wrap._qkv_params()
        assert w1 is not w0 and torch.equal(b1[64:128], att.key.bias)
        att.value.weight = torch.nn.Parameter(torch.zeros_like(att.value.weight))   # replaced
        assert torch.count_nonzero(wrap._qkv_params()[0][128:]) == 0



def test_gpt2_and_bert_blocks_carry_their_residuals():
    """GPT-2's pre-norm Block and BERT's post-norm layer: with flash attention and matmul swapped, each
    block hands its residual adds to the GEMMs that end its branches and the GELU MLPs become two
    fused-epilogue GEMMs; without flash attention only the MLPs are fused."""
    from autokernel_amd import bert, gpt2
    # Linears outside the MLPs: GPT-2 c_attn + c_proj per block and lm_head; BERT four per layer and the pooler
    for model, blocks, wrapper, linears in (
            (gpt2.GPT2(vocab_size=64, block_size=32, n_layer=2, n_head=2, n_embd=64), "transformer.h",
             verify.GPT2BlockWrapper, 2 * 2 + 1),
            (bert.BertModel(vocab_size=64, hidden_size=64, num_layers=2, num_heads=2, intermediate_size=128,
                            max_seq_len=32), "layers", verify.PostNormBlockWrapper, 4 * 2 + 1)):
        before = {n: type(x) for n, x in model.named_modules()}
        with verify.OptimizedModelContext(model, verify.ALL_KERNELS):
            blk = model.get_submodule(blocks)
            assert all(isinstance(b, wrapper) for b in blk)
            assert all(isinstance(b.original.mlp, verify.GeluMLPWrapper) for b in blk)
        assert {n: type(x) for n, x in model.named_modules()} == before
        ctx = verify.OptimizedModelContext(model, ["matmul", "layernorm"])
        with ctx:
            assert ctx.applied == {"gelu_mlp": 2, "matmul": linears, "layernorm": 5}, ctx.applied
        assert {n: type(x) for n, x in model.named_modules()} == before
