"""End-to-end plug-in on a small LLaMA-shaped model: every swappable op through libak355."""
from __future__ import annotations

import pytest
import torch

from autokernel_amd import llama, verify

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kinds", [verify.ALL_KERNELS, ("matmul",), ("rmsnorm",), ("rotary_embedding",),
                                   ("flash_attention",), ("fused_mlp",)])
def test_small_llama_all_ops(gpu, kinds):
    torch.manual_seed(0)
    with torch.device(gpu):
        m = llama.LlamaModel(vocab_size=1000, dim=512, n_layers=2, n_heads=8, n_kv_heads=2, hidden_dim=1024,
                             max_seq_len=512).half()
    llama.init_weights(m, seed=1).eval()
    ids = verify.make_token_ids(m, (2, 300), gpu)
    with torch.no_grad():
        ref = m(ids)
        with verify.OptimizedModelContext(m, kinds) as pm:
            out = pm(ids)
    c = verify.compare_outputs(ref, out, torch.float16, 1e-2, 1e-2)
    assert c["correctness"] == "PASS", (kinds, c)
