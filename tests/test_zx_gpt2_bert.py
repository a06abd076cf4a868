"""GPT-2 small and BERT-base at the reference's configurations with libak355 plugged in.

Models: autokernel_amd.gpt2.GPT2 (models/gpt2.py:87-141: 12 x 768, 12 heads, vocab 50257,
explicit-softmax causal attention, exact GELU) on token ids [2, 1024]; autokernel_amd.bert.BertModel
(models/bert_base.py:69-114: 12 x 768, 12 heads, intermediate 3072, non-causal SDPA) on [8, 512];
f16, seeded N(0, 0.02) weights, ids from seed 42. The swap rules are verify.py:557-637 plus
libak355's attention, GELU-MLP and residual-block strategies. Each test asserts:
  * the swaps engage where expected (module counts);
  * the north star's check: allclose to stock at atol = rtol = 1e-2, NaN / Inf only where stock has them;
  * the swapped output is on average no farther from the same weights run in fp32 than stock f16
    is (+10 %); the largest deviations are printed beside stock's.
Collected after the op-parity files.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _fp32_copy(build, model):
    m32 = build(torch.float32, next(model.parameters()).device)
    with torch.no_grad():
        for p16, p32 in zip(model.parameters(), m32.parameters()):
            p32.copy_(p16.float())
    return m32


def _report(name, ref, out, out32):
    from autokernel_amd import verify
    cmp = verify.compare_outputs(ref, out, torch.float16, 1e-2, 1e-2)
    e_stock = (ref.float() - out32).abs()
    e_ak = (out.float() - out32).abs()
    print(f"{name}: vs stock (1e-2) {cmp['correctness']} max |d| {cmp['max_abs_error']:.4e} mean "
          f"{cmp['mean_abs_error']:.4e}; vs fp32 stock max {e_stock.max().item():.4e} mean {e_stock.mean().item():.4e}, "
          f"libak355 max {e_ak.max().item():.4e} mean {e_ak.mean().item():.4e}", flush=True)
    assert cmp["correctness"] == "PASS", (name, cmp)
    assert e_ak.mean() <= 1.1 * e_stock.mean(), name
    return cmp


def test_gpt2_small_plugged_in(gpu):
    from autokernel_amd import gpt2, verify
    print("building GPT-2 small f16", flush=True)
    model = gpt2.build(torch.float16, gpu)
    ids = verify.make_token_ids(model, (2, 1024), gpu)
    with torch.no_grad():
        ref = model(ids)
        out32 = _fp32_copy(gpt2.build, model)(ids).float()
    ctx = verify.OptimizedModelContext(model, verify.ALL_KERNELS)
    with torch.no_grad(), ctx as m:
        out = m(ids)
    assert ctx.applied == {"attention": 12, "gelu_mlp": 12, "matmul": 1, "layernorm": 25,
                           "residual_block": 12}, ctx.applied
    _report("GPT-2 all swapped", ref, out, out32)
    with torch.no_grad(), verify.OptimizedModelContext(model, ["matmul", "layernorm"]) as m:
        out_ref_set = m(ids)
    _report("GPT-2 matmul + layernorm (the reference verify's swap set)", ref, out_ref_set, out32)


def test_bert_base_plugged_in(gpu):
    from autokernel_amd import bert, verify
    print("building BERT-base f16", flush=True)
    model = bert.build(torch.float16, gpu)
    ids = verify.make_token_ids(model, (8, 512), gpu)
    with torch.no_grad():
        ref_h, ref = model.encode(ids), model(ids)
        m32 = _fp32_copy(bert.build, model)
        h32, out32 = m32.encode(ids).float(), m32(ids).float()
    ctx = verify.OptimizedModelContext(model, verify.ALL_KERNELS)
    with torch.no_grad(), ctx as m:
        out_h, out = m.encode(ids), m(ids)
    assert ctx.applied == {"attention": 12, "gelu_mlp": 12, "matmul": 1, "layernorm": 25,
                           "residual_block": 12}, ctx.applied
    _report("BERT all swapped, hidden states", ref_h, out_h, h32)
    _report("BERT all swapped, pooled output", ref, out, out32)
