"""The LLaMA-7B-shaped forward with libak355 plugged in, against stock PyTorch.

Model: autokernel_amd.llama.LlamaModel7B (the reference's models/llama_7b.py:164-209 architecture:
32 layers, d 4096, 32 heads / 8 KV heads, FFN 11008, vocab 32000), f16, N(0, 0.02) weights with
seed 0, token ids [1, 2048] uniform in [0, 32000) from seed 42 (verify.py:242-243). Comparison as
verify.py:687-765 does it (NaN / Inf asymmetry fails, allclose on the rest):
  * the reference verify's own swap set (matmul, rmsnorm) is bit-identical to stock;
  * every op but attention swapped is bit-identical to stock;
  * everything swapped (attention too) fails the north star's 1e-2 check against stock (printed):
    the model amplifies one-ulp attention differences past it, as it does between PyTorch's own two
    SDPA backends; asserted is that it is no farther from fp32 than stock f16 is.
Collected after the op-parity files, so a failure here leaves none of them unreached.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model7b(gpu):
    from autokernel_amd import llama, verify
    print("building LlamaModel7B f16 (seed 0)", flush=True)
    model = llama.build("7b", torch.float16, gpu)
    ids = verify.make_token_ids(model, (1, 2048), gpu)
    with torch.no_grad():
        ref = model(ids)
    torch.cuda.synchronize()
    yield model, ids, ref
    del model
    torch.cuda.empty_cache()


def _swapped(model, ids, kinds):
    from autokernel_amd import verify
    with torch.no_grad(), verify.OptimizedModelContext(model, kinds) as m:
        out = m(ids)
    torch.cuda.synchronize()
    return out


def test_llama7b_reference_swap_set_bit_identical(model7b):
    model, ids, ref = model7b
    out = _swapped(model, ids, ["matmul", "rmsnorm"])
    print(f"matmul+rmsnorm vs stock: max |d| {(out.float() - ref.float()).abs().max().item():.3e}", flush=True)
    assert torch.equal(out, ref)


def test_llama7b_all_but_attention_bit_identical(model7b):
    from autokernel_amd import verify
    model, ids, ref = model7b
    kinds = [k for k in verify.ALL_KERNELS if k != "flash_attention"]
    out = _swapped(model, ids, kinds)
    print(f"all but attention vs stock: max |d| {(out.float() - ref.float()).abs().max().item():.3e}", flush=True)
    assert torch.equal(out, ref)


def test_llama7b_all_swapped_as_accurate_as_stock(model7b):
    """Everything swapped, attention included. This forward does NOT pass the north star's check
    against stock (allclose at atol = rtol = 1e-2; printed here and in bench.py's e2e): the model
    amplifies one-ulp attention differences through 32 layers to ~5e-2 in the logits, and stock
    PyTorch's own math SDPA backend fails the same check against its flash backend (printed too).
    Asserted: no NaN / Inf, and the swapped logits are no farther from the same weights run in fp32
    than stock f16's are (+10 %), in max and in mean."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from autokernel_amd import llama, verify
    model, ids, ref = model7b
    out = _swapped(model, ids, verify.ALL_KERNELS)
    cmp = verify.compare_outputs(ref, out, torch.float16, 1e-2, 1e-2)
    print(f"all swapped vs stock (atol = rtol = 1e-2): {cmp['correctness']}, max |d| {cmp['max_abs_error']:.4e}, "
          f"mean |d| {cmp['mean_abs_error']:.4e}", flush=True)
    assert not cmp["opt_has_nan"] and not cmp["opt_has_inf"]
    with torch.no_grad(), sdpa_kernel([SDPBackend.MATH]):
        ref_math = model(ids)
    d_math = (ref_math.float() - ref.float()).abs()
    print(f"stock math SDPA vs stock flash SDPA: max |d| {d_math.max().item():.4e}, mean |d| "
          f"{d_math.mean().item():.4e}", flush=True)
    del ref_math
    m32 = llama.build("7b", torch.float32, ref.device)
    with torch.no_grad():
        for p16, p32 in zip(model.parameters(), m32.parameters()):
            p32.copy_(p16.float())
        out32 = m32(ids).float()
    del m32
    e_stock, e_ak = (ref.float() - out32).abs(), (out.float() - out32).abs()
    print(f"vs fp32: stock max {e_stock.max().item():.4e} mean {e_stock.mean().item():.4e}; libak355 max "
          f"{e_ak.max().item():.4e} mean {e_ak.mean().item():.4e}", flush=True)
    assert e_ak.max() <= 1.1 * e_stock.max() and e_ak.mean() <= 1.1 * e_stock.mean()
