"""Pin the CPU oracle (oracle/reference_ops.py) before trusting it (CPU only).

Each oracle function is checked against (a) golden fixtures written by the numpy brute force,
(b) fp64 brute force on fresh random inputs, and (c) closed forms, chosen so that a plausible
slip (dropped eps, swapped sign, transposed operand, fp32 instead of f16 rounding) fails. The
last tests plant such slips in copies of the oracle and check that the pins catch them.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import brute
from oracle import reference_ops as R

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def fx(name):
    with np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def close(a, b, atol, rtol):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    assert a.shape == b.shape, (a.shape, b.shape)
    np.testing.assert_allclose(a, b, atol=atol, rtol=rtol, equal_nan=True)


# ------------------------------------------------------------------------- golden fixtures
def test_rmsnorm_golden_f16_bitexact_steps():
    f = fx("rmsnorm_f16")
    y = R.rmsnorm_ref(t(f["x"]), t(f["w"]))
    # torch CPU and the numpy step emulation agree to within one f16 ulp (mean summation order)
    close(y.float().numpy(), f["y"], atol=2e-3, rtol=2e-3)
    # the overflowing row is exactly zero in both (x**2 -> inf -> rms inf -> x / inf = 0)
    assert np.all(f["y"][2] == 0) and torch.all(y[2] == 0)
    # the non-overflowing rows match fp64 mathematics to f16 precision
    rows = [0, 1, 3, 4, 5]
    close(y.float().numpy()[rows], f["y64"][rows], atol=1e-2, rtol=1e-2)


def test_rmsnorm_golden_f32():
    f = fx("rmsnorm_f32")
    close(R.rmsnorm_ref(t(f["x"]), t(f["w"])).numpy(), f["y64"], 1e-5, 1e-5)


@pytest.mark.parametrize("name", ["rope_f16", "rope_f32"])
def test_rope_golden_bitexact(name):
    f = fx(name)
    y = R.rotary_embedding_ref(t(f["x"]), t(f["cos"]), t(f["sin"]))
    assert np.array_equal(y.numpy(), f["y"]), "per-op rounding must match bit for bit"
    tol = 2e-2 if name.endswith("f16") else 1e-5
    close(y.double().numpy(), f["y64"], tol, tol)


@pytest.mark.parametrize("name,tol", [("softmax_f32", 1e-6), ("softmax_f16", 1e-3)])
def test_softmax_golden(name, tol):
    f = fx(name)
    close(R.softmax_ref(t(f["x"])).float().numpy(), f["y64"], tol, tol)


def test_layernorm_golden():
    f = fx("layernorm_f32")
    close(R.layernorm_ref(t(f["x"]), t(f["w"]), t(f["b"])).numpy(), f["y64"], 1e-5, 1e-5)


@pytest.mark.parametrize("name,tol", [("cross_entropy_f32", 1e-6), ("cross_entropy_f16", 1e-2)])
def test_cross_entropy_golden(name, tol):
    f = fx(name)
    y = R.cross_entropy_ref(t(f["logits"]), t(f["targets"]))
    close(y.float().item(), f["y64"], tol, tol)


def test_reduce_golden():
    f = fx("reduce_f32")
    close(R.reduce_sum_ref(t(f["x"])).numpy(), f["sum64"], 1e-5, 1e-5)
    mx = R.reduce_max_ref(t(f["x"])).numpy()
    assert np.array_equal(mx, f["max"], equal_nan=True) and np.isnan(mx[2])


@pytest.mark.parametrize("name,tol", [("matmul_f32", 1e-4), ("matmul_f16", 1e-2)])
def test_matmul_golden(name, tol):
    f = fx(name)
    close(R.matmul_ref(t(f["A"]), t(f["B"])).float().numpy(), f["y64"], tol, tol)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_golden(causal):
    f = fx("attention_f16")
    y = R.flash_attention_ref(t(f["Q"]), t(f["K"]), t(f["V"]), causal=causal)
    close(y.float().numpy(), f["causal64" if causal else "full64"], 1e-2, 1e-2)


@pytest.mark.parametrize("act", ["silu", "gelu", "relu2"])
def test_fused_mlp_golden(act):
    f = fx("fused_mlp_f32")
    y = R.fused_mlp_ref(t(f["x"]), t(f["wg"]), t(f["wu"]), t(f["wd"]), act)
    close(y.numpy(), f[act + "64"], 1e-5, 1e-5)


# ------------------------------------------------------- 16-bit fixtures (one rounding away)
TORCH_DT = {"f16": torch.float16, "bf16": torch.bfloat16}


def ulp_match(out: torch.Tensor, exp: np.ndarray, dt: str, min_equal: float = 0.99):
    """out (a torch 16-bit tensor) against the fixture's once-rounded float64 result: at least
    min_equal of the elements bit-identical, every other one a single rounding step away."""
    e = t(exp).to(TORCH_DT[dt])
    assert out.dtype == e.dtype and out.shape == e.shape, (out.dtype, out.shape, e.shape)
    same = (out == e) | (torch.isnan(out) & torch.isnan(e))
    frac = same.float().mean().item()
    step = 2.0 ** -10 if dt == "f16" else 2.0 ** -7  # relative spacing at the bottom of a binade
    far = (out.double() - e.double()).abs() > step * e.double().abs().clamp_min(2.0 ** -14) * 1.0001
    assert frac >= min_equal, f"only {frac:.2%} bit-identical"
    assert not bool(far[~same].any()), "an element more than one rounding step off"


def test_round_bf16_is_round_half_even_from_float32():
    """brute.round_bf16 agrees with torch's float32 -> bfloat16 conversion (a single rounding) on
    random float32 values and on exact ties (which must go to the even neighbour)."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(100000, generator=g) * 10.0 ** torch.randint(-20, 20, (100000,), generator=g).float()
    ties = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(2.0 + 2 ** -7), 3.0e38, 1.5])
    for v in (x, ties):
        got = t(brute.round_bf16(v.double().numpy()))
        assert torch.equal(got, v.bfloat16().float())


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_layernorm_golden_16bit(dt):
    f = fx(f"layernorm_{dt}")
    x, w, b = (t(f[k]).to(TORCH_DT[dt]) for k in ("x", "w", "b"))
    ulp_match(R.layernorm_ref(x, w, b), f["y"], dt)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_reduce_golden_16bit(dt):
    f = fx(f"reduce_{dt}")
    x = t(f["x"]).to(TORCH_DT[dt])
    ulp_match(R.reduce_sum_ref(x), f["sum"], dt)
    assert torch.equal(R.reduce_max_ref(x), t(f["max"]).to(TORCH_DT[dt]))


@pytest.mark.parametrize("act", ["silu", "gelu", "relu2"])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_fused_mlp_golden_16bit(dt, act):
    f = fx(f"fused_mlp_{dt}")
    x, wg, wu, wd = (t(f[k]).to(TORCH_DT[dt]) for k in ("x", "wg", "wu", "wd"))
    ulp_match(R.fused_mlp_ref(x, wg, wu, wd, act), f[act], dt, min_equal=0.95)


def test_16bit_pins_catch_unrounded_intermediates():
    """A fused MLP that keeps gate / up / the activation in fp32 and rounds only the output fails
    the step-rounded fixture; so does a layernorm whose statistics are taken in the element type."""
    f = fx("fused_mlp_f16")
    x, wg, wu, wd = (t(f[k]).float() for k in ("x", "wg", "wu", "wd"))
    slip = ((torch.nn.functional.silu(x @ wg.T) * (x @ wu.T)) @ wd.T).half()
    with pytest.raises(AssertionError):
        ulp_match(slip, f["silu"], "f16", min_equal=0.95)
    f = fx("layernorm_bf16")
    x, w, b = (t(f[k]).bfloat16() for k in ("x", "w", "b"))
    mu = x.mean(-1, keepdim=True)
    slip = ((x - mu) / torch.sqrt(((x - mu) ** 2).mean(-1, keepdim=True) + 1e-5)) * w + b
    with pytest.raises(AssertionError):
        ulp_match(slip, f["y"], "bf16")


# ----------------------------------------------------------------- fresh fp64 brute force
@pytest.mark.parametrize("seed", [0, 1])
def test_brute_force_random(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(7, 33, generator=g)
    w = torch.randn(33, generator=g)
    b = torch.randn(33, generator=g)
    close(R.softmax_ref(x).numpy(), brute.softmax(x.numpy()), 1e-6, 1e-6)
    close(R.layernorm_ref(x, w, b).numpy(), brute.layernorm(x.numpy(), w.numpy(), b.numpy()), 1e-5, 1e-5)
    close(R.rmsnorm_ref(x, w).numpy(), brute.rmsnorm(x.numpy(), w.numpy()), 1e-5, 1e-5)
    A = torch.randn(9, 33, generator=g)
    close(R.matmul_ref(A, x.T).numpy(), brute.matmul(A.numpy(), x.T.numpy()), 1e-4, 1e-4)
    tg = torch.randint(0, 33, (7,), generator=g)
    close(R.cross_entropy_ref(x, tg).item(), brute.cross_entropy(x.numpy(), tg.numpy()), 1e-6, 1e-6)
    Q, K, V = (torch.randn(2, 3, 11, 8, generator=g) for _ in range(3))
    for causal in (True, False):
        close(R.flash_attention_ref(Q, K, V, causal).numpy(), brute.attention(Q.numpy(), K.numpy(), V.numpy(), causal), 1e-5, 1e-5)
    c, s = torch.randn(11, 4, generator=g), torch.randn(11, 4, generator=g)
    close(R.rotary_embedding_ref(Q, c, s).numpy(), brute.rope(Q.numpy(), c.numpy(), s.numpy()), 1e-5, 1e-5)


# --------------------------------------------------------------------------- closed forms
def test_softmax_closed_forms():
    x = torch.randn(5, 64)
    y = R.softmax_ref(x)
    assert torch.allclose(y.sum(-1), torch.ones(5), atol=1e-6)
    assert torch.allclose(R.softmax_ref(torch.full((2, 50), 3.5)), torch.full((2, 50), 1 / 50))
    assert torch.allclose(R.softmax_ref(x + 100.0), y, atol=1e-6)  # shift invariance
    assert torch.isnan(R.softmax_ref(torch.tensor([[float("inf"), 0.0]]))).all()


def test_norm_closed_forms():
    w = torch.randn(32)
    c = torch.full((3, 32), 2.0)
    # rmsnorm of a constant row c is w * c / sqrt(c^2 + eps)
    assert torch.allclose(R.rmsnorm_ref(c, w), w * 2.0 / math.sqrt(4.0 + 1e-6), atol=1e-6)
    b = torch.randn(32)
    assert torch.allclose(R.layernorm_ref(c, w, b), b.expand(3, 32), atol=1e-5)


def test_rope_closed_forms():
    x = torch.randn(2, 4, 8, 16).half()
    one, zero = torch.ones(8, 8).half(), torch.zeros(8, 8).half()
    assert torch.equal(R.rotary_embedding_ref(x, one, zero), x)  # identity rotation
    y = R.rotary_embedding_ref(x, zero, one)  # quarter turn: (a, b) -> (-b, a)
    assert torch.equal(y[..., 0::2], -x[..., 1::2]) and torch.equal(y[..., 1::2], x[..., 0::2])


def test_cross_entropy_closed_form():
    logits = torch.zeros(6, 1000)
    tg = torch.randint(0, 1000, (6,))
    assert abs(R.cross_entropy_ref(logits, tg).item() - math.log(1000)) < 1e-5
    tg[:] = -100
    assert math.isnan(R.cross_entropy_ref(logits, tg).item())


def test_reduce_closed_forms():
    assert torch.equal(R.reduce_sum_ref(torch.ones(3, 777)), torch.full((3,), 777.0))
    perm = torch.randperm(4096).float().view(1, -1)
    assert R.reduce_max_ref(perm).item() == 4095.0


def test_matmul_identity():
    A = torch.randn(17, 17).half()
    assert torch.equal(R.matmul_ref(A, torch.eye(17).half()), A)


def test_attention_closed_forms():
    Q, K, V = (torch.randn(1, 2, 9, 8) for _ in range(3))
    y = R.flash_attention_ref(Q, K, V, causal=True)
    assert torch.allclose(y[..., 0, :], V[..., 0, :], atol=1e-6)  # row 0 sees only key 0
    y0 = R.flash_attention_ref(Q, K, V, causal=True, sm_scale=0.0)  # uniform weights
    prefix_mean = V.cumsum(-2) / torch.arange(1, 10).view(1, 1, 9, 1)
    assert torch.allclose(y0, prefix_mean, atol=1e-6)


def test_fused_mlp_zero_up():
    x = torch.randn(4, 16)
    wg, wd = torch.randn(8, 16), torch.randn(16, 8)
    assert torch.equal(R.fused_mlp_ref(x, wg, torch.zeros(8, 16), wd), torch.zeros(4, 16))


def test_stage3_overflow_semantics_f16():
    """The reference harness's mixed_scale case: x**2 overflows in f16, rows become exactly 0."""
    x = torch.randn(4, 256).half() * 1000
    y = R.rmsnorm_ref(x, torch.ones(256).half())
    assert torch.all(y == 0)
    Q = torch.randn(1, 1, 16, 64).half() * 1000
    y = R.flash_attention_ref(Q, Q, Q)
    assert torch.isnan(y).any()  # QK^T overflows to inf in f16 -> NaN rows


# ------------------------------------------------------------ planted mistakes must be caught
def _rope_sign_slip(x, cos, sin):
    e, o = x[..., 0::2], x[..., 1::2]
    return torch.stack((e * cos + o * sin, e * sin + o * cos), -1).flatten(-2)


def _rmsnorm_fp32_slip(x, w, eps=1e-6):
    xf = x.float()
    return (xf / torch.sqrt((xf * xf).mean(-1, keepdim=True) + eps) * w.float()).to(x.dtype)


def _softmax_transposed_slip(x):
    return torch.softmax(x, dim=0)


def test_pins_catch_planted_mistakes():
    f = fx("rope_f16")
    assert not np.array_equal(_rope_sign_slip(t(f["x"]), t(f["cos"]), t(f["sin"])).numpy(), f["y"])
    f = fx("rmsnorm_f16")
    slip = _rmsnorm_fp32_slip(t(f["x"]), t(f["w"]))
    assert not torch.all(slip[2] == 0), "fp32 accumulation misses the f16 overflow row"
    f = fx("softmax_f32")
    with pytest.raises(AssertionError):
        close(_softmax_transposed_slip(t(f["x"])).numpy(), f["y64"], 1e-6, 1e-6)
