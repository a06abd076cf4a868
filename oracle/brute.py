"""Independent numpy restatements that pin oracle.reference_ops (test infrastructure only).

Two kinds:
  * float64 brute force of the mathematics (any input dtype, compared with a tolerance);
  * float16 / float32 step-by-step emulations of the reference's op sequence for the ops whose
    per-op rounding is the point (rmsnorm: x**2 rounds and may overflow before the mean;
    rotary embedding: every product and sum rounds). numpy's float16 arithmetic rounds each
    operation to binary16 exactly like a torch f16 tensor op, so these are bit-comparable.
No torch import: these share no code with the thing they check.
"""
from __future__ import annotations

import math

import numpy as np

try:
    from scipy.special import erf as _erf
except Exception:  # pragma: no cover - scipy is present in this image
    _erf = np.vectorize(math.erf)


def f64(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float64)


# ------------------------------------------------------------------------------------- float64
def matmul(A, B):
    return f64(A) @ f64(B)


def softmax(x, axis=-1):
    x = f64(x)
    m = np.max(x, axis=axis, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=axis, keepdims=True)


def layernorm(x, w, b, eps=1e-5):
    x = f64(x)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    y = (x - mu) / np.sqrt(var + eps)
    if w is not None:
        y = y * f64(w)
    if b is not None:
        y = y + f64(b)
    return y


def rmsnorm(x, w, eps=1e-6):
    x = f64(x)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * f64(w)


def rope(x, cos, sin):
    x = f64(x)
    e, o = x[..., 0::2], x[..., 1::2]
    c, s = f64(cos), f64(sin)
    out = np.empty(np.broadcast_shapes(e.shape, c.shape)[:-1] + (x.shape[-1],))
    out[..., 0::2] = e * c - o * s
    out[..., 1::2] = e * s + o * c
    return out


def cross_entropy(logits, targets, ignore_index=-100):
    x = f64(logits).reshape(-1, np.shape(logits)[-1])
    t = np.asarray(targets).reshape(-1)
    m = x.max(-1)
    lse = m + np.log(np.exp(x - m[:, None]).sum(-1))
    keep = t != ignore_index
    rows = np.nonzero(keep)[0]
    if rows.size == 0:
        return float("nan")
    return float(np.mean(lse[rows] - x[rows, t[rows]]))


def reduce_sum(x, axis=-1):
    return f64(x).sum(axis)


def reduce_max(x, axis=-1):
    return np.max(np.asarray(x), axis=axis)


def attention(Q, K, V, causal=True, sm_scale=None):
    Q, K, V = f64(Q), f64(K), f64(V)
    if sm_scale is None:
        sm_scale = Q.shape[-1] ** -0.5
    s = (Q @ np.swapaxes(K, -1, -2)) * sm_scale
    if causal:
        sq, sk = Q.shape[-2], K.shape[-2]
        s = np.where(np.triu(np.ones((sq, sk), dtype=bool), 1), -np.inf, s)
    return softmax(s) @ V


def gelu_erf(x):
    x = f64(x)
    return 0.5 * x * (1.0 + _erf(x / math.sqrt(2.0)))


def fused_mlp(x, wg, wu, wd, activation="silu"):
    x = f64(x)
    g = x @ f64(wg).T
    u = x @ f64(wu).T
    if activation == "silu":
        g = g / (1.0 + np.exp(-g))
    elif activation == "gelu":
        g = gelu_erf(g)
    elif activation == "relu2":
        g = np.maximum(g, 0.0) ** 2
    return (g * u) @ f64(wd).T


# ----------------------------------------------------------- step-by-step rounding emulations
def rmsnorm_steps(x, w, eps=1e-6):
    """reference.py:28-29 step by step in x's numpy dtype (float16 or float32).

    x**2 rounds (float16 overflows to inf past 255.9), the mean accumulates the rounded squares in
    float64 and rounds once, then + eps, sqrt, divide and multiply each round.
    """
    x = np.asarray(x)
    dt = x.dtype.type
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        sq = (x * x).astype(dt)
        ms = dt(1) * (sq.astype(np.float64).sum(-1, keepdims=True) / x.shape[-1]).astype(dt)
        t = (ms.astype(np.float32) + np.float32(eps)).astype(dt)
        rms = np.sqrt(t.astype(np.float32)).astype(dt)
        q = (x.astype(np.float32) / rms.astype(np.float32)).astype(dt)
        return (q.astype(np.float32) * np.asarray(w).astype(np.float32)).astype(dt)


def rope_steps(x, cos, sin):
    """reference.py:65-69 step by step in the numpy dtype of x (float16 / float32): bit-exact."""
    x = np.asarray(x)
    dt = x.dtype.type
    c, s = np.asarray(cos).astype(dt), np.asarray(sin).astype(dt)
    e, o = x[..., 0::2], x[..., 1::2]
    with np.errstate(over="ignore", invalid="ignore"):
        a = (e * c).astype(dt) - (o * s).astype(dt)
        b = (e * s).astype(dt) + (o * c).astype(dt)
    out = np.empty(a.shape[:-1] + (x.shape[-1],), dtype=dt)
    out[..., 0::2] = a.astype(dt)
    out[..., 1::2] = b.astype(dt)
    return out


# ---------------------------------------------------------------- rounding to 16-bit types
def round_f16(a) -> np.ndarray:
    """float64 -> nearest float16 (round half to even), held as float16."""
    return f64(a).astype(np.float16)


def round_bf16(a) -> np.ndarray:
    """float64 -> nearest bfloat16 (8 significant bits, round half to even, overflow to inf), held as
    float32 (every bfloat16 value is a float32). Rounds once from float64: no float32 step, so no
    double rounding."""
    x = f64(a)
    with np.errstate(over="ignore", invalid="ignore"):
        m, e = np.frexp(x)                      # x = m * 2**e, |m| in [0.5, 1)
        r = np.ldexp(np.rint(m * 256.0), e - 8)  # 8 significant bits, rint is half-to-even
        r = np.where(np.abs(r) > 3.3895313892515355e38, np.copysign(np.inf, x), r)
    r = np.where(np.isfinite(x), r, x)
    return r.astype(np.float32)


ROUND = {"f16": round_f16, "bf16": round_bf16}


def fused_mlp_steps(x, wg, wu, wd, activation="silu", dtype="f16"):
    """reference.py:47-55 with each materialised tensor rounded to `dtype` ("f16" / "bf16"): gate,
    up, the activation, the product and the output; every product and activation is evaluated in
    float64 from the rounded inputs, then rounded once."""
    rnd = ROUND[dtype]
    x = f64(x)
    g = f64(rnd(x @ f64(wg).T))
    u = f64(rnd(x @ f64(wu).T))
    if activation == "silu":
        a = g / (1.0 + np.exp(-g))
    elif activation == "gelu":
        a = gelu_erf(g)
    elif activation == "relu2":
        a = f64(rnd(np.maximum(g, 0.0))) ** 2
    else:
        a = g
    a = f64(rnd(a))
    h = f64(rnd(a * u))
    return rnd(h @ f64(wd).T)
