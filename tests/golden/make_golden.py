"""Write the golden fixtures under tests/golden/ from the numpy brute force (oracle/brute.py).

    python tests/golden/make_golden.py

Inputs come from a seeded numpy generator; expected outputs from float64 brute force, or from
the float16 / float32 step-by-step emulations where the reference's per-op rounding is the
point (rmsnorm, rotary embedding). The fixtures pin the torch restatement in oracle/ (CPU tests)
and the HIP kernels (GPU tests). The reference's own tests hold no vectors for this path.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import brute  # noqa: E402


def main() -> None:
    rng = np.random.default_rng(20241201)
    out = {}

    # rmsnorm f16: row 2 holds a value past 255.9 whose square overflows -> rms = inf -> zeros
    x = rng.standard_normal((6, 64)).astype(np.float16)
    x[2, 5] = np.float16(300.0)
    x[4] *= np.float16(40.0)  # large but finite squares
    w = (1.0 + 0.02 * rng.standard_normal(64)).astype(np.float16)
    out["rmsnorm_f16"] = dict(x=x, w=w, y=brute.rmsnorm_steps(x, w, 1e-6), y64=brute.rmsnorm(x, w, 1e-6))
    x32 = rng.standard_normal((5, 96)).astype(np.float32)
    w32 = rng.standard_normal(96).astype(np.float32)
    out["rmsnorm_f32"] = dict(x=x32, w=w32, y64=brute.rmsnorm(x32, w32, 1e-6))

    # rotary f16 / f32 (bit-exact step emulation) with random tables, and theta tables
    for name, dt in (("rope_f16", np.float16), ("rope_f32", np.float32)):
        xr = rng.standard_normal((1, 3, 16, 64)).astype(dt)
        c = rng.standard_normal((16, 32)).astype(dt)
        s = rng.standard_normal((16, 32)).astype(dt)
        out[name] = dict(x=xr, cos=c, sin=s, y=brute.rope_steps(xr, c, s), y64=brute.rope(xr, c, s))

    # softmax (incl. a row with -inf entries and a constant row)
    xs = (3.0 * rng.standard_normal((6, 130))).astype(np.float32)
    xs[1, :7] = -np.inf
    xs[3] = 0.25
    out["softmax_f32"] = dict(x=xs, y64=brute.softmax(xs))
    xh = (3.0 * rng.standard_normal((4, 256))).astype(np.float16)
    out["softmax_f16"] = dict(x=xh, y64=brute.softmax(xh))

    # layernorm
    xl = rng.standard_normal((5, 96)).astype(np.float32) * 2 + 1
    wl = rng.standard_normal(96).astype(np.float32)
    bl = rng.standard_normal(96).astype(np.float32)
    out["layernorm_f32"] = dict(x=xl, w=wl, b=bl, y64=brute.layernorm(xl, wl, bl, 1e-5))

    # cross entropy with an ignored row
    lg = rng.standard_normal((9, 40)).astype(np.float32) * 2
    tg = rng.integers(0, 40, 9).astype(np.int64)
    tg[4] = -100
    out["cross_entropy_f32"] = dict(logits=lg, targets=tg, y64=np.float64(brute.cross_entropy(lg, tg)))
    lg16 = rng.standard_normal((16, 256)).astype(np.float16)
    tg16 = rng.integers(0, 256, 16).astype(np.int64)
    out["cross_entropy_f16"] = dict(logits=lg16, targets=tg16, y64=np.float64(brute.cross_entropy(lg16, tg16)))

    # reductions (max with a NaN row)
    xr = rng.standard_normal((4, 72)).astype(np.float32)
    xr[2, 9] = np.nan
    out["reduce_f32"] = dict(x=xr, sum64=brute.reduce_sum(xr), max=brute.reduce_max(xr))

    # matmul
    A = rng.standard_normal((65, 72)).astype(np.float32)
    B = rng.standard_normal((72, 40)).astype(np.float32)
    out["matmul_f32"] = dict(A=A, B=B, y64=brute.matmul(A, B))
    A16 = rng.standard_normal((64, 128)).astype(np.float16)
    B16 = rng.standard_normal((128, 64)).astype(np.float16)
    out["matmul_f16"] = dict(A=A16, B=B16, y64=brute.matmul(A16, B16))

    # attention f16 [1, 2, 40, 64], causal and not
    Q, K, V = (rng.standard_normal((1, 2, 40, 64)).astype(np.float16) for _ in range(3))
    out["attention_f16"] = dict(Q=Q, K=K, V=V, causal64=brute.attention(Q, K, V, True),
                                full64=brute.attention(Q, K, V, False))

    # fused MLP f32, three activations
    xm = rng.standard_normal((7, 32)).astype(np.float32)
    wg, wu = (0.2 * rng.standard_normal((24, 32))).astype(np.float32), (0.2 * rng.standard_normal((24, 32))).astype(np.float32)
    wd = (0.2 * rng.standard_normal((32, 24))).astype(np.float32)
    out["fused_mlp_f32"] = dict(x=xm, wg=wg, wu=wu, wd=wd,
                                silu64=brute.fused_mlp(xm, wg, wu, wd, "silu"),
                                gelu64=brute.fused_mlp(xm, wg, wu, wd, "gelu"),
                                relu264=brute.fused_mlp(xm, wg, wu, wd, "relu2"))

    # 16-bit fixtures for the ops whose reference computes in fp32 and rounds once (layernorm,
    # reduce sum) or rounds every materialised step (fused MLP). bfloat16 values are stored as
    # float32 arrays (exact); the expected outputs are rounded once from float64.
    for dt, rnd in (("f16", brute.round_f16), ("bf16", brute.round_bf16)):
        xl = rnd(rng.standard_normal((6, 160)) * 2 + 0.5)
        wl, bl = rnd(rng.standard_normal(160)), rnd(rng.standard_normal(160))
        out[f"layernorm_{dt}"] = dict(x=xl, w=wl, b=bl, y=rnd(brute.layernorm(xl, wl, bl, 1e-5)))
        xr = rnd(rng.standard_normal((5, 300)))
        out[f"reduce_{dt}"] = dict(x=xr, sum=rnd(brute.reduce_sum(xr)), max=brute.reduce_max(xr))
        xm = rnd(rng.standard_normal((9, 64)))
        wg, wu, wd = (rnd(0.1 * rng.standard_normal(sh)) for sh in ((48, 64), (48, 64), (64, 48)))
        out[f"fused_mlp_{dt}"] = dict(x=xm, wg=wg, wu=wu, wd=wd,
                                      **{act: brute.fused_mlp_steps(xm, wg, wu, wd, act, dt)
                                         for act in ("silu", "gelu", "relu2")})

    for name, arrays in out.items():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    print(f"wrote {len(out)} fixtures to {HERE}")


if __name__ == "__main__":
    main()
