"""Rotary-embedding drop-in: kernel_fn(x, cos, sin).

Mirrors reference.py:63-69 (interleaved pairs, cos / sin of shape [..., D/2] broadcast against
x[..., ::2]) and kernels/rotary_embedding.py:75. The table row of each x row is found from the
broadcast pattern without copying for the two layouts models use:
  * cos [S, D/2] (or with leading 1s) against x [..., S, D]        -> row r uses r % S
  * cos [S, 1, D/2] (or [1, S, 1, D/2]) against x [..., S, H, D]    -> row r uses (r // H) % S
Other broadcasts are expanded to one table row per x row. Mixed dtypes follow torch type
promotion (all operands are cast to the promoted dtype, which is exact). Runs ak_rope (rope.hip).
"""
from __future__ import annotations

import torch

from .. import _lib
from ._common import device_guard

KERNEL_TYPE = "rotary_embedding"


def _table_plan(xs: tuple, cs: tuple) -> tuple[int, int] | None:
    """(table_rows, rep_inner) when cos of shape cs indexes rows of x (shape xs[:-1]) cheaply."""
    lead = list(cs[:-1])
    while lead and lead[0] == 1:
        lead.pop(0)
    rows_shape = list(xs[:-1])
    if not lead:
        return 1, 1
    if len(lead) == 1 and rows_shape and rows_shape[-1] == lead[0]:
        return lead[0], 1
    if len(lead) == 2 and lead[1] == 1 and len(rows_shape) >= 2 and rows_shape[-2] == lead[0]:
        return lead[0], rows_shape[-1]
    return None


def kernel_fn(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    _lib.require_gpu("rotary_embedding", x, cos, sin)
    dt = torch.promote_types(torch.promote_types(x.dtype, cos.dtype), sin.dtype)
    xx, cc, ss = (t if t.dtype == dt else t.to(dt) for t in (x, cos, sin))
    code = _lib.dtype_code(xx, "rotary_embedding")
    d = xx.shape[-1]
    if d % 2:
        raise ValueError(f"rotary_embedding: head_dim {d} is odd")
    half = d // 2
    out_shape = torch.broadcast_shapes(xx.shape[:-1] + (half,), cc.shape, ss.shape)
    if out_shape[:-1] != xx.shape[:-1] or out_shape[-1] != half:
        # cos / sin add leading dims: x broadcasts up to the table's shape
        xx = xx.expand(*out_shape[:-1], d)
    xs = tuple(xx.shape)
    if cc.shape != ss.shape:
        cc, ss = torch.broadcast_tensors(cc, ss)
    plan = _table_plan(xs, tuple(cc.shape))
    if plan is None:
        cc = cc.expand(*xs[:-1], half)
        ss = ss.expand(*xs[:-1], half)
        plan = (cc.numel() // max(half, 1), 1)
    table_rows, rep = plan
    cc = cc.contiguous().view(-1, half)[:table_rows] if table_rows == 1 else cc.contiguous().view(table_rows, half)
    ss = ss.contiguous().view(-1, half)[:table_rows] if table_rows == 1 else ss.contiguous().view(table_rows, half)
    x2 = xx.contiguous().view(-1, d)
    y = torch.empty_like(x2)
    with device_guard(x):
        st = _lib.load().ak_rope(code, x2.data_ptr(), cc.data_ptr(), ss.data_ptr(), y.data_ptr(),
                                 x2.shape[0], d, table_rows, rep, _lib.stream_of(x))
    _lib.check(st, "ak_rope", shape=xs, dtype=dt)
    return y.view(xs)


def apply_fp32_tables(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """A LLaMA block's RoPE (models/llama_7b.py:40-48) on x [B, T, H, D]: fp32 tables [>= T, D/2],
    fp32 arithmetic, one rounding to x's dtype. x may be a column slice of a wider projection
    output (head and dim contiguous, any token stride). Returns a dense [B, T, H, D] tensor.
    Runs ak_rope_f32_tables."""
    _lib.require_gpu("rope_fp32_tables", x, cos, sin)
    B, T, H, D = x.shape
    code = _lib.dtype_code(x, "rope_fp32_tables")
    if not (x.stride(3) == 1 and x.stride(2) == D and x.stride(0) == T * x.stride(1)):
        x = x.contiguous()
    c = cos[:T].float().contiguous()
    s = sin[:T].float().contiguous()
    y = torch.empty((B, T, H, D), device=x.device, dtype=x.dtype)
    with device_guard(x):
        st = _lib.load().ak_rope_f32_tables(code, x.data_ptr(), c.data_ptr(), s.data_ptr(), y.data_ptr(),
                                            B * T * H, D, T, H, x.stride(1), _lib.stream_of(x))
    _lib.check(st, "ak_rope_f32_tables", shape=tuple(x.shape), dtype=x.dtype)
    return y
