"""The tensor-level ops behind kernels/host.py, over libak355's C ABI through ctypes.

Each function has the name and signature of the torch op that the HuggingFace Kernels package
registers for the same C entry point (hf_export/torch_binding.cpp): outputs first, then inputs,
then scalars. So kernels/host.py, the one shape / dtype layer of every kernel_fn, runs unchanged
on either: bound to this module in-tree, bound to the package's torch ops in the export. Each op
makes the input's device current (when it is not already), launches on torch's current stream of
that device and raises AkError on a non-OK status.
"""
from __future__ import annotations

import functools

import torch

from .. import _lib


def _code(t: torch.Tensor, op: str) -> int:
    return _lib.dtype_code(t, op)


def _run(fn_name: str, ref: torch.Tensor, *args, **info) -> None:
    idx = ref.get_device()
    if idx < 0:
        raise RuntimeError(f"{fn_name}: expected GPU tensors, got one on {ref.device} (no CPU path)")
    fn = getattr(_lib.load(), fn_name)
    if idx == torch.cuda.current_device():
        st = fn(*args, _lib.stream_of(ref))
    else:
        with torch.cuda.device(idx):
            st = fn(*args, _lib.stream_of(ref))
    if st != _lib.AK_OK:
        _lib.check(st, fn_name, **info)


def rmsnorm(y: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, eps: float) -> None:
    _run("ak_rmsnorm", x, _code(x, "rmsnorm"), x.data_ptr(), weight.data_ptr(), y.data_ptr(), x.shape[0],
         x.shape[1], float(eps), shape=tuple(x.shape), dtype=x.dtype)


def rmsnorm_rsqrt(y: torch.Tensor, x: torch.Tensor, weight: torch.Tensor, eps: float) -> None:
    _run("ak_rmsnorm_rsqrt", x, _code(x, "rmsnorm"), x.data_ptr(), weight.data_ptr(), y.data_ptr(),
         x.shape[0], x.shape[1], float(eps), shape=tuple(x.shape), dtype=x.dtype)


def layernorm(y: torch.Tensor, x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
              eps: float) -> None:
    _run("ak_layernorm", x, _code(x, "layernorm"), x.data_ptr(), _lib.ptr(weight), _lib.ptr(bias), y.data_ptr(),
         x.shape[0], x.shape[1], float(eps), shape=tuple(x.shape), dtype=x.dtype)


def softmax(y: torch.Tensor, x: torch.Tensor) -> None:
    _run("ak_softmax", x, _code(x, "softmax"), x.data_ptr(), y.data_ptr(), x.shape[0], x.shape[1],
         shape=tuple(x.shape), dtype=x.dtype)


def rope(y: torch.Tensor, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rep_inner: int) -> None:
    _run("ak_rope", x, _code(x, "rotary_embedding"), x.data_ptr(), cos.data_ptr(), sin.data_ptr(), y.data_ptr(),
         x.shape[0], x.shape[1], cos.shape[0], int(rep_inner), shape=tuple(x.shape), dtype=x.dtype)


def cross_entropy(out: torch.Tensor, row_loss: torch.Tensor, logits: torch.Tensor, targets: torch.Tensor,
                  ignore_index: int) -> None:
    _run("ak_cross_entropy", logits, _code(logits, "cross_entropy"), logits.data_ptr(), targets.data_ptr(),
         row_loss.data_ptr(), out.data_ptr(), logits.shape[0], logits.shape[1], int(ignore_index),
         shape=tuple(logits.shape), dtype=logits.dtype)


def reduce_sum(y: torch.Tensor, x: torch.Tensor, outer: int, reduce: int, inner: int) -> None:
    _run("ak_reduce_sum", x, _code(x, "reduce_sum"), x.data_ptr(), y.data_ptr(), outer, reduce, inner,
         shape=tuple(x.shape), dtype=x.dtype)


def reduce_max(y: torch.Tensor, x: torch.Tensor, outer: int, reduce: int, inner: int) -> None:
    _run("ak_reduce_max", x, _code(x, "reduce_max"), x.data_ptr(), y.data_ptr(), outer, reduce, inner,
         shape=tuple(x.shape), dtype=x.dtype)


def _ld(t: torch.Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)


def gemm(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor, b_trans: bool,
         workspace: torch.Tensor | None = None) -> None:
    """c [M, N] = a [M, K] @ op(b): b stored [K, N] (b_trans False) or [N, K] (True); every operand
    with a unit stride along its last dim, row strides passed through."""
    M, K = a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    code = _code(a, "matmul")
    if workspace is not None and workspace.numel() > 0:
        _run("ak_gemm_ws", a, code, a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, _ld(a), _ld(b), _ld(c),
             int(bool(b_trans)), workspace.data_ptr(), workspace.numel() * 4, M=M, N=N, K=K, b_trans=b_trans,
             dtype=a.dtype)
        return
    _run("ak_gemm", a, code, a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, _ld(a), _ld(b), _ld(c),
         int(bool(b_trans)), M=M, N=N, K=K, b_trans=b_trans, dtype=a.dtype)


def gemm_batched(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor, b_trans: bool) -> None:
    """c [Z, M, N] = a [Z, M, K] @ op(b) for each batch item z: b stored [Z, K, N] (b_trans False) or
    [Z, N, K] (True); unit stride along each last dim, any row and batch strides (0 broadcasts)."""
    Z, M, K = a.shape
    N = b.shape[1] if b_trans else b.shape[2]

    def ld(t):
        return t.stride(1) if t.shape[1] > 1 else max(t.shape[2], 1)
    _run("ak_gemm_batched", a, _code(a, "matmul"), a.data_ptr(), b.data_ptr(), c.data_ptr(), Z, M, N, K, ld(a),
         ld(b), ld(c), a.stride(0), b.stride(0), c.stride(0), int(bool(b_trans)), Z=Z, M=M, N=N, K=K,
         b_trans=b_trans, dtype=a.dtype)


def gemm_bias(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor, b_trans: bool) -> None:
    """c = a @ op(b) + bias [N], the bias added to the fp32 accumulator (one rounding)."""
    M, K = a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    _run("ak_gemm_bias", a, _code(a, "gemm_bias"), a.data_ptr(), b.data_ptr(), bias.data_ptr(), c.data_ptr(), M, N, K,
         _ld(a), _ld(b), _ld(c), int(bool(b_trans)), M=M, N=N, K=K, b_trans=b_trans, dtype=a.dtype)


def gemm_bias_gelu(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor, b_trans: bool) -> None:
    """c = gelu(a @ op(b) + bias): the biased product rounded, then exact GELU, rounded again."""
    M, K = a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    _run("ak_gemm_bias_gelu", a, _code(a, "gemm_bias_gelu"), a.data_ptr(), b.data_ptr(), bias.data_ptr(),
         c.data_ptr(), M, N, K, _ld(a), _ld(b), _ld(c), int(bool(b_trans)), M=M, N=N, K=K, b_trans=b_trans,
         dtype=a.dtype)


def gemm_bias_residual(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor, r: torch.Tensor,
                       b_trans: bool) -> None:
    """c = r + (a @ op(b) + bias): the biased product rounded, then the sum (r shares c's row stride)."""
    M, K = a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    _run("ak_gemm_bias_residual", a, _code(a, "gemm_bias_residual"), a.data_ptr(), b.data_ptr(), bias.data_ptr(),
         r.data_ptr(), c.data_ptr(), M, N, K, _ld(a), _ld(b), _ld(c), int(bool(b_trans)), M=M, N=N, K=K,
         b_trans=b_trans, dtype=a.dtype)


def gemm_residual(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor, r: torch.Tensor, b_trans: bool) -> None:
    """c = r + a @ op(b), the product rounded, then the sum (r shares c's row stride)."""
    M, K = a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    _run("ak_gemm_residual", a, _code(a, "gemm_residual"), a.data_ptr(), b.data_ptr(), r.data_ptr(), c.data_ptr(),
         M, N, K, _ld(a), _ld(b), _ld(c), int(bool(b_trans)), M=M, N=N, K=K, b_trans=b_trans, dtype=a.dtype)


def gemm_rope(c: torch.Tensor, a: torch.Tensor, b: torch.Tensor, b_trans: bool, cos: torch.Tensor, sin: torch.Tensor,
              seq_len: int, head_dim: int, rot_cols: int) -> None:
    """c = a @ op(b) with the model's rotary embedding on columns [0, rot_cols) (fp32 tables)."""
    M, K = a.shape
    N = b.shape[0] if b_trans else b.shape[1]
    _run("ak_gemm_rope", a, _code(a, "gemm_rope"), a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, _ld(a), _ld(b),
         _ld(c), int(bool(b_trans)), cos.data_ptr(), sin.data_ptr(), seq_len, head_dim, rot_cols, M=M, N=N, K=K,
         head_dim=head_dim, rot_cols=rot_cols, dtype=a.dtype)


def rope_f32_tables(y: torch.Tensor, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rows: int, head_dim: int,
                    table_rows: int, rep_inner: int, x_tok_stride: int) -> None:
    """The model's RoPE: x (rows / rep_inner tokens of rep_inner heads, token stride x_tok_stride)
    rotated by fp32 tables into dense y."""
    _run("ak_rope_f32_tables", x, _code(x, "rope_f32_tables"), x.data_ptr(), cos.data_ptr(), sin.data_ptr(),
         y.data_ptr(), rows, head_dim, table_rows, rep_inner, x_tok_stride, shape=tuple(x.shape), dtype=x.dtype)


@functools.lru_cache(maxsize=1024)
def gemm_workspace_bytes(dtype: int, M: int, N: int, K: int, lda: int, ldb: int, ldc: int, b_trans: bool) -> int:
    """Remembered per argument tuple: the split decision depends on the arguments alone."""
    return _lib.load().ak_gemm_workspace_bytes(dtype, M, N, K, lda, ldb, ldc, int(bool(b_trans)))


def mlp_gate_up(h: torch.Tensor, x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, activation: int) -> None:
    M, D = x.shape
    H = w_gate.shape[0]
    _run("ak_mlp_gate_up", x, _code(x, "fused_mlp"), x.data_ptr(), w_gate.data_ptr(), w_up.data_ptr(), h.data_ptr(),
         M, H, D, int(activation), M=M, H=H, D=D, dtype=x.dtype)


def flash_attn_fwd(o: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool,
                   sm_scale: float) -> None:
    """Q, O [B, Hq, Sq, D], K, V [B, Hkv, Sk, D], any strides with a contiguous head_dim."""
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    st = [_lib.i64_array(t.stride()[:3]) for t in (q, k, v, o)]
    _run("ak_flash_attn_fwd", q, _code(q, "flash_attention"), q.data_ptr(), k.data_ptr(), v.data_ptr(),
         o.data_ptr(), B, Hq, Hkv, Sq, Sk, D, st[0], st[1], st[2], st[3], int(bool(causal)), float(sm_scale),
         Q=tuple(q.shape), K=tuple(k.shape), dtype=q.dtype)
