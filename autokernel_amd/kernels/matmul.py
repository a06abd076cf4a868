"""Matmul drop-in: kernel_fn(A, B) = torch.matmul(A, B).

Mirrors reference.py:10-12 and kernels/matmul.py:62. A: [..., M, K] (leading dims flattened into
M when B is 2-D), B: [K, N]; batched B loops over the batch. When B is a transposed view of a
row-major [N, K] tensor (nn.Linear's weight.t()), the GEMM reads it in place (b_trans = 1)
instead of copying; a row-major [K, N] B is read in place too (b_trans = 0). Runs ak_gemm
(gemm.hip), or, for kernel_fn, ak_gemm_ws with a torch-allocated fp32 workspace when few output tiles
and a long K would leave most CUs idle (K split into slices that run side by side, then added in a
fixed order). kernel_fn is kernels/host.py's matmul; gemm, gemm_bias, gemm_bias_gelu, gemm_bias_residual,
gemm_residual and gemm_rope are the 2-D forms (and fused epilogues) the model plug-in uses.
"""
from __future__ import annotations

import torch

from . import _ops, host
from .host import matmul as kernel_fn  # noqa: F401

KERNEL_TYPE = "matmul"


def _b_layout(B: torch.Tensor) -> tuple[torch.Tensor, bool]:
    """(stored matrix, b_trans) for a 2-D B [K, N] without copying when possible."""
    K, N = B.shape
    if B.stride(1) == 1 and B.stride(0) >= max(N, 1):
        return B, False
    if B.stride(0) == 1 and B.stride(1) >= max(K, 1):
        return B.t(), True  # the stored [N, K] matrix
    return B.contiguous(), False


def _a_rows(A: torch.Tensor) -> torch.Tensor:
    K = A.shape[1]
    return A if (A.stride(1) == 1 and A.stride(0) >= max(K, 1)) else A.contiguous()


def gemm(A: torch.Tensor, B: torch.Tensor, out: torch.Tensor | None = None, split_k: bool = False) -> torch.Tensor:
    """C = A @ B for 2-D A [M, K] and 2-D B [K, N] (B may be a transposed [N, K] view).

    split_k: let grids that leave most CUs idle split K (ak_gemm_ws); kernel_fn sets it. The model
    plug-in's projections keep the unsplit kernel, whose fp32 summation order reproduces stock
    PyTorch's f16 logits bit for bit."""
    return host._gemm(A, B, out=out, split_k=split_k)


def _epilogue_operands(op: str, A: torch.Tensor, B: torch.Tensor):
    M, K = A.shape
    K2, N = B.shape
    if K != K2:
        raise ValueError(f"{op}: shapes {tuple(A.shape)} and {tuple(B.shape)} do not align")
    if A.dtype != B.dtype or A.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"{op}: needs one f16 / bf16 dtype, got {A.dtype}, {B.dtype}")
    host._check(op, A, B)
    Bs, bt = _b_layout(B)
    return _a_rows(A), Bs, bt, M, N


def _bias_operand(op: str, bias: torch.Tensor, A: torch.Tensor, N: int) -> torch.Tensor:
    if tuple(bias.shape) != (N,) or bias.dtype != A.dtype:
        raise ValueError(f"{op}: bias {tuple(bias.shape)} {bias.dtype} does not fit [{N}] {A.dtype}")
    return bias.contiguous()


def gemm_bias(A: torch.Tensor, B: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """A @ B + bias for 2-D A [M, K], B [K, N] (a transposed [N, K] view is read in place) and
    bias [N], f16 / bf16, in one ak_gemm_bias launch: the bias joins the fp32 accumulator and the
    sum is rounded once, as torch's addmm (a biased nn.Linear) rounds it."""
    A, Bs, bt, M, N = _epilogue_operands("gemm_bias", A, B)
    bias = _bias_operand("gemm_bias", bias, A, N)
    C = torch.empty((M, N), device=A.device, dtype=A.dtype)
    _ops.gemm_bias(C, A, Bs, bias, bt)
    return C


def gemm_bias_gelu(A: torch.Tensor, B: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """gelu(A @ B + bias) (exact erf GELU) for 2-D A [M, K], B [K, N] (a transposed [N, K] view is
    read in place) and bias [N], f16 / bf16, in one ak_gemm_bias_gelu launch: the biased product is
    rounded as gemm_bias rounds it, then GELU in fp32 is rounded again, as a biased nn.Linear
    followed by nn.GELU computes it (models/gpt2.py:60-62, models/bert_base.py:47-48)."""
    A, Bs, bt, M, N = _epilogue_operands("gemm_bias_gelu", A, B)
    bias = _bias_operand("gemm_bias_gelu", bias, A, N)
    C = torch.empty((M, N), device=A.device, dtype=A.dtype)
    _ops.gemm_bias_gelu(C, A, Bs, bias, bt)
    return C


def gemm_bias_residual(A: torch.Tensor, B: torch.Tensor, bias: torch.Tensor, R: torch.Tensor) -> torch.Tensor:
    """R + (A @ B + bias) for 2-D A [M, K], B [K, N] (a transposed [N, K] view is read in place),
    bias [N] and R [M, N], f16 / bf16, in one ak_gemm_bias_residual launch: the biased product is
    rounded, then the add, so the result equals torch's `R + linear(x)` for a biased Linear bit for
    bit (models/gpt2.py:63-65, models/bert_base.py:60-62)."""
    A, Bs, bt, M, N = _epilogue_operands("gemm_bias_residual", A, B)
    bias = _bias_operand("gemm_bias_residual", bias, A, N)
    if tuple(R.shape) != (M, N) or R.dtype != A.dtype:
        raise ValueError(f"gemm_bias_residual: R {tuple(R.shape)} {R.dtype} does not fit [{M}, {N}] {A.dtype}")
    C = torch.empty((M, N), device=A.device, dtype=A.dtype)
    _ops.gemm_bias_residual(C, A, Bs, bias, R.contiguous(), bt)
    return C


def gemm_residual(A: torch.Tensor, B: torch.Tensor, R: torch.Tensor) -> torch.Tensor:
    """R + A @ B for 2-D A [M, K], B [K, N] (a transposed [N, K] view is read in place) and
    R [M, N], f16 / bf16, in one ak_gemm_residual launch: the product is rounded, then the add,
    so the result equals torch's `R + A @ B` bit for bit (models/llama_7b.py:110-111)."""
    A, Bs, bt, M, N = _epilogue_operands("gemm_residual", A, B)
    if tuple(R.shape) != (M, N) or R.dtype != A.dtype:
        raise ValueError(f"gemm_residual: R {tuple(R.shape)} {R.dtype} does not fit [{M}, {N}] {A.dtype}")
    C = torch.empty((M, N), device=A.device, dtype=A.dtype)
    _ops.gemm_residual(C, A, Bs, R.contiguous(), bt)
    return C


def gemm_rope(A: torch.Tensor, B: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, seq_len: int,
              head_dim: int, rot_cols: int) -> torch.Tensor:
    """A @ B (2-D, f16 / bf16) with the model's rotary embedding applied in the GEMM epilogue to
    columns [0, rot_cols): each head of head_dim columns rotated pairwise in fp32 by the fp32
    tables cos / sin [>= seq_len, head_dim / 2], row m being token m % seq_len, then rounded once.
    One ak_gemm_rope launch; equals the projection followed by the fp32 rotation
    (models/llama_7b.py:40-48, :67-71) bit for bit."""
    A, Bs, bt, M, N = _epilogue_operands("gemm_rope", A, B)
    half = head_dim // 2
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape[0] < seq_len or \
            cos.shape[-1] != half or sin.shape != cos.shape:
        raise ValueError(f"gemm_rope: tables must be fp32 [>= {seq_len}, {half}], got {tuple(cos.shape)} {cos.dtype}")
    C = torch.empty((M, N), device=A.device, dtype=A.dtype)
    _ops.gemm_rope(C, A, Bs, bt, cos.contiguous(), sin.contiguous(), seq_len, head_dim, rot_cols)
    return C
