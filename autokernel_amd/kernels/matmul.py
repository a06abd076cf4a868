"""Matmul drop-in: kernel_fn(A, B) = torch.matmul(A, B).

Mirrors reference.py:10-12 and kernels/matmul.py:62. A: [..., M, K] (leading dims flattened into
M when B is 2-D), B: [K, N]; batched B loops over the batch. When B is a transposed view of a
row-major [N, K] tensor (nn.Linear's weight.t()), the GEMM reads it in place (b_trans = 1)
instead of copying; a row-major [K, N] B is read in place too (b_trans = 0). Runs ak_gemm
(gemm.hip), or, for kernel_fn, ak_gemm_ws with a torch-allocated fp32 workspace when few output tiles
and a long K would leave most CUs idle (K split into slices that run side by side, then added in a
fixed order).
"""
from __future__ import annotations

import functools

import torch

from .. import _lib
from ._common import device_guard


@functools.lru_cache(maxsize=1024)
def _workspace_bytes(code: int, M: int, N: int, K: int, lda: int, ldb: int, ldc: int, bt: int) -> int:
    """ak_gemm_workspace_bytes, remembered per argument tuple: the split decision depends on the
    arguments alone, and a repeated shape then costs no library call."""
    return _lib.load().ak_gemm_workspace_bytes(code, M, N, K, lda, ldb, ldc, bt)


KERNEL_TYPE = "matmul"


def _b_layout(B: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    """(tensor, ldb, b_trans) for a 2-D B [K, N] without copying when possible."""
    K, N = B.shape
    if B.stride(1) == 1 and B.stride(0) >= max(N, 1):
        return B, B.stride(0), 0
    if B.stride(0) == 1 and B.stride(1) >= max(K, 1):
        return B, B.stride(1), 1
    Bc = B.contiguous()
    return Bc, max(N, 1), 0


def gemm(A: torch.Tensor, B: torch.Tensor, out: torch.Tensor | None = None, split_k: bool = False) -> torch.Tensor:
    """C = A @ B for 2-D A [M, K] and 2-D B [K, N] (B may be a transposed [N, K] view).

    split_k: let grids that leave most CUs idle split K (ak_gemm_ws); kernel_fn sets it. The model
    plug-in's projections keep the unsplit kernel, whose fp32 summation order reproduces stock
    PyTorch's f16 logits bit for bit."""
    M, K = A.shape
    K2, N = B.shape
    if K != K2:
        raise ValueError(f"matmul: shapes {tuple(A.shape)} and {tuple(B.shape)} do not align")
    if A.dtype != B.dtype:
        raise ValueError(f"matmul: dtype mismatch {A.dtype} vs {B.dtype}")
    code = _lib.dtype_code(A, "matmul")
    if not (A.stride(1) == 1 and A.stride(0) >= max(K, 1)):
        A = A.contiguous()
    lda = A.stride(0) if M > 1 else max(K, 1)
    Bt, ldb, bt = _b_layout(B)
    C = out if out is not None else torch.empty((M, N), device=A.device, dtype=A.dtype)
    if K == 0:
        return C.zero_()
    lib = _lib.load()
    ldc = C.stride(0) if M > 1 else max(N, 1)
    with device_guard(A):
        # grids that leave most CUs idle split K over a torch-allocated fp32 workspace (ak_gemm_ws)
        ws_bytes = _workspace_bytes(code, M, N, K, lda, ldb, ldc, bt) if split_k else 0
        if ws_bytes > 0:
            ws = torch.empty(ws_bytes // 4, device=A.device, dtype=torch.float32)
            st = lib.ak_gemm_ws(code, A.data_ptr(), Bt.data_ptr(), C.data_ptr(), M, N, K, lda, ldb, ldc, bt,
                                ws.data_ptr(), ws_bytes, _lib.stream_of(A))
        else:
            st = lib.ak_gemm(code, A.data_ptr(), Bt.data_ptr(), C.data_ptr(), M, N, K, lda, ldb, ldc, bt,
                             _lib.stream_of(A))
    _lib.check(st, "ak_gemm", M=M, N=N, K=K, b_trans=bt, dtype=A.dtype)
    return C


def gemm_residual(A: torch.Tensor, B: torch.Tensor, R: torch.Tensor) -> torch.Tensor:
    """R + A @ B for 2-D A [M, K], B [K, N] (a transposed [N, K] view is read in place) and
    R [M, N], f16 / bf16, in one ak_gemm_residual launch: the product is rounded, then the add,
    so the result equals torch's `R + A @ B` bit for bit (models/llama_7b.py:110-111)."""
    M, K = A.shape
    K2, N = B.shape
    if K != K2 or tuple(R.shape) != (M, N):
        raise ValueError(f"gemm_residual: shapes {tuple(A.shape)} @ {tuple(B.shape)} + {tuple(R.shape)} do not align")
    if not (A.dtype == B.dtype == R.dtype) or A.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"gemm_residual: needs one f16 / bf16 dtype, got {A.dtype}, {B.dtype}, {R.dtype}")
    code = _lib.dtype_code(A, "gemm_residual")
    if not (A.stride(1) == 1 and A.stride(0) >= max(K, 1)):
        A = A.contiguous()
    lda = A.stride(0) if M > 1 else max(K, 1)
    Bt, ldb, bt = _b_layout(B)
    R = R.contiguous()
    C = torch.empty((M, N), device=A.device, dtype=A.dtype)
    with device_guard(A):
        st = _lib.load().ak_gemm_residual(code, A.data_ptr(), Bt.data_ptr(), R.data_ptr(), C.data_ptr(), M, N,
                                          K, lda, ldb, max(N, 1), bt, _lib.stream_of(A))
    _lib.check(st, "ak_gemm_residual", M=M, N=N, K=K, b_trans=bt, dtype=A.dtype)
    return C


def gemm_bias(A: torch.Tensor, B: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """A @ B + bias for 2-D A [M, K], B [K, N] (a transposed [N, K] view is read in place) and
    bias [N], f16 / bf16, in one ak_gemm_bias launch: the bias joins the fp32 accumulator and the
    sum is rounded once, as torch's addmm (a biased nn.Linear) rounds it."""
    M, K = A.shape
    K2, N = B.shape
    if K != K2 or tuple(bias.shape) != (N,):
        raise ValueError(f"gemm_bias: shapes {tuple(A.shape)} @ {tuple(B.shape)} + {tuple(bias.shape)} do not align")
    if not (A.dtype == B.dtype == bias.dtype) or A.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"gemm_bias: needs one f16 / bf16 dtype, got {A.dtype}, {B.dtype}, {bias.dtype}")
    code = _lib.dtype_code(A, "gemm_bias")
    if not (A.stride(1) == 1 and A.stride(0) >= max(K, 1)):
        A = A.contiguous()
    lda = A.stride(0) if M > 1 else max(K, 1)
    Bt, ldb, bt = _b_layout(B)
    b = bias.contiguous()
    C = torch.empty((M, N), device=A.device, dtype=A.dtype)
    with device_guard(A):
        st = _lib.load().ak_gemm_bias(code, A.data_ptr(), Bt.data_ptr(), b.data_ptr(), C.data_ptr(), M, N, K,
                                      lda, ldb, max(N, 1), bt, _lib.stream_of(A))
    _lib.check(st, "ak_gemm_bias", M=M, N=N, K=K, b_trans=bt, dtype=A.dtype)
    return C


def gemm_rope(A: torch.Tensor, B: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, seq_len: int,
              head_dim: int, rot_cols: int) -> torch.Tensor:
    """A @ B (2-D, f16 / bf16) with the model's rotary embedding applied in the GEMM epilogue to
    columns [0, rot_cols): each head of head_dim columns rotated pairwise in fp32 by the fp32
    tables cos / sin [>= seq_len, head_dim / 2], row m being token m % seq_len, then rounded once.
    One ak_gemm_rope launch; equals the projection followed by the fp32 rotation
    (models/llama_7b.py:40-48, :67-71) bit for bit."""
    M, K = A.shape
    K2, N = B.shape
    if K != K2:
        raise ValueError(f"gemm_rope: shapes {tuple(A.shape)} and {tuple(B.shape)} do not align")
    if A.dtype != B.dtype or A.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"gemm_rope: needs one f16 / bf16 dtype, got {A.dtype}, {B.dtype}")
    half = head_dim // 2
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape[0] < seq_len or \
            cos.shape[-1] != half or sin.shape != cos.shape:
        raise ValueError(f"gemm_rope: tables must be fp32 [>= {seq_len}, {half}], got {tuple(cos.shape)} {cos.dtype}")
    code = _lib.dtype_code(A, "gemm_rope")
    if not (A.stride(1) == 1 and A.stride(0) >= max(K, 1)):
        A = A.contiguous()
    lda = A.stride(0) if M > 1 else max(K, 1)
    Bt, ldb, bt = _b_layout(B)
    c, s = cos.contiguous(), sin.contiguous()
    C = torch.empty((M, N), device=A.device, dtype=A.dtype)
    with device_guard(A):
        st = _lib.load().ak_gemm_rope(code, A.data_ptr(), Bt.data_ptr(), C.data_ptr(), M, N, K, lda, ldb,
                                      max(N, 1), bt, c.data_ptr(), s.data_ptr(), seq_len, head_dim, rot_cols,
                                      _lib.stream_of(A))
    _lib.check(st, "ak_gemm_rope", M=M, N=N, K=K, head_dim=head_dim, rot_cols=rot_cols, dtype=A.dtype)
    return C


def kernel_fn(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    _lib.require_gpu("matmul", A, B)
    if A.dim() == 1 and B.dim() == 1:
        return gemm(A.view(1, -1), B.view(-1, 1), split_k=True).view(())
    if A.dim() == 1:
        return kernel_fn(A.view(1, -1), B).squeeze(-2)
    if B.dim() == 1:
        return kernel_fn(A, B.view(-1, 1)).squeeze(-1)
    if B.dim() == 2:
        lead = A.shape[:-1]
        A2 = A.reshape(-1, A.shape[-1]) if A.dim() > 2 else A
        return gemm(A2, B, split_k=True).view(*lead, B.shape[-1])
    # batched B: broadcast batch dims, one GEMM per batch entry
    batch = torch.broadcast_shapes(A.shape[:-2], B.shape[:-2])
    Ab = A.expand(*batch, *A.shape[-2:]).reshape(-1, *A.shape[-2:])
    Bb = B.expand(*batch, *B.shape[-2:]).reshape(-1, *B.shape[-2:])
    C = torch.empty((Ab.shape[0], A.shape[-2], B.shape[-1]), device=A.device, dtype=A.dtype)
    for i in range(Ab.shape[0]):
        gemm(Ab[i], Bb[i], out=C[i], split_k=True)
    return C.view(*batch, A.shape[-2], B.shape[-1])
