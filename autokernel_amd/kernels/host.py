"""The shape / dtype layer of every kernel_fn: the reference's signatures and semantics
(reference.py:10-78, kernels/<op>.py kernel_fn) over a namespace of tensor-level ops, one per
libak355 C entry point (outputs first). Each function checks devices, shapes and dtypes
(ValueError for a bad argument, RuntimeError for a CPU tensor: there is no CPU path), flattens
to the rows layout the op takes, allocates the output and calls the op.

One layer, two backends: ``bind(ops)`` receives the op namespace once. In-tree it is
autokernel_amd.kernels._ops (ctypes over libak355.so); the HuggingFace Kernels package ships this
file unchanged as ``_host.py`` and binds it to its registered torch ops (torch_binding.cpp), which
have the same names and signatures.
"""
from __future__ import annotations

import math

import torch

ops = None  # set by bind()

ACTIVATIONS = {"silu": 0, "gelu": 1, "relu2": 2}
ACT_NONE = 3
IGNORE_INDEX = -100
_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def bind(namespace) -> None:
    global ops
    ops = namespace


def _check(op: str, *ts) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{op}: no CPU path (tensors must be on the GPU)")
    if ts[0].dtype not in _DTYPES:
        raise ValueError(f"{op}: dtype {ts[0].dtype} unsupported (float32, float16, bfloat16)")


def _rows(x: torch.Tensor) -> torch.Tensor:
    """[..., N] -> contiguous [rows, N]."""
    if x.dim() == 2 and x.is_contiguous():
        return x  # the common case, without the cost of two more torch calls
    if x.dim() == 0:
        x = x.reshape(1, 1)
    elif x.dim() == 1:
        x = x.reshape(1, -1)
    x = x.contiguous()
    return x.view(-1, x.shape[-1])


def _as(t, dtype):
    return t if t is None or t.dtype == dtype else t.to(dtype)


def _vec(t):
    """A weight / bias as a contiguous 1-D tensor (itself when it already is one)."""
    if t is None or (t.dim() == 1 and t.is_contiguous()):
        return t
    return t.contiguous().view(-1)


def _shaped(y: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    return y if y.dim() == x.dim() else y.view(x.shape)


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    _check("rmsnorm", x, weight)
    x2 = _rows(x)
    w = _vec(_as(weight, x.dtype))
    if w.numel() != x2.shape[1]:
        raise ValueError(f"rmsnorm: weight has {w.numel()} elements, x rows have {x2.shape[1]}")
    y = torch.empty_like(x2)
    ops.rmsnorm(y, x2, w, float(eps))
    return _shaped(y, x)


def layernorm(x: torch.Tensor, weight: torch.Tensor | None, bias: torch.Tensor | None,
              eps: float = 1e-5) -> torch.Tensor:
    _check("layernorm", x, weight, bias)
    x2 = _rows(x)
    w = _vec(_as(weight, x.dtype))
    b = _vec(_as(bias, x.dtype))
    for name, t in (("weight", w), ("bias", b)):
        if t is not None and t.numel() != x2.shape[1]:
            raise ValueError(f"layernorm: {name} has {t.numel()} elements, x rows have {x2.shape[1]}")
    y = torch.empty_like(x2)
    ops.layernorm(y, x2, w, b, float(eps))
    return _shaped(y, x)


def softmax(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    _check("softmax", x)
    if x.dim() == 0:
        return softmax(x.reshape(1)).reshape(())
    d = dim % x.dim()
    xm = x if d == x.dim() - 1 else x.movedim(d, -1)
    x2 = _rows(xm)
    y = torch.empty_like(x2)
    ops.softmax(y, x2)
    y = y.view(xm.shape)
    return y if d == x.dim() - 1 else y.movedim(-1, d)


def _table_plan(xs: tuple, cs: tuple):
    """(table_rows, rep_inner) when a table of shape cs indexes the rows of x (shape xs) directly."""
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


def rotary_embedding(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    _check("rotary_embedding", x, cos, sin)
    dt = torch.promote_types(torch.promote_types(x.dtype, cos.dtype), sin.dtype)
    xx, cc, ss = (t if t.dtype == dt else t.to(dt) for t in (x, cos, sin))
    d = xx.shape[-1]
    if d % 2:
        raise ValueError(f"rotary_embedding: head_dim {d} is odd")
    half = d // 2
    out_shape = torch.broadcast_shapes(xx.shape[:-1] + (half,), cc.shape, ss.shape)
    if out_shape[:-1] != xx.shape[:-1] or out_shape[-1] != half:
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
    cc = cc.contiguous().view(-1, half)[:table_rows].contiguous()
    ss = ss.contiguous().view(-1, half)[:table_rows].contiguous()
    x2 = xx.contiguous().view(-1, d)
    y = torch.empty_like(x2)
    ops.rope(y, x2, cc, ss, rep)
    return y.view(xs)


def cross_entropy(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    _check("cross_entropy", logits, targets)
    v = logits.shape[-1]
    x2 = logits.contiguous().view(-1, v)
    t = targets.reshape(-1)
    t = (t if t.dtype == torch.int64 else t.to(torch.int64)).contiguous()
    if t.numel() != x2.shape[0]:
        raise ValueError(f"cross_entropy: {x2.shape[0]} rows of logits but {t.numel()} targets")
    loss = torch.empty(max(x2.shape[0], 1), device=logits.device, dtype=torch.float32)
    out = torch.empty((), device=logits.device, dtype=logits.dtype)
    ops.cross_entropy(out, loss, x2, t, IGNORE_INDEX)
    return out


def _reduce(x: torch.Tensor, dim: int, is_max: bool) -> torch.Tensor:
    op = "reduce_max" if is_max else "reduce_sum"
    _check(op, x)
    if x.dim() == 0:
        return x.clone()
    d = dim % x.dim()
    outer, red, inner = math.prod(x.shape[:d]), x.shape[d], math.prod(x.shape[d + 1:])
    if is_max and red == 0:
        raise ValueError("reduce_max: cannot reduce an empty dimension")
    y = torch.empty(x.shape[:d] + x.shape[d + 1:], device=x.device, dtype=x.dtype)
    (ops.reduce_max if is_max else ops.reduce_sum)(y, x.contiguous(), outer, red, inner)
    return y


def reduce(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    return _reduce(x, dim, False)


def reduce_max(x: torch.Tensor, dim: int = -1) -> torch.Tensor:
    return _reduce(x, dim, True)


# f16 / bf16 operands that the LDS-DMA GEMM cannot read as 16-byte chunks (K or a row stride not a
# multiple of 8 elements, a base that is not 16-byte aligned, a [K, N] B with N % 8 != 0) would take
# the register-staged kernel's element loads, 4-5x slower from 255^3 up (f16 1023^3: 151 us against
# 28 us repacked; 4095^3: 882 against 228 us). Above this size they are copied once into zero-padded
# operands whose K is a multiple of 64. The extra products are exact zeros at the end of each sum,
# so the result is the same.
_REPACK_MIN_MNK = 1 << 21


def _ld(t: torch.Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else max(t.shape[1], 1)


def _repack(A: torch.Tensor, Bs: torch.Tensor, bt: bool, N: int, K: int):
    """A [M, Kp] and B as [N, Kp] (bt) or [Kp, N] (a [K, N] B with N % 8 == 0), zero-padded."""
    Kp = -(-K // 64) * 64
    A = torch.nn.functional.pad(A, (0, Kp - K)).contiguous()
    if bt:
        Bs = torch.nn.functional.pad(Bs, (0, Kp - K)).contiguous()
    elif N % 8 == 0:
        Bs = torch.nn.functional.pad(Bs, (0, 0, 0, Kp - K)).contiguous()
    else:
        Bs, bt = torch.nn.functional.pad(Bs.t(), (0, Kp - K)).contiguous(), True
    return A, Bs, bt, Kp


def _gemm(A: torch.Tensor, B: torch.Tensor, out: torch.Tensor | None = None, split_k: bool = False) -> torch.Tensor:
    """C = A @ B for 2-D A [M, K] and B [K, N]; a transposed [N, K] view of B is read in place.
    split_k: grids that leave most CUs idle split K (the matmul op does; fused_mlp does not)."""
    M, K = A.shape
    K2, N = B.shape
    if K != K2:
        raise ValueError(f"matmul: shapes {tuple(A.shape)} and {tuple(B.shape)} do not align")
    if A.dtype != B.dtype:
        raise ValueError(f"matmul: dtype mismatch {A.dtype} vs {B.dtype}")
    if not (A.stride(1) == 1 and A.stride(0) >= max(K, 1)):
        A = A.contiguous()
    if B.stride(1) == 1 and B.stride(0) >= max(N, 1):
        Bs, bt = B, False
    elif B.stride(0) == 1 and B.stride(1) >= max(K, 1):
        Bs, bt = B.t(), True  # the stored [N, K] matrix
    else:
        Bs, bt = B.contiguous(), False
    C = out if out is not None else torch.empty((M, N), device=A.device, dtype=A.dtype)
    if K == 0:
        return C.zero_()
    if A.dtype != torch.float32 and M * N * K >= _REPACK_MIN_MNK and not (
            K % 8 == 0 and _ld(A) % 8 == 0 and _ld(Bs) % 8 == 0 and A.data_ptr() % 16 == 0
            and Bs.data_ptr() % 16 == 0 and (bt or N % 8 == 0)):
        A, Bs, bt, K = _repack(A, Bs, bt, N, K)
    ws = None
    if split_k:
        code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[A.dtype]
        nbytes = ops.gemm_workspace_bytes(code, M, N, K, _ld(A), _ld(Bs), _ld(C), bt)
        if nbytes > 0:
            ws = torch.empty(nbytes // 4, device=A.device, dtype=torch.float32)
    ops.gemm(C, A, Bs, bt, ws)
    return C


def matmul(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    _check("matmul", A, B)
    if A.dim() == 1 and B.dim() == 1:
        return _gemm(A.view(1, -1), B.view(-1, 1), split_k=True).view(())
    if A.dim() == 1:
        return matmul(A.view(1, -1), B).squeeze(-2)
    if B.dim() == 1:
        return matmul(A, B.view(-1, 1)).squeeze(-1)
    if B.dim() == 2:
        lead = A.shape[:-1]
        A2 = A.reshape(-1, A.shape[-1]) if A.dim() > 2 else A
        return _gemm(A2, B, split_k=True).view(*lead, B.shape[-1])
    # batched: broadcast batch dims (a stride of 0 shares an operand), one batched launch
    batch = torch.broadcast_shapes(A.shape[:-2], B.shape[:-2])
    M, K = A.shape[-2:]
    K2, N = B.shape[-2:]
    if K != K2:
        raise ValueError(f"matmul: shapes {tuple(A.shape)} and {tuple(B.shape)} do not align")
    if A.dtype != B.dtype:
        raise ValueError(f"matmul: dtype mismatch {A.dtype} vs {B.dtype}")
    nb = math.prod(batch)
    C = torch.empty((nb, M, N), device=A.device, dtype=A.dtype)
    if nb == 0 or M == 0 or N == 0:
        return C.view(*batch, M, N)
    if K == 0:
        return C.zero_().view(*batch, M, N)
    Ab = A.expand(*batch, M, K).reshape(nb, M, K)
    Bb = B.expand(*batch, K, N).reshape(nb, K, N)
    if not (Ab.stride(2) == 1 and Ab.stride(1) >= max(K, 1)):
        Ab = Ab.contiguous()
    if Bb.stride(2) == 1 and Bb.stride(1) >= max(N, 1):
        Bs, bt = Bb, False
    elif Bb.stride(1) == 1 and Bb.stride(2) >= max(K, 1):
        Bs, bt = Bb.transpose(1, 2), True  # the stored [N, K] matrices
    else:
        Bs, bt = Bb.contiguous(), False
    ops.gemm_batched(C, Ab, Bs, bt)
    return C.view(*batch, M, N)


def fused_mlp(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor,
              activation: str = "silu") -> torch.Tensor:
    _check("fused_mlp", x, w_gate, w_up, w_down)
    for name, w in (("w_gate", w_gate), ("w_up", w_up), ("w_down", w_down)):
        if w.dtype != x.dtype:
            raise ValueError(f"fused_mlp: {name} dtype {w.dtype} != x dtype {x.dtype}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    M, D = x2.shape
    H = w_gate.shape[0]
    if w_gate.shape != (H, D) or w_up.shape != (H, D) or w_down.shape[1] != H:
        raise ValueError(f"fused_mlp: weight shapes {tuple(w_gate.shape)}, {tuple(w_up.shape)}, "
                         f"{tuple(w_down.shape)} do not fit x [*, {D}]")
    h = torch.empty((M, H), device=x.device, dtype=x.dtype)
    ops.mlp_gate_up(h, x2, w_gate.contiguous(), w_up.contiguous(), ACTIVATIONS.get(activation, ACT_NONE))
    return _gemm(h, w_down.t()).view(*lead, w_down.shape[0])


def _attn_operand(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or any(s % 8 for s in t.stride()[:-1]) or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def flash_attention(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, causal: bool = True,
                    sm_scale: float | None = None) -> torch.Tensor:
    _check("flash_attention", Q, K, V)
    if Q.dim() == 3:
        return flash_attention(Q[None], K[None], V[None], causal, sm_scale)[0]
    if Q.dim() != 4:
        raise ValueError(f"flash_attention: expected 3-D or 4-D Q, got {Q.dim()}-D")
    if K.shape[0] != Q.shape[0] and K.shape[0] == 1:
        K = K.expand(Q.shape[0], *K.shape[1:])
        V = V.expand(Q.shape[0], *V.shape[1:])
    B, Hq, Sq, D = Q.shape
    Bk, Hkv, Sk, Dk = K.shape
    if V.shape != K.shape or Dk != D or Bk != B:
        raise ValueError(f"flash_attention: shapes Q{tuple(Q.shape)} K{tuple(K.shape)} V{tuple(V.shape)}")
    if Hkv == 0 or Hq % Hkv:
        raise ValueError(f"flash_attention: {Hq} query heads not a multiple of {Hkv} KV heads")
    if not (Q.dtype == K.dtype == V.dtype) or Q.dtype not in _DTYPES:
        raise ValueError("flash_attention: Q, K, V must share a float32, float16 or bfloat16 dtype")
    if not 1 <= D <= 256:
        raise ValueError(f"flash_attention: head_dim {D} unsupported (1 .. 256)")
    if Sk == 0:
        raise ValueError("flash_attention: empty key sequence")
    scale = float(D ** -0.5 if sm_scale is None else sm_scale)
    if Q.dtype != torch.float32 and D < 128 and D != 64:
        # narrow f16 / bf16 heads: zero-padded to 64 / 128 onto the MFMA kernels, padding dropped
        Dp = 64 if D < 64 else 128
        padded = [torch.nn.functional.pad(t, (0, Dp - D)) for t in (Q, K, V)]
        return flash_attention(*padded, causal, scale)[..., :D].contiguous()
    if Q.is_contiguous():
        O = torch.empty((B, Hq, Sq, D), device=Q.device, dtype=Q.dtype)
    else:
        # Q is a view of a model's [B, S, H, D] projection: O is written in that order too, so the
        # caller's transpose back to [B, S, H * D] is a view rather than a copy (stock SDPA's layout)
        O = torch.empty((B, Sq, Hq, D), device=Q.device, dtype=Q.dtype).transpose(1, 2)
    ops.flash_attn_fwd(O, _attn_operand(Q), _attn_operand(K), _attn_operand(V), bool(causal), scale)
    return O


# kernel_fn of each reference op type (KERNEL_CONFIGS key)
KERNEL_FNS = {
    "rmsnorm": rmsnorm,
    "layernorm": layernorm,
    "softmax": softmax,
    "rotary_embedding": rotary_embedding,
    "cross_entropy": cross_entropy,
    "reduce": reduce,
    "matmul": matmul,
    "fused_mlp": fused_mlp,
    "flash_attention": flash_attention,
}
